"""The avi-v1 artefact reader (fp8lin.artifact) on the CPU: the loader's
checks of src/engine.cpp:44-68 as errors, and the load-time steps of
src/engine.cpp:95-143 (MTP filter, vocab-sharded head slice, projection
fusion including the mixed FP8/BF16 GDN group) on a small artefact laid out
as tools/import_fp8.py:60-83 writes it."""
import json
import os

import numpy as np
import pytest
import torch

HIDDEN, INTER, VOCAB = 256, 384, 512
# name -> (rows, cols, kind); kind "fp8" has a block scale, "bf16"/"f32" not
LAYER0 = {  # linear_attention (GDN) layer
    "linear_attn.in_proj_qkv": (384, HIDDEN, "fp8"), "linear_attn.in_proj_z": (128, HIDDEN, "fp8"),
    "linear_attn.in_proj_b": (4, HIDDEN, "bf16"), "linear_attn.in_proj_a": (4, HIDDEN, "bf16"),
    "linear_attn.out_proj": (HIDDEN, 128, "fp8"),
}
LAYER1 = {  # full_attention layer
    "self_attn.q_proj": (256, HIDDEN, "fp8"), "self_attn.k_proj": (128, HIDDEN, "fp8"),
    "self_attn.v_proj": (128, HIDDEN, "fp8"), "self_attn.o_proj": (HIDDEN, 128, "fp8"),
}
MLP = {"mlp.gate_proj": (INTER, HIDDEN, "fp8"), "mlp.up_proj": (INTER, HIDDEN, "fp8"),
       "mlp.down_proj": (HIDDEN, INTER, "fp8")}


def model_tensors(seed=0):
    """name -> numpy array (codes u8 + scales f32, or bf16 bits, or f32)."""
    rng = np.random.default_rng(seed)
    out = {}

    def fp8(name, n, k):
        codes = rng.integers(0, 127, (n, k)).astype(np.uint8) | (rng.integers(0, 2, (n, k)) << 7).astype(np.uint8)
        scales = (rng.random((n, (k + 127) // 128)) * 0.01 + 1e-3).astype(np.float32)
        out[name] = (codes, scales)

    def bf16(name, shape):
        f = rng.standard_normal(shape).astype(np.float32)
        out[name] = (torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy(), None)

    for i, layer in enumerate((LAYER0, LAYER1)):
        p = f"model.language_model.layers.{i}."
        for short, (n, k, kind) in {**layer, **MLP}.items():
            (fp8 if kind == "fp8" else lambda nm, a, b: bf16(nm, (a, b)))(p + short + ".weight", n, k)
        bf16(p + "input_layernorm.weight", (HIDDEN,))
        bf16(p + "post_attention_layernorm.weight", (HIDDEN,))
    out["model.language_model.layers.0.linear_attn.A_log"] = (rng.standard_normal(4).astype(np.float32), None)
    fp8("lm_head.weight", VOCAB, HIDDEN)
    bf16("model.language_model.norm.weight", (HIDDEN,))
    fp8("mtp.layers.0.mlp.gate_proj.weight", INTER, HIDDEN)
    fp8("mtp.layers.0.mlp.up_proj.weight", INTER, HIDDEN)
    for short, (n, k, _) in LAYER1.items():
        fp8(f"mtp.layers.0.{short}.weight", n, k)
    return out


def write_artifact(root, tensors, tp=1, incomplete=False, fmt="avi-v1", edit=None):
    """The layout of tools/import_fp8.py:60-83 (every rank gets the full
    tensors; the tests only slice the head)."""
    os.makedirs(root, exist_ok=True)
    config = {"model_type": "qwen3_5", "text_config": {
        "vocab_size": VOCAB, "hidden_size": HIDDEN, "layer_types": ["linear_attention", "full_attention"]}}
    manifest = {"format": fmt, "tp": tp, "config": config, "ranks": [{"tensors": {}} for _ in range(tp)]}
    for r in range(tp):
        os.makedirs(os.path.join(root, f"rank{r}"), exist_ok=True)
        for name, (data, scale) in tensors.items():
            fn = f"rank{r}/{name}.bin"
            data.tofile(os.path.join(root, fn))
            dtype = {np.uint8: "U8", np.int16: "BF16", np.float32: "F32"}[data.dtype.type]
            desc = {"file": fn, "shape": list(data.shape), "dtype": dtype}
            if scale is not None:
                scale.tofile(os.path.join(root, fn + ".scale"))
                desc["scale"] = {"file": fn + ".scale", "dtype": "F32", "shape": list(scale.shape)}
            manifest["ranks"][r]["tensors"][name] = desc
    if edit:
        edit(manifest)
    with open(os.path.join(root, "manifest.json"), "w") as f:
        json.dump(manifest, f)
    if incomplete:
        open(os.path.join(root, "INCOMPLETE"), "w").write("Import in progress")
    return root


def as_bits(t):
    return t.contiguous().view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()


def test_load_and_fuse(fp8lin, tmp_path):
    src = model_tensors()
    root = write_artifact(str(tmp_path / "a"), src)
    engine, tensors, config = fp8lin.load_linear_engine(root, device="cpu")
    W = engine.weights
    p0, p1 = "model.language_model.layers.0", "model.language_model.layers.1"
    # gate_up = cat(gate, up) rows, codes and scales (src/engine.cpp:116,167)
    for p in (p0, p1):
        gu = W[p + ".mlp.gate_up.weight"]
        g, u = src[p + ".mlp.gate_proj.weight"], src[p + ".mlp.up_proj.weight"]
        assert np.array_equal(gu.data.numpy(), np.concatenate([g[0], u[0]]))
        assert np.array_equal(gu.scale.numpy(), np.concatenate([g[1], u[1]]))
        assert p + ".mlp.gate_proj.weight" not in W and p + ".mlp.down_proj.weight" in W
    qkv = W[p1 + ".self_attn.qkv_gate.weight"]
    assert qkv.data.shape == (512, HIDDEN)
    assert np.array_equal(qkv.data.numpy()[256:384], src[p1 + ".self_attn.k_proj.weight"][0])
    # GDN: [FP8 qkv + z] and [BF16 b + a] become two groups (src/engine.cpp:150-163)
    kids = engine.mixed_projections[p0 + ".linear_attn.in_proj_all"]
    assert kids == [p0 + ".linear_attn.in_proj_all.group0", p0 + ".linear_attn.in_proj_all.group1"]
    g0, g1 = W[kids[0] + ".weight"], W[kids[1] + ".weight"]
    assert g0.data.shape == (512, HIDDEN) and g0.scale is not None
    assert g1.data.dtype == torch.bfloat16 and g1.scale is None and g1.data.shape == (8, HIDDEN)
    assert np.array_equal(as_bits(g1.data)[4:], src[p0 + ".linear_attn.in_proj_a.weight"][0])
    # non-matrix tensors by name, F32 kept, MTP filtered
    assert tensors["model.language_model.layers.0.linear_attn.A_log"].dtype == torch.float32
    assert as_bits(tensors["model.language_model.norm.weight"]).tolist() == \
        src["model.language_model.norm.weight"][0].tolist()
    assert not any(n.startswith("mtp.") for n in list(W) + list(tensors))
    assert config["text_config"]["vocab_size"] == VOCAB


def test_unoptimized_keeps_projections_and_mtp(fp8lin, tmp_path):
    root = write_artifact(str(tmp_path / "a"), model_tensors())
    opt = fp8lin.LinearOptions(optimized=False)
    engine, _, _ = fp8lin.load_linear_engine(root, device="cpu", options=opt, mtp=True)
    assert "model.language_model.layers.0.mlp.gate_proj.weight" in engine.weights
    assert not engine.mixed_projections
    assert "mtp.layers.0.mlp.gate_proj.weight" in engine.weights
    engine, _, _ = fp8lin.load_linear_engine(root, device="cpu", mtp=True)
    assert engine.weights["mtp.layers.0.mlp.gate_up.weight"].data.shape == (2 * INTER, HIDDEN)


def test_vocab_sharded_head(fp8lin, tmp_path):
    src = model_tensors()
    root = write_artifact(str(tmp_path / "a"), src, tp=2)
    for rank in (0, 1):
        engine, _, _ = fp8lin.load_linear_engine(root, rank=rank, world=2, device="cpu", tp_lm_head=True)
        head = engine.weights["lm_head.weight"]
        rows = slice(rank * VOCAB // 2, (rank + 1) * VOCAB // 2)
        assert np.array_equal(head.data.numpy(), src["lm_head.weight"][0][rows])
        assert np.array_equal(head.scale.numpy(), src["lm_head.weight"][1][rows])
    engine, _, _ = fp8lin.load_linear_engine(root, rank=1, world=2, device="cpu")
    assert engine.weights["lm_head.weight"].data.shape == (VOCAB, HIDDEN)


@pytest.mark.parametrize("case,msg", [
    ("incomplete", "Incomplete model export"),
    ("format", "Artifact format or TP mismatch"),
    ("tp", "Artifact format or TP mismatch"),
    ("absolute", "Absolute tensor path rejected"),
    ("traversal", "Path traversal rejected"),
    ("scalar", "Scalar tensors must be exported as [1]"),
    ("negative", "Invalid tensor shape"),
    ("dtype", "Unsupported dtype"),
    ("size", "Tensor byte count mismatch"),
    ("head", "LM head vocabulary must divide TP size"),
])
def test_loader_rejects(fp8lin, tmp_path, case, msg):
    """src/engine.cpp:46-60,66-68,106: every loader check is an error."""
    src = model_tensors()
    name = "model.language_model.norm.weight"

    def edit(m):
        d = m["ranks"][0]["tensors"][name]
        if case == "absolute":
            d["file"] = "/etc/" + d["file"]
        elif case == "traversal":
            d["file"] = "rank0/../rank0/" + name + ".bin"
        elif case == "scalar":
            d["shape"] = []
        elif case == "negative":
            d["shape"] = [-HIDDEN]
        elif case == "dtype":
            d["dtype"] = "F16"
        elif case == "size":
            d["shape"] = [HIDDEN + 1]
        elif case == "head":
            m["config"]["text_config"]["vocab_size"] = VOCAB + 1
    tp = 2 if case == "head" else 1
    root = write_artifact(str(tmp_path / "a"), src, tp=tp, incomplete=case == "incomplete",
                          fmt="avi-v0" if case == "format" else "avi-v1", edit=edit)
    world = 3 if case == "tp" else tp
    with pytest.raises(fp8lin.Fp8linError, match=msg.replace("[", r"\[").replace("]", r"\]")):
        fp8lin.load_linear_engine(root, world=world, device="cpu", tp_lm_head=case == "head")
