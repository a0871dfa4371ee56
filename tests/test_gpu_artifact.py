"""A small avi-v1 artefact loaded onto the GPU (fp8lin.load_linear_engine)
and run through Engine::linear's dispatch: fused projections, the mixed
FP8/BF16 GDN group, the decoded cache and the vocab-sharded head, each
against the oracle on the unfused source matrices."""
import numpy as np
import pytest
import torch

from parity import assert_parity
from test_artifact import HIDDEN, VOCAB, model_tensors, write_artifact

pytestmark = pytest.mark.gpu


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def rand_x(m, k, seed):
    f = np.random.default_rng(seed).standard_normal((m, k)).astype(np.float32)
    return torch.from_numpy(f).to(torch.bfloat16)


@pytest.mark.parametrize("m", [1, 4, 33])
@pytest.mark.parametrize("cache", [0, 1 << 30])
def test_artifact_projections(fp8lin, gpu, oracle, tmp_path, m, cache):
    src = model_tensors(seed=m)
    root = write_artifact(str(tmp_path / "a"), src)
    engine, _, _ = fp8lin.load_linear_engine(root, device=gpu, weight_cache_bytes=cache)
    assert bool(engine.decoded_weights) == bool(cache)
    x = rand_x(m, HIDDEN, seed=m)
    xb = bits(x)
    xg = x.to(gpu)
    p0, p1 = "model.language_model.layers.0", "model.language_model.layers.1"

    def ref(*names):
        parts = []
        for n in names:
            data, scale = src[n + ".weight"]
            if scale is None:
                parts.append(oracle.linear_bf16w(xb, data.view(np.uint16)))
            else:
                parts.append(oracle.linear(xb, data, scale))
        return np.concatenate(parts, axis=1)

    cases = {
        p0 + ".mlp.gate_up": [p0 + ".mlp.gate_proj", p0 + ".mlp.up_proj"],
        p1 + ".self_attn.qkv_gate": [p1 + ".self_attn.q_proj", p1 + ".self_attn.k_proj",
                                     p1 + ".self_attn.v_proj"],
        p0 + ".linear_attn.in_proj_all": [p0 + ".linear_attn.in_proj_qkv", p0 + ".linear_attn.in_proj_z",
                                          p0 + ".linear_attn.in_proj_b", p0 + ".linear_attn.in_proj_a"],
        "lm_head": ["lm_head"],
    }
    for fused, parts in cases.items():
        y = engine.linear(xg, fused)
        assert_parity(bits(y), ref(*parts), f"{fused} m={m} cache={cache}")


def test_artifact_sharded_head_candidates(fp8lin, gpu, tmp_path):
    """Two ranks' head shards with their vocabulary candidates, merged: the
    token equals the argmax over the unsharded head's logits."""
    src = model_tensors(seed=7)
    root = write_artifact(str(tmp_path / "a"), src, tp=2)
    x = rand_x(3, HIDDEN, seed=3).to(gpu)
    cands = []
    for rank in (0, 1):
        engine, _, _ = fp8lin.load_linear_engine(root, rank=rank, world=2, device=gpu, tp_lm_head=True)
        w = engine.weights["lm_head.weight"]
        cands.append(fp8lin.linear_candidates(x, w.data, w.scale, rank * (VOCAB // 2)))
    ids = fp8lin.merge_candidates(torch.stack(cands).contiguous())
    codes, scales = src["lm_head.weight"]
    full = fp8lin.fp8_linear(x, torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu))
    assert torch.equal(ids, full.float().argmax(-1))
