"""Reader for the reference's on-disk model artefact ("avi-v1") feeding the
linear path: the manifest, the per-rank raw tensor files and the load-time
steps of `Engine::Engine` that concern linear weights.

Layout (written by the reference's tools/import_fp8.py:60-83):
  <dir>/manifest.json   {"format": "avi-v1", "tp": T, "config": {...},
                         "ranks": [{"tensors": {name: desc}}, ...]}
  <dir>/rank<r>/<name>.bin          raw little-endian tensor bytes
  <dir>/rank<r>/<name>.bin.scale    FP32 row-expanded block scales (FP8 only)
  desc = {"file": relative path, "shape": [...], "dtype": "U8"|"BF16"|"F32"|"I64",
          "scale": desc (FP8 codes only)}
  <dir>/INCOMPLETE exists while an import is in progress.

Checks follow src/engine.cpp:44-62 (`raw`) and :63-67 (manifest); the
steps after loading follow :95-143 (MTP filter, vocab-sharded head slice,
projection fusion, decoded cache).
"""
import json
import os

import numpy as np
import torch

from ._lib import ERR_ARGUMENT, ERR_SHAPE, Fp8linError

_DTYPES = {
    "BF16": (np.int16, torch.bfloat16),
    "F32": (np.float32, torch.float32),
    "I64": (np.int64, torch.int64),
    "U8": (np.uint8, torch.uint8),
}


def _fail(msg, code=ERR_ARGUMENT):
    raise Fp8linError(code, msg)


def read_manifest(directory, world):
    """src/engine.cpp:66-68: a finished import of format avi-v1 for `world`
    tensor-parallel ranks."""
    if os.path.exists(os.path.join(directory, "INCOMPLETE")):
        _fail("Incomplete model export")
    path = os.path.join(directory, "manifest.json")
    if not os.path.isfile(path):
        _fail(f"Cannot open {path}")
    with open(path, encoding="utf-8") as f:
        manifest = json.load(f)
    if manifest.get("format") != "avi-v1" or manifest.get("tp") != world:
        _fail("Artifact format or TP mismatch")
    return manifest


def read_tensor(directory, desc, device="cpu"):
    """`raw(dir, desc, device)` (src/engine.cpp:45-62): a relative path with
    no "..", a non-empty shape of positive extents, a supported dtype and a
    file of exactly the tensor's byte count."""
    rel = desc["file"]
    if os.path.isabs(rel):
        _fail("Absolute tensor path rejected")
    if any(part == ".." for part in rel.replace("\\", "/").split("/")):
        _fail("Path traversal rejected")
    shape = [int(s) for s in desc["shape"]]
    if not shape:
        _fail("Scalar tensors must be exported as [1]", ERR_SHAPE)
    n = 1
    for s in shape:
        if s <= 0 or n > (2 ** 63 - 1) // s:
            _fail("Invalid tensor shape", ERR_SHAPE)
        n *= s
    if desc["dtype"] not in _DTYPES:
        _fail(f"Unsupported dtype {desc['dtype']}")
    np_type, torch_type = _DTYPES[desc["dtype"]]
    path = os.path.join(directory, rel)
    nbytes = n * np.dtype(np_type).itemsize
    if not os.path.isfile(path) or os.path.getsize(path) != nbytes:
        _fail(f"Tensor byte count mismatch: {path}", ERR_SHAPE)
    data = np.fromfile(path, dtype=np.dtype(np_type).newbyteorder("<"), count=n)
    if data.size != n:
        _fail(f"Short tensor read: {path}", ERR_SHAPE)
    t = torch.from_numpy(data.astype(np_type, copy=False).reshape(shape))
    if torch_type == torch.bfloat16:
        t = t.view(torch.bfloat16)
    return t.to(device)


def load_linear_engine(directory, rank=0, world=1, device="cuda", options=None, weight_cache_bytes=0,
                       tp_lm_head=False, mtp=False, cache_vision_weights=False):
    """Load one rank's tensors and prepare the linear path as
    `Engine::Engine` does (src/engine.cpp:95-143).

    Returns (engine, tensors, config): a LinearEngine holding every 2-D
    `.weight` matrix (FP8 codes with their scales, or BF16), fused per the
    model's layer types when `options.optimized`, and every BF16 `.bias`
    vector of such a matrix (added by `LinearEngine.linear`,
    src/engine.cpp:240); every tensor that is not a matrix by name (biases
    included); the manifest's model config."""
    from ._lib import LinearOptions
    from .engine import LinearEngine

    options = options or LinearOptions()
    manifest = read_manifest(directory, world)
    if not 0 <= rank < world:
        _fail("Invalid rank")
    config = manifest["config"]
    text = config.get("text_config", config)
    engine = LinearEngine(options, weight_cache_bytes, cache_vision_weights=cache_vision_weights)
    tensors = {}
    for name, desc in manifest["ranks"][rank]["tensors"].items():
        if not mtp and name.startswith("mtp."):  # src/engine.cpp:97
            continue
        data = read_tensor(directory, desc, device)
        scale = read_tensor(directory, desc["scale"], device) if "scale" in desc else None
        if scale is not None and data.dtype != torch.uint8:  # tools/import_fp8.py:69-71
            _fail(f"Non-FP8 weight has a scale: {name}")
        if name.endswith(".weight") and data.dim() == 2:
            engine.add(name, data, scale)
        else:
            tensors[name] = data
    if tp_lm_head and world > 1:  # src/engine.cpp:104-112
        head = engine.weights.get("lm_head.weight")
        vocab = int(text["vocab_size"])
        if head is None or vocab % world or head.data.size(0) != vocab:
            _fail("LM head vocabulary must divide TP size")
        rows = vocab // world
        begin = rank * rows
        head.data = head.data.narrow(0, begin, rows).clone()
        if head.scale is not None:
            head.scale = head.scale.narrow(0, begin, rows).clone()
        if "lm_head.bias" in tensors:
            tensors["lm_head.bias"] = tensors["lm_head.bias"].narrow(0, begin, rows).clone()
    if options.optimized:  # src/engine.cpp:113-125
        for i, kind in enumerate(text["layer_types"]):
            p = f"model.language_model.layers.{i}"
            engine.fuse_weights(p + ".mlp.gate_up", [p + ".mlp.gate_proj", p + ".mlp.up_proj"])
            if kind == "full_attention":
                engine.fuse_weights(p + ".self_attn.qkv_gate",
                                    [p + ".self_attn.q_proj", p + ".self_attn.k_proj", p + ".self_attn.v_proj"])
            else:
                engine.fuse_weights(p + ".linear_attn.in_proj_all",
                                    [p + ".linear_attn.in_proj_qkv", p + ".linear_attn.in_proj_z",
                                     p + ".linear_attn.in_proj_b", p + ".linear_attn.in_proj_a"])
        if mtp:
            engine.fuse_weights("mtp.layers.0.mlp.gate_up", ["mtp.layers.0.mlp.gate_proj", "mtp.layers.0.mlp.up_proj"])
            engine.fuse_weights("mtp.layers.0.self_attn.qkv_gate",
                                ["mtp.layers.0.self_attn.q_proj", "mtp.layers.0.self_attn.k_proj",
                                 "mtp.layers.0.self_attn.v_proj"])
    for name, data in tensors.items():  # src/engine.cpp:240 finds `name.bias` by name
        if name.endswith(".bias") and data.dim() == 1 and data.dtype == torch.bfloat16 and \
                name[:-5] + ".weight" in engine.weights:
            engine.add(name, data)
    if weight_cache_bytes:  # src/engine.cpp:127-143
        engine.build_cache(engine.cache_candidates())
    return engine, tensors, config
