"""Host-side logic of the engine mirror that needs no GPU: load-time fusion of
projections and mixed-precision grouping (src/engine.cpp:147-177), and the
tensor checks of the operator wrappers."""
import pytest
import torch


def _fp8(n, k):
    return torch.randint(0, 126, (n, k), dtype=torch.uint8), torch.rand(n, (k + 127) // 128)


def test_fuse_compatible_rows(fp8lin):
    eng = fp8lin.LinearEngine()
    g, gs = _fp8(256, 384)
    u, us = _fp8(256, 384)
    eng.add("l.mlp.gate_proj.weight", g, gs)
    eng.add("l.mlp.up_proj.weight", u, us)
    eng.fuse_weights("l.mlp.gate_up", ["l.mlp.gate_proj", "l.mlp.up_proj"])
    fused = eng.weights["l.mlp.gate_up.weight"]
    assert torch.equal(fused.data, torch.cat([g, u])) and torch.equal(fused.scale, torch.cat([gs, us]))
    assert "l.mlp.gate_proj.weight" not in eng.weights and not eng.mixed_projections


def test_fuse_mixed_groups_keep_order(fp8lin):
    """Qwen GDN in_proj_all: [FP8 qkv + z] and [BF16 b + a] become two groups
    (src/engine.cpp:151-165, tests/optimized_test.cpp:89-98)."""
    eng = fp8lin.LinearEngine()
    q, qs = _fp8(384, 256)
    z, zs = _fp8(128, 256)
    b = torch.randn(4, 256).to(torch.bfloat16)
    a = torch.randn(4, 256).to(torch.bfloat16)
    for name, d, s in [("qkv", q, qs), ("z", z, zs), ("b", b, None), ("a", a, None)]:
        eng.add(f"p.{name}.weight", d, s)
    eng.fuse_weights("p.all", ["p.qkv", "p.z", "p.b", "p.a"])
    assert eng.mixed_projections["p.all"] == ["p.all.group0", "p.all.group1"]
    assert torch.equal(eng.weights["p.all.group0.weight"].data, torch.cat([q, z]))
    assert torch.equal(eng.weights["p.all.group1.weight"].data, torch.cat([b, a]))
    assert eng.weights["p.all.group1.weight"].scale is None


def test_fuse_single_members_stay_unfused(fp8lin):
    eng = fp8lin.LinearEngine()
    q, qs = _fp8(128, 256)
    q1, q1s = torch.randint(0, 126, (128, 256), dtype=torch.uint8), torch.rand(128)   # 1-D scales
    b = torch.randn(4, 256).to(torch.bfloat16)
    eng.add("p.q.weight", q, qs)
    eng.add("p.r.weight", q1, q1s)
    eng.add("p.b.weight", b)
    eng.fuse_weights("p.all", ["p.q", "p.r", "p.b"])
    assert eng.mixed_projections["p.all"] == ["p.q", "p.r", "p.b"]


def test_operator_checks_raise(fp8lin):
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    codes = torch.zeros(16, 128, dtype=torch.uint8)
    scales = torch.ones(16, 1)
    with pytest.raises(fp8lin.Fp8linError):
        fp8lin.fp8_linear(x, codes, scales)            # CPU tensors are rejected
    with pytest.raises(fp8lin.Fp8linError):
        fp8lin.fused_swiglu(torch.zeros(2, 3, dtype=torch.bfloat16))
    with pytest.raises(fp8lin.Fp8linError):
        fp8lin.fp8_tensor_small(x, codes, scales, split=4)


def test_qkv_gate_views(fp8lin):
    """src/engine.cpp:279-282: q_proj rows are per head [q(D) | gate(D)], then
    k_proj and v_proj; the fused output splits back into the four parts."""
    import torch
    T, H, HK, D = 3, 2, 1, 4
    q_proj = torch.arange(T * H * 2 * D, dtype=torch.float32).reshape(T, H * 2 * D)
    k_proj = 1000 + torch.arange(T * HK * D, dtype=torch.float32).reshape(T, HK * D)
    v_proj = 2000 + torch.arange(T * HK * D, dtype=torch.float32).reshape(T, HK * D)
    fused = torch.cat([q_proj, k_proj, v_proj], 1)
    q, gate, k, v = fp8lin.LinearEngine.qkv_gate_views(fused, H, HK, D)
    per_head = q_proj.reshape(T, H, 2 * D)
    assert torch.equal(q, per_head[..., :D]) and torch.equal(gate, per_head[..., D:].reshape(T, H * D))
    assert torch.equal(k, k_proj.reshape(T, HK, D)) and torch.equal(v, v_proj.reshape(T, HK, D))
    assert q.data_ptr() == fused.data_ptr()
    import pytest
    with pytest.raises(fp8lin.Fp8linError):
        fp8lin.LinearEngine.qkv_gate_views(fused[:, 1:], H, HK, D)
