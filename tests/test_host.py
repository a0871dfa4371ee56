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


def test_reference_prefill_keeps_source_views(fp8lin):
    """--reference-prefill (src/engine.cpp:170-175): the fused weight is one
    allocation and each source name stays as a view of its rows of it."""
    eng = fp8lin.LinearEngine(reference_prefill=True)
    g, gs = _fp8(256, 384)
    u, us = _fp8(128, 384)
    eng.add("l.mlp.gate_proj.weight", g, gs)
    eng.add("l.mlp.up_proj.weight", u, us)
    eng.fuse_weights("l.mlp.gate_up", ["l.mlp.gate_proj", "l.mlp.up_proj"])
    fused = eng.weights["l.mlp.gate_up.weight"]
    gv, uv = eng.weights["l.mlp.gate_proj.weight"], eng.weights["l.mlp.up_proj.weight"]
    assert torch.equal(gv.data, g) and torch.equal(gv.scale, gs)
    assert torch.equal(uv.data, u) and torch.equal(uv.scale, us)
    assert gv.data.data_ptr() == fused.data.data_ptr()
    assert uv.data.data_ptr() == fused.data.data_ptr() + 256 * 384
    assert uv.scale.data_ptr() == fused.scale.data_ptr() + 256 * 3 * 4
    assert gv.data.is_contiguous() and uv.scale.is_contiguous()


def test_reference_prefill_step_mode(fp8lin):
    """Engine::step turns `optimized` off for a prefill step under
    --reference-prefill and restores it (src/engine.cpp:403-405); decode and
    verification steps and engines without the option keep it."""
    eng = fp8lin.LinearEngine(reference_prefill=True)
    with eng.step_mode():
        assert not eng.options.optimized
    assert eng.options.optimized
    for kw in ({"decode": True}, {"verifying": True}):
        with eng.step_mode(**kw):
            assert eng.options.optimized
    plain = fp8lin.LinearEngine()
    with plain.step_mode():
        assert plain.options.optimized
    with pytest.raises(ValueError):
        with eng.step_mode():
            raise ValueError("restored on the way out")
    assert eng.options.optimized


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


def test_engine_option_checks(fp8lin):
    """The Engine constructor's linear-path option checks (src/engine.cpp:78-81)."""
    O = fp8lin.LinearOptions
    for opt, msg in [(O(fp8_tensor_small=True, tilelang_fp8=True), "Choose one FP8 Tensor Core backend"),
                     (O(fp8_tensor_small=True, optimized=False), "FP8 Tensor Core requires optimized mode"),
                     (O(tilelang_fp8=True, optimized=False), "FP8 Tensor Core requires optimized mode"),
                     (O(fp8_tensor_split=2), "FP8 Tensor Core split must be 1 or 4")]:
        with pytest.raises(fp8lin.Fp8linError, match=msg) as e:
            fp8lin.LinearEngine(opt)
        assert e.value.code == fp8lin.ERR_ARGUMENT
    fp8lin.LinearEngine(O(optimized=False))
    fp8lin.LinearEngine(O(tilelang_fp8=True, fp8_tensor_split=4))


def test_profile_labels_and_cache_order():
    """Engine::linear's timing labels (src/engine.cpp:203) and the decoded
    cache's fill order (src/engine.cpp:133-137)."""
    from fp8lin.engine import cache_order, profile_label
    assert profile_label("lm_head") == "linear.head"
    assert profile_label("model.visual.blocks.0.mlp.fc1") == "linear.vision"
    assert profile_label("mtp.layers.0.mlp.gate_up") == "linear.mtp"
    assert profile_label("model.language_model.layers.3.mlp.down_proj") == "linear.text"
    names = ["model.language_model.layers.1.a.weight", "model.visual.b.weight", "mtp.layers.0.z.weight",
             "model.language_model.layers.0.a.weight", "model.visual.a.weight", "mtp.fc.weight"]
    assert cache_order(names, False) == sorted(names)
    assert cache_order(names, True) == ["mtp.fc.weight", "mtp.layers.0.z.weight", "model.visual.a.weight",
                                        "model.visual.b.weight", "model.language_model.layers.0.a.weight",
                                        "model.language_model.layers.1.a.weight"]


def test_cache_candidates_and_budget(fp8lin):
    """Which matrices the cache may hold (src/engine.cpp:130-132) and the
    budget rule: a matrix is decoded only if it fits in what is left."""
    eng = fp8lin.LinearEngine(cache_vision_weights=True)
    for name in ["model.language_model.layers.0.mlp.down_proj.weight", "mtp.fc.weight",
                 "model.visual.blocks.0.attn.qkv.weight", "lm_head.weight"]:
        eng.add(name, *_fp8(128, 128))
    eng.add("model.language_model.layers.0.in_proj_b.weight", torch.zeros(4, 128, dtype=torch.bfloat16))
    assert sorted(eng.cache_candidates()) == ["model.language_model.layers.0.mlp.down_proj.weight",
                                              "model.visual.blocks.0.attn.qkv.weight", "mtp.fc.weight"]
    eng.cache_vision_weights = False
    assert "model.visual.blocks.0.attn.qkv.weight" not in eng.cache_candidates()


def test_bias_record(fp8lin):
    """`name.bias` travels with the weight record (added after the product,
    src/engine.cpp:240); a bias of the wrong length or dtype is rejected."""
    eng = fp8lin.LinearEngine()
    eng.add("h.weight", *_fp8(16, 256))
    assert eng._record("h").bias is None
    b = torch.randn(16).to(torch.bfloat16)
    eng.add("h.bias", b)
    assert eng._record("h").bias == eng.biases["h.bias"].data_ptr()
    eng.add("h.bias", torch.randn(15).to(torch.bfloat16))
    with pytest.raises(fp8lin.Fp8linError):
        eng._record("h")
    with pytest.raises(fp8lin.Fp8linError):
        eng.add("g.bias", torch.randn(16))
    assert eng.cache_stats() == {"fp8_tensor_calls": 0, "tilelang_fp8_calls": 0}
    assert eng.profile_report() == {}
