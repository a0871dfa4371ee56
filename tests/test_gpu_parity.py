"""GPU parity: every HIP path against the CPU oracle on identical inputs.

Shapes and data follow the reference's own kernel tests
(tests/kernel_test.cpp, tests/optimized_test.cpp, tests/fp8_tensor_test.cpp)
with numpy's seeded RNG in place of the CUDA RNG, plus the benchmark shapes.
Bar: <= 1 BF16 ulp from the FP64 oracle (or rel-L2 <= 1e-2 and cosine >=
0.9999), allclose(rtol .01, atol .001), and -- for the kernels that keep the
reference rounding point -- >= 90% of outputs bit-identical.
"""
import numpy as np
import pytest
import torch

from parity import assert_parity, bf16_to_f32, ulp_distance

pytestmark = pytest.mark.gpu


def up(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if a.dtype == np.uint16:
        t = t.view(torch.bfloat16)
    return t.to(dev)


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def rand_bf16(rng, shape, scale=1.0):
    f = (rng.standard_normal(shape) * scale).astype(np.float32)
    return torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def rand_codes(rng, n, k, signed=True):
    c = rng.integers(0, 127, (n, k), dtype=np.uint8)
    if signed:
        c = c | (rng.integers(0, 2, (n, k), dtype=np.uint8) << 7)
    return c


# ------------------------------------------------------------- decode / dequant
def test_decode_all_codes(fp8lin, gpu, oracle):
    """tests/kernel_test.cpp:16-24 on the device: every code, scale 1."""
    codes = np.arange(256, dtype=np.uint8).reshape(1, 256)
    y = fp8lin.fp8_decode(up(codes, gpu), torch.ones(1, device=gpu))
    got = bf16_to_f32(bits(y))[0]
    ref = oracle.decode_table()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.array_equal(np.signbit(got[~nan]), np.signbit(ref[~nan]))


@pytest.mark.parametrize("n,k,blockscale", [(137, 257, True), (64, 512, True), (19, 132, False),
                                            (300, 5120, True), (3, 17, True)])
def test_dequant_bit_exact(fp8lin, gpu, oracle, n, k, blockscale):
    rng = np.random.default_rng(n * 7 + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, (k + 127) // 128) if blockscale else n) * .01 + .001).astype(np.float32)
    y = fp8lin.fp8_decode(up(codes, gpu), up(scales, gpu))
    assert np.array_equal(bits(y), oracle.dequant(codes, scales))


# ------------------------------------------------------------------ generators
def test_generators_match_oracle(fp8lin, gpu, oracle):
    z = fp8lin.gen_normal(1 << 20, seed=0, tag=1, first=12345, device=gpu).cpu().numpy()
    assert np.array_equal(z.view(np.uint32), oracle.normal(0, 1, 12345, 1 << 20).view(np.uint32))
    codes, scales = fp8lin.gen_weights(300, 520, seed=0, tag=1, device=gpu)
    oc, os_ = oracle.gen_weights(0, 1, 300, 520, 0.02)
    assert np.array_equal(codes.cpu().numpy(), oc)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), os_.view(np.uint32))
    x = fp8lin.gen_activations(3, 1000, seed=5, tag=2, device=gpu)
    assert np.array_equal(bits(x), oracle.gen_activations(5, 2, 3, 1000))


# ------------------------------------------------------------ decode GEMV (A3-A5)
@pytest.mark.parametrize("m", [1, 2, 8])
@pytest.mark.parametrize("k", [4, 128, 132, 257, 5120])
def test_gemv_signed_subnormal(fp8lin, gpu, oracle, m, k):
    """tests/optimized_test.cpp:49-56: signed/subnormal codes, block
    boundaries, batch rows, scalar fallback (K % 16 != 0)."""
    rng = np.random.default_rng(m * 100 + k)
    n = 19
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, (k + 127) // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    y = fp8lin.fp8_linear(up(x, gpu), up(codes, gpu), up(scales, gpu), vector_gemv=True)
    assert_parity(bits(y), oracle.linear(x, codes, scales), f"gemv m={m} k={k}")


@pytest.mark.parametrize("m", [1, 4, 17, 33])
@pytest.mark.parametrize("k", [32, 70])
def test_linear_row_scales(fp8lin, gpu, oracle, m, k):
    """tests/optimized_test.cpp:71-77: 1-D per-row scales, GEMV and GEMM."""
    rng = np.random.default_rng(m * 10 + k)
    n = 79
    codes = rng.integers(0, 126, (n, k), dtype=np.uint8)
    scales = (rng.random(n) * .01).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    y = fp8lin.fp8_linear(up(x, gpu), up(codes, gpu), up(scales, gpu))
    assert_parity(bits(y), oracle.linear(x, codes, scales), f"row scales m={m} k={k}")


@pytest.mark.parametrize("m", [1, 4, 17])
def test_linear_block_tail(fp8lin, gpu, oracle, m):
    """tests/optimized_test.cpp:79-88: N=137, K=257, three scale blocks."""
    rng = np.random.default_rng(m)
    n, k = 137, 257
    codes = rng.integers(0, 126, (n, k), dtype=np.uint8)
    scales = (rng.random((n, 3)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    y = fp8lin.fp8_linear(up(x, gpu), up(codes, gpu), up(scales, gpu))
    assert_parity(bits(y), oracle.linear(x, codes, scales), f"block tail m={m}")


def test_unaligned_view_bit_equal(fp8lin, gpu, oracle):
    """tests/optimized_test.cpp:57-62: an unaligned contiguous view takes the
    byte-load path and gives the same bits as the aligned one."""
    rng = np.random.default_rng(9)
    k = 5120
    x = rand_bf16(rng, (1, k))
    codes = rand_codes(rng, 64, k)
    scales = (rng.random((64, k // 128)) * .01 + .001).astype(np.float32)
    big = torch.zeros(k + 1, dtype=torch.bfloat16, device=gpu)
    big[1:] = up(x, gpu)[0]
    xu = big.narrow(0, 1, k).reshape(1, k)
    cbig = torch.zeros(64 * k + 1, dtype=torch.uint8, device=gpu)
    cbig[1:] = up(codes, gpu).reshape(-1)
    cu = cbig.narrow(0, 1, 64 * k).reshape(64, k)
    ya = fp8lin.fp8_linear(up(x, gpu), up(codes, gpu), up(scales, gpu), True)
    yu = fp8lin.fp8_linear(xu, cu, up(scales, gpu), True)
    assert torch.equal(ya, yu)
    assert_parity(bits(ya), oracle.linear(x, codes, scales), "aligned")


@pytest.mark.parametrize("m", [1, 2, 4, 6, 8])
@pytest.mark.parametrize("k", [17, 128, 257, 5120])
def test_shared_gemv_fp8_equals_bf16(fp8lin, gpu, oracle, m, k):
    """tests/optimized_test.cpp:7-14: shared GEMV on FP8 == on the decoded
    BF16 weights, bit for bit (pins the rounding point)."""
    rng = np.random.default_rng(m * 1000 + k)
    n = 19
    codes = rng.integers(0, 126, (n, k), dtype=np.uint8)
    scales = (rng.random((n, (k + 127) // 128)) * .01 + .001).astype(np.float32)
    x = up(rand_bf16(rng, (m, k)), gpu)
    c, s = up(codes, gpu), up(scales, gpu)
    decoded = fp8lin.fp8_decode(c, s)
    a = fp8lin.small_linear_shared(x, c, s)
    b = fp8lin.small_linear_shared(x, decoded)
    assert torch.equal(a, b)
    assert_parity(bits(a), oracle.linear(bits(x), codes, scales), f"shared m={m} k={k}")


# ---------------------------------------------------------- small-M tensor path
@pytest.mark.parametrize("m", [2, 3, 5, 8])
@pytest.mark.parametrize("k", [128, 384, 5120])
@pytest.mark.parametrize("n", [17, 80, 144])
def test_tensor_small_vs_fp64(fp8lin, gpu, oracle, m, k, n):
    """tests/fp8_tensor_test.cpp:28-39: M 2..8, tails, empty split ranges."""
    rng = np.random.default_rng(m * 10000 + k + n)
    codes = rng.integers(0, 256, (n, k), dtype=np.uint8)
    codes[(codes == 127) | (codes == 255)] = 0
    scales = (rng.random((n, k // 128)) * .001 + .0001).astype(np.float32)
    x = rand_bf16(rng, (m, k), 0.1)
    ref = oracle.linear(x, codes, scales)
    for split in (1, 4):
        y = fp8lin.fp8_tensor_small(up(x, gpu), up(codes, gpu), up(scales, gpu), split)
        assert_parity(bits(y), ref, f"tensor_small m={m} k={k} n={n} split={split}")
        if n % 16 == 0:
            y2 = fp8lin.tilelang_fp8_small(up(x, gpu), up(codes, gpu), up(scales, gpu), split)
            assert torch.equal(y, y2)


@pytest.mark.parametrize("n,k,m", [(8192, 4096, 2), (8200, 3584, 8), (9000, 8704, 5), (8240, 5120, 3),
                                   (12000, 4224, 7), (8192, 5120, 8), (5120, 8704, 8), (7168, 5120, 4),
                                   (4100, 4096, 3), (4352, 5120, 2), (12288, 4096, 8), (31040, 4096, 4),
                                   (24000, 5120, 6)])
def test_tensor_small_wide(fp8lin, gpu, oracle, n, k, m):
    """The small-M kernels by rows per compute unit at M <= 8: up to 32 rows
    the row-staged form (the decode down and QKV-gate shapes, 17 and 32 rows
    per CU); 33..80 rows at K <= 5120 the wide row-staged form (33, 36 and
    47 rows; K = 3584, 4224 and 5120), except from 48 rows at K = 4096 and
    from 81 rows, which take the persistent row-range kernel (48, 122 and 94
    rows per CU), as do K > 5120 from 33 rows (9000 x 8704: 36 rows in pieces
    of 12).  Every row against the FP64 oracle; split 1 and 4 bit-equal."""
    rng = np.random.default_rng(n + k + m)
    codes = rng.integers(0, 256, (n, k), dtype=np.uint8)
    codes[(codes == 127) | (codes == 255)] = 0
    scales = (rng.random((n, k // 128)) * .001 + .0001).astype(np.float32)
    x = rand_bf16(rng, (m, k), 0.1)
    ref = oracle.linear(x, codes, scales)
    xg, cg, sg = up(x, gpu), up(codes, gpu), up(scales, gpu)
    y1 = fp8lin.fp8_tensor_small(xg, cg, sg, 1)
    assert_parity(bits(y1), ref, f"tensor_small wide {m}x{n}x{k}")
    assert torch.equal(y1, fp8lin.fp8_tensor_small(xg, cg, sg, 4))


def test_tensor_small_graph_replay(fp8lin, gpu, oracle):
    """tests/fp8_tensor_test.cpp:40-52: a captured graph sees updated
    activations on every replay."""
    rng = np.random.default_rng(11)
    x = up(rand_bf16(rng, (4, 384), 0.1), gpu)
    codes_np = np.full((144, 384), 24, np.uint8)
    scales_np = (rng.random((144, 3)) * .1).astype(np.float32)
    codes, scales = up(codes_np, gpu), up(scales_np, gpu)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        out = fp8lin.fp8_tensor_small(x, codes, scales, 4)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = fp8lin.fp8_tensor_small(x, codes, scales, 4)
    for i in range(4):
        if i:
            x.add_(0.015625)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_parity(bits(out), oracle.linear(bits(x), codes_np, scales_np), f"replay {i}")


# ----------------------------------------------------------------- prefill GEMM
@pytest.mark.parametrize("m,n,k", [(17, 137, 257), (33, 256, 384), (256, 512, 1024),
                                   (300, 520, 640), (9, 75, 64)])
def test_gemm_fp8(fp8lin, gpu, oracle, m, n, k):
    rng = np.random.default_rng(m + n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, (k + 127) // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    y = fp8lin.fp8_linear(up(x, gpu), up(codes, gpu), up(scales, gpu))
    assert_parity(bits(y), oracle.linear(x, codes, scales), f"gemm {m}x{n}x{k}")


@pytest.mark.parametrize("n,k,swiglu", [(520, 512, False), (8200, 1024, False), (8200, 768, True),
                                        (17408, 5120, True)])
def test_gemm_tile_heights_agree(fp8lin, gpu, oracle, n, k, swiglu):
    """The FP8 GEMM runs 128-row tiles for M <= 128 and 256-row tiles above.
    Unsplit, both give every output the same FP32 sum (same K order, same
    accumulator position), so an M = 128 call equals rows 0..127 of an
    M = 129 call on the same rows bit for bit; the M = 128 call also holds
    the oracle bar (plain: a column sample, SwiGLU: all outputs of a row
    sample).  The weights have more than 32 rows per CU or at most 1024
    rows, so M = 128 runs the GEMM (narrow weights of more than 1024 rows
    run 65..128 rows as two small-M halves without a workspace)."""
    rng = np.random.default_rng(n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (129, k))
    c, s = up(codes, gpu), up(scales, gpu)
    xg = up(x, gpu)
    if swiglu:
        small = fp8lin.linear_swiglu(xg[:128].contiguous(), c, s, split=False)
        big = fp8lin.linear_swiglu(xg, c, s, split=False)
    else:
        small = fp8lin.fp8_linear(xg[:128].contiguous(), c, s, split=False)
        big = fp8lin.fp8_linear(xg, c, s, split=False)
    assert torch.equal(small, big[:128])
    if swiglu:
        rows = [0, 1, 63, 64, 127]
        ref = oracle.swiglu(oracle.linear(x[rows], codes, scales))
        assert_parity(bits(small)[rows], ref, f"swiglu tiles {n}x{k}", elementwise=False)
    else:
        cols = (max(0, n - 300), n)
        ref = oracle.linear(x[:128], codes, scales, rows=cols)
        assert_parity(bits(small)[:, cols[0]:cols[1]], ref[:, cols[0]:cols[1]], f"gemm tiles {n}x{k}")


@pytest.mark.parametrize("m,n,k", [(17, 137, 257), (300, 520, 640)])
def test_gemm_bf16(fp8lin, gpu, oracle, m, n, k):
    rng = np.random.default_rng(m * n)
    w = rand_bf16(rng, (n, k), 0.05)
    x = rand_bf16(rng, (m, k))
    y = fp8lin.gemm_bf16(up(x, gpu), up(w, gpu))
    assert_parity(bits(y), oracle.linear_bf16w(x, w), f"bf16 gemm {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(512, 48, 5120), (9, 24, 5120), (300, 256, 8704), (77, 40, 640),
                                   (4096, 48, 5120)])
@pytest.mark.parametrize("fp8", [False, True])
def test_few_weight_rows_prefill(fp8lin, gpu, oracle, m, n, k, fp8):
    """256 weight rows or fewer at more than 8 activation rows (the GDN
    in_proj_all group's 48 BF16 rows at a prefill chunk): the GEMV's prefill
    form over blocks of 8 activation rows (a ragged last block at 9, 77 and
    300 rows), against the oracle on every output; the fused SwiGLU form
    bit-equal to SwiGLU of the plain form."""
    rng = np.random.default_rng(m + n + k + fp8)
    x = rand_bf16(rng, (m, k))
    if fp8:
        codes = rand_codes(rng, n, k)
        scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
        c, s = up(codes, gpu), up(scales, gpu)
        y = fp8lin.fp8_linear(up(x, gpu), c, s)
        ref = oracle.linear(x, codes, scales)
        if n % 2 == 0:
            fused = fp8lin.linear_swiglu(up(x, gpu), c, s, split=False)
            assert torch.equal(fused, fp8lin.fused_swiglu(y))
    else:
        w = rand_bf16(rng, (n, k), 0.05)
        y = fp8lin.gemm_bf16(up(x, gpu), up(w, gpu))
        ref = oracle.linear_bf16w(x, w)
    assert_parity(bits(y), ref, f"few rows {m}x{n}x{k} fp8={fp8}")


# ---------------------------------------------------------------------- SwiGLU
def test_swiglu_standalone(fp8lin, gpu, oracle):
    rng = np.random.default_rng(12)
    g = rand_bf16(rng, (17, 2 * 257), 3.0)
    y = bits(fp8lin.fused_swiglu(up(g, gpu)))
    ref = oracle.swiglu(g)
    assert ulp_distance(y, ref).max() <= 1
    assert (y == ref).mean() > 0.99


@pytest.mark.parametrize("m,n,k", [(1, 512, 384), (5, 260, 256), (64, 512, 512), (300, 1040, 640)])
def test_linear_swiglu_fused_equals_unfused(fp8lin, gpu, oracle, m, n, k):
    """gate/up + SwiGLU fused == fused_swiglu(fp8_linear(x, gate_up))."""
    rng = np.random.default_rng(m + n)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, (k + 127) // 128)) * .01 + .001).astype(np.float32)
    x = up(rand_bf16(rng, (m, k)), gpu)
    c, s = up(codes, gpu), up(scales, gpu)
    fused = fp8lin.linear_swiglu(x, c, s, split=False)
    gate_up = fp8lin.fp8_linear(x, c, s, split=False)
    ref_gu = oracle.linear(bits(x), codes, scales)
    assert_parity(bits(gate_up), ref_gu, "gate/up")
    # SwiGLU of the device's own gate/up: only expf may differ (<= 1 ulp).
    own = oracle.swiglu(bits(gate_up))
    if m > 8:
        # Same GEMM accumulation, different epilogue: bit-identical.
        assert torch.equal(fused, fp8lin.fused_swiglu(gate_up))
        assert ulp_distance(bits(fused), own).max() <= 1
        # With a workspace the GEMM may split K (FP32 order of the split
        # tiles only); the result stays at the bar.
        split = fp8lin.linear_swiglu(x, c, s)
        assert_parity(bits(split), oracle.swiglu(ref_gu), "fused swiglu, split K", elementwise=False)
    # Against the oracle composition a 1-ulp gate difference can move a tiny
    # silu(a) (a << 0) by many ulps, so the tolerance clause applies.
    assert_parity(bits(fused), oracle.swiglu(ref_gu), "fused swiglu", elementwise=False)


# ---------------------------------------------------------- Engine::linear paths
def test_engine_paths(fp8lin, gpu, oracle):
    F = fp8lin
    rng = np.random.default_rng(13)
    n, k = 272, 640
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    ref_w = oracle.dequant(codes, scales)
    cases = [
        (F.LinearOptions(), 1, F.PATH_FP8_GEMV, False),
        (F.LinearOptions(), 20, F.PATH_FP8_GEMM, False),
        (F.LinearOptions(cublas_prefill=True), 20, F.PATH_DEQUANT_GEMM, False),
        (F.LinearOptions(optimized=False), 3, F.PATH_DEQUANT_GEMM, False),
        (F.LinearOptions(fp8_tensor_small=True, fp8_tensor_split=4), 4, F.PATH_TENSOR_SMALL, False),
        (F.LinearOptions(multi_token_gemv=True), 3, F.PATH_SHARED_GEMV, False),
        (F.LinearOptions(), 12, F.PATH_CACHED_BF16, True),
        (F.LinearOptions(multi_token_gemv=True), 3, F.PATH_SHARED_GEMV, True),
    ]
    for opt, rows, path, cache in cases:
        eng = F.LinearEngine(opt, weight_cache_bytes=(1 << 30) if cache else 0)
        eng.add("w.weight", up(codes, gpu), up(scales, gpu))
        if cache:
            eng.build_cache()
        x = rand_bf16(rng, (rows, k))
        y, p = eng.linear(up(x, gpu), "w", return_path=True)
        assert p == path, (opt, rows, p)
        assert_parity(bits(y), oracle.linear_bf16w(x, ref_w), f"engine path {path}")


@pytest.mark.parametrize("m", [1, 40])
def test_engine_reference_prefill_mlp(fp8lin, gpu, oracle, m):
    """--reference-prefill (src/engine.cpp:170-175, :403-416): gate_proj and
    up_proj stay as views of the fused gate_up; a prefill step runs them
    unoptimized (dequant-then-GEMM, src/engine.cpp:225-233) and unfused
    (silu(gate) * up), a decode step runs the fused gate_up + SwiGLU; both
    against the oracle composition, each down projection too."""
    F = fp8lin
    rng = np.random.default_rng(15 + m)
    d, k = 384, 512
    w = {}
    for name, n, kk in (("gate_proj", d, k), ("up_proj", d, k), ("down_proj", k, d)):
        c = rand_codes(rng, n, kk)
        sc = (rng.random((n, kk // 128)) * .01 + .001).astype(np.float32)
        w[name] = (c, sc)
    eng = F.LinearEngine(reference_prefill=True)
    for name, (c, sc) in w.items():
        eng.add(f"l.mlp.{name}.weight", up(c, gpu), up(sc, gpu))
    eng.fuse_weights("l.mlp.gate_up", ["l.mlp.gate_proj", "l.mlp.up_proj"])
    x = rand_bf16(rng, (m, k))
    xg = up(x, gpu)
    ref_gu = np.concatenate([oracle.linear(x, *w["gate_proj"]), oracle.linear(x, *w["up_proj"])], axis=1)
    for decode in (False, True):
        with eng.step_mode(decode=decode):
            if not decode:
                _, p = eng.linear(xg, "l.mlp.gate_proj", return_path=True)
                assert p == F.PATH_DEQUANT_GEMM
            out = eng.mlp(xg, "l.mlp")
            gated = F.fused_swiglu(eng.linear(xg, "l.mlp.gate_up")) if eng.options.optimized else None
        assert eng.options.optimized
        ref_g = oracle.swiglu(ref_gu)
        if gated is not None:
            assert_parity(bits(gated), ref_g, f"reference prefill gated m={m}", elementwise=False)
        ref = oracle.linear(ref_g, *w["down_proj"])
        assert_parity(bits(out), ref, f"reference prefill mlp m={m} decode={decode}", min_exact=None,
                      elementwise=False)


def test_engine_mixed_groups(fp8lin, gpu, oracle):
    """tests/optimized_test.cpp:89-98: grouped == separate projections."""
    F = fp8lin
    rng = np.random.default_rng(14)
    for m in (1, 17):
        qkv = rng.integers(0, 126, (384, 256), dtype=np.uint8)
        z = rng.integers(0, 126, (128, 256), dtype=np.uint8)
        qs = (rng.random((384, 2)) * .01).astype(np.float32)
        zs = (rng.random((128, 2)) * .01).astype(np.float32)
        b = rand_bf16(rng, (4, 256))
        a = rand_bf16(rng, (4, 256))
        eng = F.LinearEngine()
        for name, d, s in [("qkv", qkv, qs), ("z", z, zs), ("b", b, None), ("a", a, None)]:
            eng.add(f"p.{name}.weight", up(d, gpu), up(s, gpu) if s is not None else None)
        eng.fuse_weights("p.all", ["p.qkv", "p.z", "p.b", "p.a"])
        x = rand_bf16(rng, (m, 256))
        y = bits(eng.linear(up(x, gpu), "p.all"))
        sep = np.concatenate([oracle.linear(x, qkv, qs), oracle.linear(x, z, zs),
                              oracle.linear_bf16w(x, b), oracle.linear_bf16w(x, a)], axis=1)
        assert_parity(y, sep, f"mixed groups m={m}")


@pytest.mark.parametrize("m", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("k", [9344, 10240, 12288])
def test_gemv_long_k(fp8lin, gpu, oracle, m, k):
    """K > 9216: the decode GEMV's four-wave step split (and its byte-load
    form on an unaligned view) against the oracle."""
    rng = np.random.default_rng(m * 7 + k)
    n = 300
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s = up(codes, gpu), up(scales, gpu)
    xg = up(x, gpu)
    y = fp8lin.fp8_linear(xg, c, s, True)
    assert_parity(bits(y), ref, f"gemv K={k} m={m}")
    flat = torch.empty(m * k + 1, dtype=torch.bfloat16, device=gpu)
    xu = flat[1:].view(m, k)
    xu.copy_(xg)
    assert torch.equal(fp8lin.fp8_linear(xu, c, s, True), y)


# ------------------------------------------------------------ split-K GEMM
def splitk_bytes(m, n, k, cus=256):
    """Split-K workspace of the FP8 GEMM plan on a device of `cus` CUs, with
    bm x 256 tiles (bm = 128 for m <= 128, else 256): every tile split when
    the tiles number at most half the CUs, else the tiles of a last round on
    at most half the CUs; min(CUs / tiles, K / 256, 8) K ranges of one
    bm x 256 FP32 partial each."""
    bm = 128 if m <= 128 else 256
    tiles = -(-m // bm) * -(-n // 256)
    split = tiles if 2 * tiles <= cus else tiles % cus if tiles > cus and 2 * (tiles % cus) <= cus else 0
    if split == 0:
        return 0
    s = min(cus // split, k // 256, 8)
    return split * s * bm * 256 * 4 if s > 1 else 0


@pytest.mark.parametrize("m,n,k", [(300, 1040, 1024), (33, 520, 2560), (17, 384, 8704), (600, 7168, 512),
                                   (512, 7168, 5120), (512, 5120, 8704), (1024, 22784, 512)])
def test_engine_splitk_gemm(fp8lin, gpu, oracle, m, n, k):
    """Engine::linear's FP8 GEMM branch (src/engine.cpp:222-224) with few
    output tiles, or a short last round of tiles, splits K over more CUs:
    FP32 partials per K range, added in order by a second launch.  Parity
    with the oracle on the last columns (inside the split tiles in every
    case), and with the unsplit kernel: only the FP32 summation order
    differs, so all but outputs next to a rounding boundary (or near zero,
    where an ulp is tiny) match."""
    F = fp8lin
    rng = np.random.default_rng(m + n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    eng = F.LinearEngine()
    eng.add("w.weight", up(codes, gpu), up(scales, gpu))
    rec = eng._record("w")
    import ctypes
    need = F.lib().fp8lin_engine_linear_workspace_bytes(ctypes.byref(eng.options), ctypes.byref(rec), m)
    assert need == splitk_bytes(m, n, k)
    assert need > 0
    x = rand_bf16(rng, (m, k))
    y, path = eng.linear(up(x, gpu), "w", return_path=True)
    assert path == F.PATH_FP8_GEMM
    cols = (max(0, n - 600), n)
    ref = oracle.linear(x, codes, scales, rows=cols)
    got = bits(y)
    assert_parity(got[:, cols[0]:cols[1]], ref[:, cols[0]:cols[1]], f"split-K {m}x{n}x{k}")
    plain = bits(F.fp8_linear(up(x, gpu), up(codes, gpu), up(scales, gpu), split=False))
    assert_parity(got, plain, f"split-K vs unsplit {m}x{n}x{k}", min_exact=0.99)
    # at most one output in 10^4 (and at least one allowed) beyond 1 ulp
    assert (ulp_distance(got, plain) > 1).sum() <= max(1, got.size // 10000)
    # too small a workspace is an error, not a silent fallback
    if need:
        y2 = torch.empty((m, n), dtype=torch.bfloat16, device=gpu)
        stream = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        rc = F.lib().fp8lin_engine_linear(ctypes.byref(eng.options), ctypes.byref(rec),
                                          ctypes.c_void_p(up(x, gpu).data_ptr()), m, ctypes.c_void_p(y2.data_ptr()),
                                          n, ctypes.c_void_p(ws.data_ptr()), need - 16, None, stream)
        assert rc == F.ERR_WORKSPACE


def test_engine_splitk_graph_replay(fp8lin, gpu, oracle):
    """A captured split-K GEMM (two launches) matches eager on every replay."""
    F = fp8lin
    rng = np.random.default_rng(5)
    m, n, k = 64, 768, 2048
    codes, scales = rand_codes(rng, n, k), (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    eng = F.LinearEngine()
    eng.add("w.weight", up(codes, gpu), up(scales, gpu))
    x = up(rand_bf16(rng, (m, k)), gpu)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        out = eng.linear(x, "w")
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = eng.linear(x, "w")
    for i in range(4):
        if i:
            x.copy_(up(rand_bf16(rng, (m, k)), gpu))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = eng.linear(x, "w")
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"


# ------------------------------------------------------------- benchmark shapes
def test_config1_gemv_seed0(fp8lin, gpu, oracle):
    """Benchmark config 1: M=1, N=K=4096, seed 0, N(0,0.02) weights."""
    codes, scales = fp8lin.gen_weights(4096, 4096, seed=0, tag=1, device=gpu)
    x = fp8lin.gen_activations(1, 4096, seed=0, tag=2, device=gpu)
    y = fp8lin.fp8_linear(x, codes, scales, True)
    ref = oracle.linear(bits(x), codes.cpu().numpy(), scales.cpu().numpy())
    s = assert_parity(bits(y), ref, "config 1")
    assert s["max_ulp"] <= 1


@pytest.mark.parametrize("n,k", [(17408, 5120), (5120, 8704), (7168, 5120)])
@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_decode_shapes(fp8lin, gpu, oracle, n, k, m):
    """Benchmark configs 2 and 3 at one TP rank's shard shapes, all rows."""
    codes, scales = fp8lin.gen_weights(n, k, seed=0, tag=1, device=gpu)
    x = fp8lin.gen_activations(m, k, seed=0, tag=2, device=gpu)
    c_np, s_np = codes.cpu().numpy(), scales.cpu().numpy()
    ref = oracle.linear(bits(x), c_np, s_np)
    assert_parity(bits(fp8lin.fp8_linear(x, codes, scales, True)), ref, f"gemv {m}x{n}x{k}")
    if m >= 2:
        for split in (1, 4):
            y = fp8lin.fp8_tensor_small(x, codes, scales, split)
            assert_parity(bits(y), ref, f"tensor_small {m}x{n}x{k} s{split}")


@pytest.mark.parametrize("m", [512, 4096])
def test_prefill_swiglu_shape(fp8lin, gpu, oracle, m):
    """Benchmark config 4: gate/up N=17408, K=5120, fused SwiGLU; oracle on a
    row sample plus the last rows."""
    n, k = 17408, 5120
    codes, scales = fp8lin.gen_weights(n, k, seed=0, tag=1, device=gpu)
    x = fp8lin.gen_activations(m, k, seed=0, tag=2, device=gpu)
    y = fp8lin.linear_swiglu(x, codes, scales)
    rng = np.random.default_rng(m)
    rows = np.unique(np.concatenate([rng.choice(m, 24, replace=False), [0, m - 1]]))
    xs = bits(x)[rows]
    ref = oracle.swiglu(oracle.linear(xs, codes.cpu().numpy(), scales.cpu().numpy()))
    assert_parity(bits(y)[rows], ref, f"prefill swiglu M={m}", elementwise=False)


def test_ceiling_probes(fp8lin, gpu):
    """The measurement probes run and report: the streaming read touches no
    sink word for ordinary data, and the MFMA probe's shader-clock ticks match
    16 MFMAs x 32 cycles per iteration (register-only, so nothing stalls)."""
    src = torch.arange(1 << 20, dtype=torch.int32, device=gpu)
    sink = torch.zeros(4096, dtype=torch.float32, device=gpu)
    fp8lin.stream_read(src, sink)
    clocks = torch.zeros(2, dtype=torch.int64, device=gpu)
    one = torch.zeros(1, dtype=torch.float32, device=gpu)
    iters = 200
    fp8lin.mfma_ceiling(iters, one, clocks)
    torch.cuda.synchronize()
    assert float(sink.abs().sum()) == 0.0
    assert float(one[0]) == 0.0
    ticks, rt = clocks.cpu().tolist()
    assert rt > 0
    per_mfma = ticks / (iters * 16)
    assert 31.0 <= per_mfma <= 40.0, per_mfma


def test_swiglu_every_gate_value(fp8lin, gpu, oracle):
    """All 65536 BF16 gate values a, with u = 1 (so y = g) and with a spread
    of u: g = bf16(a/(1+exp(-a))) is a function of a's 16 bits, and
    y = bf16(g*u) rounds an exact FP32 product, so agreeing with the oracle on
    this set agrees on every input pair (src/optimized.cu:73)."""
    a = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    rng = np.random.default_rng(7)
    u_rand = rand_bf16(rng, (65536,), 2.0)
    for u in (np.full(65536, 0x3F80, np.uint16), u_rand):
        g = np.concatenate([a, u])[None, :]
        y = bits(fp8lin.fused_swiglu(up(g, gpu)))[0]
        ref = oracle.swiglu(g)[0]
        yf, rf = bf16_to_f32(y), bf16_to_f32(ref)
        both_nan = np.isnan(yf) & np.isnan(rf)
        bad = (y != ref) & ~both_nan
        assert not bad.any(), (f"{int(bad.sum())} of 65536 differ, e.g. a={a[bad][:8]} "
                               f"got={y[bad][:8]} want={ref[bad][:8]}")


# ------------------------------------------------------------------ bias add
def test_engine_bias(fp8lin, gpu, oracle):
    """Engine::linear adds `name.bias` after the product as a BF16 tensor sum
    (src/engine.cpp:240): on every branch the biased output equals torch's
    BF16 `y + b` of the unbiased one, bit for bit; mixed groups add each
    group's own bias; the head candidates see the biased logits."""
    F = fp8lin
    rng = np.random.default_rng(21)
    n, k = 272, 640
    codes, scales = rand_codes(rng, n, k), (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    bias = up(rand_bf16(rng, (n,), 0.5), gpu)
    cases = [(F.LinearOptions(), 1), (F.LinearOptions(), 33), (F.LinearOptions(fp8_tensor_small=True), 4),
             (F.LinearOptions(multi_token_gemv=True), 3), (F.LinearOptions(cublas_prefill=True), 20),
             (F.LinearOptions(), 600)]
    for opt, rows in cases:
        plain, biased = F.LinearEngine(opt), F.LinearEngine(opt)
        for e in (plain, biased):
            e.add("h.weight", up(codes, gpu), up(scales, gpu))
        biased.add("h.bias", bias)
        x = up(rand_bf16(rng, (rows, k)), gpu)
        y0, y1 = plain.linear(x, "h"), biased.linear(x, "h")
        assert torch.equal(y1, y0 + bias), (opt, rows)
        c1 = biased.local_candidates(x, "h", offset=7)
        assert torch.equal(c1, F.vocabulary_candidates(y0 + bias, 7)), (opt, rows)
        y2 = y0.clone()
        F.add_bias(y2, bias)
        assert torch.equal(y2, y1)
    # mixed FP8 / BF16 groups, each with its own bias
    eng = F.LinearEngine()
    w8, s8 = up(codes, gpu), up(scales, gpu)
    wb = up(rand_bf16(rng, (48, k), 0.05), gpu)
    eng.add("g.fp8.weight", w8, s8)
    eng.add("g.bf.weight", wb)
    eng.fuse_weights("g.all", ["g.fp8", "g.bf"])
    assert eng.mixed_projections["g.all"] == ["g.fp8", "g.bf"]
    bb = up(rand_bf16(rng, (48,), 0.5), gpu)
    x = up(rand_bf16(rng, (5, k)), gpu)
    y0 = eng.linear(x, "g.all")
    eng.add("g.fp8.bias", bias)
    eng.add("g.bf.bias", bb)
    y1 = eng.linear(x, "g.all")
    assert torch.equal(y1, y0 + torch.cat([bias, bb]))


def test_engine_workspace_under_capture(fp8lin, gpu, oracle):
    """A captured LinearEngine call keeps its own workspace: larger eager calls
    between replays (on the capture stream and on another) grow and replace
    the engine's per-stream buffers without touching the graph's, so every
    replay still matches eager (the MTP draft graph captures
    Engine::local_candidates, src/speculative.cpp:113-121)."""
    F = fp8lin
    rng = np.random.default_rng(22)
    n, k = 4096, 512
    codes, scales = rand_codes(rng, n, k), (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    eng = F.LinearEngine()
    eng.add("lm_head.weight", up(codes, gpu), up(scales, gpu))
    x = up(rand_bf16(rng, (1, k)), gpu)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        out = eng.local_candidates(x)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = eng.local_candidates(x)
            logits = eng.linear(x, "lm_head")
    for i in range(4):
        x.copy_(up(rand_bf16(rng, (1, k)), gpu))
        big = up(rand_bf16(rng, (600 + 100 * i, k)), gpu)
        with torch.cuda.stream(stream):
            eng.local_candidates(big)
            eng.linear(big, "lm_head")
        eng.local_candidates(big)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = eng.local_candidates(x)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        assert torch.equal(logits, eng.linear(x, "lm_head")), f"replay {i}"


# ------------------------------------- fp8_linear at 2..8 rows on the matrix cores
@pytest.mark.parametrize("m,n,k", [(3, 2056, 384), (8, 2056, 384), (5, 8208, 4096), (4, 8208, 5120),
                                   (2, 2064, 5248), (6, 1040, 8704)])
def test_linear_small_m_rows(fp8lin, gpu, oracle, m, n, k):
    """fp8_linear with 2..8 rows (3..8, or 2 at K > 5120) against more than
    1024 weight rows runs the small-M matrix-core kernel: the row-staged
    form (n = 2056, 2064, 1040: 8 or 9 rows per workgroup, 4 or 5 SwiGLU
    pairs, both tiles ragged; K tails of 384, 5248 and 8704 within the last
    1024-wide stage) or its wide form (n = 8208: 33 rows per CU in three
    tiles, 17 SwiGLU pairs).  Every output
    against the FP64 oracle; fp8_tensor_small bit-equal (the same kernel);
    the fused SwiGLU bit-equal to fused_swiglu(fp8_linear); an unaligned
    view of x runs the multi-row GEMV, at the bar."""
    rng = np.random.default_rng(m * 100003 + n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s, xg = up(codes, gpu), up(scales, gpu), up(x, gpu)
    y = fp8lin.fp8_linear(xg, c, s, True)
    assert_parity(bits(y), ref, f"small-M rows {m}x{n}x{k}")
    assert torch.equal(fp8lin.fp8_tensor_small(xg, c, s, 1), y)
    fused = fp8lin.linear_swiglu(xg, c, s, split=False)
    assert torch.equal(fused, fp8lin.fused_swiglu(y)), "fused != fused_swiglu(fp8_linear)"
    assert torch.equal(fp8lin.linear_swiglu(xg, c, s), fused)
    assert ulp_distance(bits(fused), oracle.swiglu(bits(y))).max() <= 1
    flat = torch.empty(m * k + 1, dtype=torch.bfloat16, device=gpu)
    xu = flat[1:].view(m, k)
    xu.copy_(xg)
    assert_parity(bits(fp8lin.fp8_linear(xu, c, s, True)), ref, f"unaligned x {m}x{n}x{k}")
    assert_parity(bits(fp8lin.linear_swiglu(xu, c, s, split=False)), oracle.swiglu(ref),
                  f"unaligned x swiglu {m}x{n}x{k}", elementwise=False)


@pytest.mark.parametrize("m,n,k", [(8, 8190, 9216), (7, 8190, 9216), (5, 300, 1152), (2, 1154, 2176),
                                   (4, 2050, 8192)])
def test_small_m_row_staged_limits(fp8lin, gpu, oracle, m, n, k):
    """The row-staged small-M form at its K limit and smallest row counts:
    32 rows (16 SwiGLU pairs) per workgroup with K = 9216 (two tiles, the
    72-block scale table of 32 rows, 18 stages of 512 values), one or two
    rows per workgroup with a last stage of 128 values (K = 1152), a last
    stage of 128 of 512 values at an odd pair count (1154 rows, 577 pairs),
    and K a whole number of stages.  Every output of fp8_tensor_small (the
    small-M kernel at any row count) against the FP64 oracle, split 1 and 4
    bit-equal; where fp8_linear takes the same kernel (more than 1024 rows,
    3..8 activation rows or 2 at K > 5120) it gives the same bits; the fused
    SwiGLU bit-equal to fused_swiglu(fp8_linear)."""
    rng = np.random.default_rng(m * 7919 + n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s, xg = up(codes, gpu), up(scales, gpu), up(x, gpu)
    yt = fp8lin.fp8_tensor_small(xg, c, s, 1)
    assert_parity(bits(yt), ref, f"row-staged {m}x{n}x{k}")
    assert torch.equal(fp8lin.fp8_tensor_small(xg, c, s, 4), yt)
    y = fp8lin.fp8_linear(xg, c, s, True)
    assert_parity(bits(y), ref, f"fp8_linear {m}x{n}x{k}")
    if n > 1024 and (m > 2 or k > 5120):
        assert torch.equal(y, yt)
    fused = fp8lin.linear_swiglu(xg, c, s, split=False)
    assert torch.equal(fused, fp8lin.fused_swiglu(y)), "fused != fused_swiglu(fp8_linear)"
    assert ulp_distance(bits(fused), oracle.swiglu(bits(y))).max() <= 1


@pytest.mark.parametrize("m,n,k", [(8, 17408, 5120), (7, 20480, 5120), (5, 8240, 4096), (3, 12000, 4224),
                                   (2, 9000, 2048), (4, 12288, 4096)])
def test_small_m_row_wide(fp8lin, gpu, oracle, m, n, k):
    """The wide row-staged small-M form (33..80 rows per CU, 512-byte
    stages, up to 5 tiles): 68 rows (34 SwiGLU pairs) per workgroup at the
    gate/up shape, the 80-row maximum, 33 rows at K = 4096, a last stage of
    128 values (K = 4224), K outside the row-range kernel's bands (2048), and
    48 rows at K = 4096, which stays on the row-range kernel.  Every output of
    fp8_tensor_small against the FP64 oracle, split 1 and 4 bit-equal;
    fp8_linear the same bits where it takes the small-M path; the fused
    SwiGLU bit-equal to fused_swiglu(fp8_linear); the head candidates of
    one call equal to those of the stored logits."""
    rng = np.random.default_rng(m * 104729 + n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s, xg = up(codes, gpu), up(scales, gpu), up(x, gpu)
    yt = fp8lin.fp8_tensor_small(xg, c, s, 1)
    assert_parity(bits(yt), ref, f"row-wide {m}x{n}x{k}")
    assert torch.equal(fp8lin.fp8_tensor_small(xg, c, s, 4), yt)
    y = fp8lin.fp8_linear(xg, c, s, True)
    assert_parity(bits(y), ref, f"fp8_linear {m}x{n}x{k}")
    if m > 2 or k > 5120:
        assert torch.equal(y, yt)
    fused = fp8lin.linear_swiglu(xg, c, s, split=False)
    assert torch.equal(fused, fp8lin.fused_swiglu(y)), "fused != fused_swiglu(fp8_linear)"
    assert ulp_distance(bits(fused), oracle.swiglu(bits(y))).max() <= 1
    want = fp8lin.vocabulary_candidates(y, 0)
    assert torch.equal(fp8lin.linear_candidates(xg, c, s, 0), want)


@pytest.mark.parametrize("m,n,k", [(16, 16384, 5120), (12, 12288, 4096), (9, 4100, 4224), (16, 8190, 9216),
                                   (11, 1100, 8704), (14, 6000, 640)])
def test_small_m_row_wide_16_rows(fp8lin, gpu, oracle, m, n, k):
    """The wide row-staged form with 16 staged activation rows (fp8_linear at
    9..16 rows): 64 rows per workgroup (4 tiles, the most with 512-byte
    stages; 32 SwiGLU pairs), 48 rows at K = 4096, a last stage of 128 values (K = 4224), 32
    rows at K = 9216 (18 stages, the longest), one tile at K = 8704 and a
    short K.  Every output against the FP64 oracle; the first 9 rows those of
    a 9-row call (the summation depends on K only); the fused SwiGLU
    bit-equal to fused_swiglu(fp8_linear) and within 1 ulp of the oracle
    SwiGLU of the same sums; the head candidates of one call equal to those
    of the stored logits."""
    rng = np.random.default_rng(m * 7919 + n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s, xg = up(codes, gpu), up(scales, gpu), up(x, gpu)
    y = fp8lin.fp8_linear(xg, c, s, True)
    assert_parity(bits(y), ref, f"row-wide 16 {m}x{n}x{k}")
    if m > 9:
        assert torch.equal(fp8lin.fp8_linear(xg[:9].contiguous(), c, s, True), y[:9])
    fused = fp8lin.linear_swiglu(xg, c, s, split=False)
    assert torch.equal(fused, fp8lin.fused_swiglu(y)), "fused != fused_swiglu(fp8_linear)"
    assert ulp_distance(bits(fused), oracle.swiglu(bits(y))).max() <= 1
    want = fp8lin.vocabulary_candidates(y, 0)
    assert torch.equal(fp8lin.linear_candidates(xg, c, s, 0), want)


@pytest.mark.parametrize("m,n,k", [(32, 5120, 8704), (24, 7168, 5120), (17, 2048, 5120), (32, 6144, 4096),
                                   (20, 3100, 9216), (31, 8190, 640), (25, 4100, 4224)])
def test_small_m_row_wide_32_rows(fp8lin, gpu, oracle, m, n, k):
    """The wide row-staged form with 32 staged activation rows (fp8_linear at
    17..32 rows, up to 32 weight rows per CU): two tiles at K = 8704 (18
    stages, the ring at its LDS limit), K = 5120 and K = 4096, one tile at
    K = 5120 and at K = 9216 (the longest), a short K, and a last stage of
    128 values (K = 4224).  Every output against the FP64 oracle; the first
    17 rows those of a 17-row call, and rows 16.. changing none of the first
    16 outputs (each activation tile sums on its own, in an order that
    depends on K only); the fused SwiGLU bit-equal to fused_swiglu(fp8_linear)
    and within 1 ulp of the oracle SwiGLU of the same sums."""
    rng = np.random.default_rng(m * 7907 + n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s, xg = up(codes, gpu), up(scales, gpu), up(x, gpu)
    y = fp8lin.fp8_linear(xg, c, s, True)
    assert_parity(bits(y), ref, f"row-wide 32 {m}x{n}x{k}")
    if m > 17:
        assert torch.equal(fp8lin.fp8_linear(xg[:17].contiguous(), c, s, True), y[:17])
    xz = xg.clone()
    xz[16:] = 0
    assert torch.equal(fp8lin.fp8_linear(xz, c, s, True)[:16], y[:16])
    fused = fp8lin.linear_swiglu(xg, c, s, split=False)
    assert torch.equal(fused, fp8lin.fused_swiglu(y)), "fused != fused_swiglu(fp8_linear)"
    assert ulp_distance(bits(fused), oracle.swiglu(bits(y))).max() <= 1


@pytest.mark.parametrize("m,n,k", [(16, 17408, 5120), (9, 20000, 4224), (32, 17408, 5120), (17, 12288, 5120),
                                   (24, 16000, 4608), (32, 8240, 5120)])
def test_small_m_row_wide_half_stages(fp8lin, gpu, oracle, m, n, k):
    """The wide row-staged form with 256-byte stages (fp8_linear at 9..16
    rows with 5 tiles per workgroup, at 17..32 rows with 3..5, K =
    4224..5120): 80 rows per workgroup at 16 and at 32 staged rows (gate/up),
    a last stage of 128 values (K = 4224), 48 and 64 rows per workgroup, and
    33 rows (in_proj_all: the third tile holds one row).  Every output
    against the FP64 oracle; the first 9 (17) rows those of a 9-row (17-row)
    call; at 17..32 rows, rows 16.. changing none of the first 16 outputs;
    the fused SwiGLU bit-equal to fused_swiglu(fp8_linear) and within 1 ulp
    of the oracle SwiGLU of the same sums."""
    rng = np.random.default_rng(m * 7901 + n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s, xg = up(codes, gpu), up(scales, gpu), up(x, gpu)
    y = fp8lin.fp8_linear(xg, c, s, True)
    assert_parity(bits(y), ref, f"row-wide half stages {m}x{n}x{k}")
    first = 17 if m > 17 else 9 if 9 < m <= 16 else 0
    if first:
        assert torch.equal(fp8lin.fp8_linear(xg[:first].contiguous(), c, s, True), y[:first])
    if m > 16:
        xz = xg.clone()
        xz[16:] = 0
        assert torch.equal(fp8lin.fp8_linear(xz, c, s, True)[:16], y[:16])
    fused = fp8lin.linear_swiglu(xg, c, s, split=False)
    assert torch.equal(fused, fp8lin.fused_swiglu(y)), "fused != fused_swiglu(fp8_linear)"
    assert ulp_distance(bits(fused), oracle.swiglu(bits(y))).max() <= 1


@pytest.mark.parametrize("m,n,k", [(64, 5120, 8704), (48, 7168, 5120), (33, 2048, 5120), (64, 6144, 4096),
                                   (40, 3100, 9216), (57, 4100, 4224), (64, 8190, 640)])
def test_small_m_row_wide_64_rows(fp8lin, gpu, oracle, m, n, k):
    """fp8_linear at 33..64 rows on weights of up to 32 rows per CU: the
    row-staged form with 64 staged activation rows in 256-byte stages (four
    activation tiles) instead of the GEMM: two tiles at K = 8704 (34 stages)
    and at K = 5120 and 4096, one tile at K = 5120 and at K = 9216 (the
    longest), a last stage of 128 values (K = 4224) and a short K.  Every
    output against the FP64 oracle; the first 33 rows those of a 33-row
    call, and rows 16.. changing none of the first 16 outputs; the fused
    SwiGLU bit-equal to fused_swiglu(fp8_linear) and within 1 ulp of the
    oracle SwiGLU of the same sums; no split-K workspace asked for."""
    rng = np.random.default_rng(m * 7883 + n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s, xg = up(codes, gpu), up(scales, gpu), up(x, gpu)
    y = fp8lin.fp8_linear(xg, c, s, True)
    assert_parity(bits(y), ref, f"row-wide 64 {m}x{n}x{k}")
    if m > 33:
        assert torch.equal(fp8lin.fp8_linear(xg[:33].contiguous(), c, s, True), y[:33])
    xz = xg.clone()
    xz[16:] = 0
    assert torch.equal(fp8lin.fp8_linear(xz, c, s, True)[:16], y[:16])
    fused = fp8lin.linear_swiglu(xg, c, s, split=False)
    assert torch.equal(fused, fp8lin.fused_swiglu(y)), "fused != fused_swiglu(fp8_linear)"
    assert torch.equal(fp8lin.linear_swiglu(xg, c, s), fused)
    assert ulp_distance(bits(fused), oracle.swiglu(bits(y))).max() <= 1
    assert fp8lin.lib().fp8lin_linear_workspace_bytes(m, n, k) == 0


def _mid_rows_sweep_cases(count=14, seed=2027):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < count:
        m = int(rng.integers(9, 65))
        n = 2 * int(rng.integers(520, 4200))
        k = 128 * int(rng.integers(1, 41))
        cases.append((m, n, k))
    return cases


@pytest.mark.parametrize("m,n,k", _mid_rows_sweep_cases())
def test_mid_rows_random_sweep(fp8lin, gpu, oracle, m, n, k):
    """Seeded random shapes over fp8_linear's 9..64-row routing (the
    row-staged form with 16, 32 or 64 staged rows in 512- or 256-byte
    stages, the row-range and K-split forms, or the GEMM where none holds
    the rows): every output against the FP64 oracle, and the fused SwiGLU
    bit-equal to fused_swiglu(fp8_linear) on the same weight."""
    rng = np.random.default_rng(m * 131 + n * 7 + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s, xg = up(codes, gpu), up(scales, gpu), up(x, gpu)
    y = fp8lin.fp8_linear(xg, c, s, True, split=False)
    assert_parity(bits(y), ref, f"sweep {m}x{n}x{k}")
    fused = fp8lin.linear_swiglu(xg, c, s, split=False)
    assert torch.equal(fused, fp8lin.fused_swiglu(y)), "fused != fused_swiglu(fp8_linear)"


def _small_rows_sweep_cases(count=14, seed=2029):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < count:
        m = int(rng.integers(2, 9))
        n = 2 * int(rng.integers(520, 10000))
        k = 128 * int(rng.integers(1, 73))
        cases.append((m, n, k))
    return cases


@pytest.mark.parametrize("m,n,k", _small_rows_sweep_cases())
def test_small_rows_random_sweep(fp8lin, gpu, oracle, m, n, k):
    """Seeded random shapes over fp8_linear's 2..8-row routing (the ring or
    general GEMV, the row-staged form with 1..5 tiles, the row-range form):
    every output against the FP64 oracle, the fused SwiGLU bit-equal to
    fused_swiglu(fp8_linear), and fp8_tensor_small (src/fp8_tensor.cu:53-71)
    on the same inputs at the parity bar too."""
    rng = np.random.default_rng(m * 137 + n * 3 + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s, xg = up(codes, gpu), up(scales, gpu), up(x, gpu)
    y = fp8lin.fp8_linear(xg, c, s, True)
    assert_parity(bits(y), ref, f"small sweep {m}x{n}x{k}")
    fused = fp8lin.linear_swiglu(xg, c, s, split=False)
    assert torch.equal(fused, fp8lin.fused_swiglu(y)), "fused != fused_swiglu(fp8_linear)"
    t = fp8lin.fp8_tensor_small(xg, c, s, 1)
    assert_parity(bits(t), ref, f"tensor_small sweep {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(65, 5120, 8704), (96, 7168, 5120), (128, 5120, 5120), (101, 2048, 1024)])
def test_linear_65_128_rows_no_workspace(fp8lin, gpu, oracle, m, n, k):
    """fp8_linear without a workspace at 65..128 rows on weights of up to 32
    rows per CU runs the small-M kernels on the two row halves instead of
    whole GEMM tiles: every output against the FP64 oracle, each half
    bit-equal to a call of its own rows, the fused SwiGLU bit-equal to
    fused_swiglu(fp8_linear); with a workspace the split-K GEMM runs, at
    the bar."""
    rng = np.random.default_rng(m * 101 + n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s, xg = up(codes, gpu), up(scales, gpu), up(x, gpu)
    y = fp8lin.fp8_linear(xg, c, s, True, split=False)
    assert_parity(bits(y), ref, f"65..128 rows {m}x{n}x{k}")
    h = m - m // 2
    assert torch.equal(fp8lin.fp8_linear(xg[:h].contiguous(), c, s, True, split=False), y[:h])
    assert torch.equal(fp8lin.fp8_linear(xg[h:].contiguous(), c, s, True, split=False), y[h:])
    fused = fp8lin.linear_swiglu(xg, c, s, split=False)
    assert torch.equal(fused, fp8lin.fused_swiglu(y)), "fused != fused_swiglu(fp8_linear)"
    assert_parity(bits(fp8lin.fp8_linear(xg, c, s, True)), ref, f"65..128 rows split {m}x{n}x{k}")


# ------------------------------------ fp8_linear at 9..32 rows on the matrix cores
@pytest.mark.parametrize("m,n,k", [(9, 2056, 384), (16, 2056, 384), (12, 8208, 5120), (16, 8208, 4096),
                                   (13, 1040, 8704), (16, 8240, 8704), (17, 8208, 5120), (32, 8208, 4096),
                                   (27, 8240, 3200), (17, 5120, 8704), (32, 7168, 5120), (24, 2056, 384)])
def test_linear_mid_rows(fp8lin, gpu, oracle, m, n, k):
    """fp8_linear with 9..16 rows against more than 1024 weight rows runs the
    small-M matrix-core kernel, whose 16x16 MFMA tile holds every row (the
    wide row-staged form with 16 staged activation rows up to 64 rows per CU
    and K <= 5120, 32 rows per CU up to K = 9216: every shape here but 8240 x
    8704, which takes the row-range form), instead of a mostly-padding
    GEMM tile; 17..32 rows run the wide row-staged form with 32 staged rows
    (up to 32 rows per CU: 7168, 5120, 2056) or the row-range form with two
    activation tiles (8208, 8240).  Each form's summation
    depends on K only: the first 9 rows of a 9..16-row call are those of a
    9-row call, and the second activation tile of a 17..32-row call changes
    none of the first 16 rows' outputs.  Every output against the FP64
    oracle; the fused SwiGLU bit-equal to fused_swiglu(fp8_linear), with or
    without a workspace (none is needed); Engine::linear's FP8 GEMM branch
    asks for no workspace and gives the same bits; an unaligned view of x
    runs the GEMM, at the bar."""
    import ctypes
    F = fp8lin
    rng = np.random.default_rng(m * 100019 + n + k)
    codes = rand_codes(rng, n, k)
    scales = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x = rand_bf16(rng, (m, k))
    ref = oracle.linear(x, codes, scales)
    c, s, xg = up(codes, gpu), up(scales, gpu), up(x, gpu)
    y = F.fp8_linear(xg, c, s)
    assert_parity(bits(y), ref, f"mid rows {m}x{n}x{k}")
    if m > 16:
        # the second activation tile changes no output's summation
        xz = xg.clone()
        xz[16:] = 0
        assert torch.equal(F.fp8_linear(xz, c, s)[:16], y[:16])
    elif m > 9:
        assert torch.equal(F.fp8_linear(xg[:9].contiguous(), c, s), y[:9])
    assert F.lib().fp8lin_linear_swiglu_workspace_bytes(m, n, k) == 0
    fused = F.linear_swiglu(xg, c, s, split=False)
    assert torch.equal(fused, F.fused_swiglu(y)), "fused != fused_swiglu(fp8_linear)"
    assert torch.equal(F.linear_swiglu(xg, c, s), fused)
    assert ulp_distance(bits(fused), oracle.swiglu(bits(y))).max() <= 1
    eng = F.LinearEngine()
    eng.add("w.weight", c, s)
    rec = eng._record("w")
    assert F.lib().fp8lin_engine_linear_workspace_bytes(ctypes.byref(eng.options), ctypes.byref(rec), m) == 0
    ye, path = eng.linear(xg, "w", return_path=True)
    assert path == F.PATH_FP8_GEMM
    assert torch.equal(ye, y)
    flat = torch.empty(m * k + 1, dtype=torch.bfloat16, device=gpu)
    xu = flat[1:].view(m, k)
    xu.copy_(xg)
    assert_parity(bits(F.fp8_linear(xu, c, s)), ref, f"unaligned x {m}x{n}x{k}")
