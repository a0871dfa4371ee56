"""The reference's own linear-path tests, run through the compiled LibTorch
shim (a100-vision-infer_amd/aten/avi_ops.cpp) that gives the reference's
avi:: operators over the fp8lin C ABI.

Each case restates one block of the reference's C++ tests with the same
shapes, value distributions and tolerances:
  tests/kernel_test.cpp:15-24        (FP8 decode table)
  tests/optimized_test.cpp:6-21,45-93,94-96,105-106
  tests/fp8_tensor_test.cpp:10-49   (FP64 oracle, graph replay)
  tests/dual_path_test.cpp:9-28     (residual RMS, candidates)
torch's seeded CPU generator stands in for the CUDA RNG.  References are
computed in FP32/FP64 on the CPU.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def avi(fp8lin, gpu):
    from fp8lin import aten
    return aten.load()


def randn(g, *shape):
    return torch.randn(*shape, generator=g)


def randint(g, lo, hi, shape):
    return torch.randint(lo, hi, shape, generator=g)


def host_decode(codes, scales):
    """FP32 decode of E4M3FN codes times row-expanded block (or row) scales,
    from the format (tests/fp8_tensor_test.cpp:11-19)."""
    c = codes.cpu().to(torch.int64)
    e, m = (c >> 3) & 15, c & 7
    v = torch.where(e > 0, torch.ldexp(1 + m / 8.0, (e - 7).to(torch.float64)),
                    torch.ldexp(m.to(torch.float64), torch.tensor(-9.0, dtype=torch.float64)))
    v = torch.where((e == 15) & (m == 7), torch.tensor(float("nan"), dtype=torch.float64), v)
    v = torch.where((c & 128) > 0, -v, v)
    s = scales.cpu().to(torch.float64)
    if s.dim() == 1:
        s = s[:, None].expand_as(v)
    else:
        s = s.repeat_interleave(128, 1)[:, :c.size(1)]
    return (v * s).to(torch.float32)


def matmul_ref(x, w):
    """FP64 x @ w^T on the CPU, returned as FP32."""
    return (x.cpu().double() @ w.cpu().double().t()).float()


def close(a, b, rtol, atol):
    return torch.allclose(a.cpu().float(), b.cpu().float(), rtol=rtol, atol=atol)


def test_decode_table(avi, gpu):
    """tests/kernel_test.cpp:15-24."""
    codes = torch.arange(256).to(torch.uint8).reshape(1, 256).to(gpu)
    d = avi.fp8_decode(codes, torch.ones(1, device=gpu)).cpu().float()[0]
    for b in range(256):
        e, m = (b >> 3) & 15, b & 7
        expected = math.ldexp(float(m), -9) if e == 0 else math.ldexp(1 + m / 8, e - 7)
        expected = -expected if b & 128 else expected
        if e == 15 and m == 7:
            assert math.isnan(d[b])
        else:
            assert d[b] == expected and (expected != 0 or math.copysign(1, d[b]) == (-1 if b & 128 else 1))


@pytest.mark.parametrize("m", [1, 2, 4, 6, 8])
@pytest.mark.parametrize("k", [17, 128, 257, 5120])
def test_shared_gemv_fp8_equals_bf16(avi, gpu, m, k):
    """tests/optimized_test.cpp:6-13."""
    g = torch.Generator().manual_seed(17 + m * 1000 + k)
    n = 19
    x = randn(g, m, k).to(torch.bfloat16).to(gpu)
    codes = randint(g, 0, 126, (n, k)).to(torch.uint8).to(gpu)
    scales = (torch.rand(n, (k + 127) // 128, generator=g) * .01 + .001).to(gpu)
    decoded = avi.fp8_decode(codes, scales)
    actual = avi.small_linear_shared(x, codes, scales)
    assert torch.equal(actual, avi.small_linear_shared(x, decoded))
    assert close(actual, matmul_ref(x.float(), decoded.float()).to(torch.bfloat16), .025, .05)


def test_shared_gemv_unaligned(avi, gpu):
    """tests/optimized_test.cpp:15-21."""
    g = torch.Generator().manual_seed(18)
    m, n, k = 2, 19, 132
    x = randn(g, m * k + 1).to(torch.bfloat16).to(gpu).narrow(0, 1, m * k).reshape(m, k)
    codes = randint(g, 0, 126, (n * k + 1,)).to(torch.uint8).to(gpu).narrow(0, 1, n * k).reshape(n, k)
    scales = torch.ones(n, (k + 127) // 128, device=gpu) * .01
    ref = matmul_ref(x.float(), avi.fp8_decode(codes, scales).float()).to(torch.bfloat16)
    assert close(avi.small_linear_shared(x, codes, scales), ref, .025, .05)


@pytest.mark.parametrize("m", [1, 2, 8])
@pytest.mark.parametrize("k", [4, 128, 132, 257, 5120])
def test_packed_gemv(avi, gpu, m, k):
    """tests/optimized_test.cpp:45-51: signed and subnormal codes."""
    g = torch.Generator().manual_seed(19 + m * 1000 + k)
    n = 19
    x = randn(g, m, k).to(torch.bfloat16).to(gpu)
    codes = (randint(g, 0, 127, (n, k)) + 128 * randint(g, 0, 2, (n, k))).to(torch.uint8).to(gpu)
    scales = (torch.rand(n, (k + 127) // 128, generator=g) * .01 + .001).to(gpu)
    ref = matmul_ref(x.float(), avi.fp8_decode(codes, scales).float())
    assert close(avi.fp8_linear(x, codes, scales, True), ref, .025, .05)


def test_unaligned_gemv_fallback(avi, gpu):
    """tests/optimized_test.cpp:53-57."""
    g = torch.Generator().manual_seed(20)
    x = randn(g, 133).to(torch.bfloat16).to(gpu).narrow(0, 1, 132).reshape(1, 132)
    codes = randint(g, 0, 126, (19, 132)).to(torch.uint8).to(gpu)
    scales = torch.ones(19, device=gpu) * .01
    assert torch.equal(avi.fp8_linear(x, codes, scales, True), avi.fp8_linear(x, codes, scales))


@pytest.mark.parametrize("m", [1, 4, 17, 33])
@pytest.mark.parametrize("k", [32, 70])
def test_gemv_wmma_row_scales(avi, gpu, m, k):
    """tests/optimized_test.cpp:66-72."""
    g = torch.Generator().manual_seed(21 + m * 100 + k)
    n = 79
    x = randn(g, m, k).to(torch.bfloat16).to(gpu)
    codes = randint(g, 0, 126, (n, k)).to(torch.uint8).to(gpu)
    scales = (torch.rand(n, generator=g) * .01).to(gpu)
    ref = matmul_ref(x.float(), avi.fp8_decode(codes, scales).float())
    assert close(avi.fp8_linear(x, codes, scales), ref, .025, .05), f"M={m} K={k}"


@pytest.mark.parametrize("m", [1, 4, 17])
def test_block_fp8(avi, gpu, m):
    """tests/optimized_test.cpp:74-84: block dequant equals an independent
    per-column-block expansion; GEMV/WMMA against it."""
    g = torch.Generator().manual_seed(22 + m)
    n, k = 137, 257
    x = randn(g, m, k).to(torch.bfloat16).to(gpu)
    codes = randint(g, 0, 126, (n, k)).to(torch.uint8).to(gpu)
    scales = (torch.rand(n, 3, generator=g) * .01 + .001).to(gpu)
    unit = avi.fp8_decode(codes, torch.ones(n, device=gpu)).float()
    expanded = scales.repeat_interleave(128, 1)[:, :k]
    decoded = (unit * expanded).to(torch.bfloat16)
    assert torch.equal(avi.fp8_decode(codes, scales), decoded)
    assert close(avi.fp8_linear(x, codes, scales), matmul_ref(x.float(), decoded.float()), .025, .05)
    assert torch.equal(decoded.cpu(), host_decode(codes, scales).to(torch.bfloat16))


@pytest.mark.parametrize("m", [1, 17])
def test_mixed_projection_order(avi, gpu, m):
    """tests/optimized_test.cpp:86-93: [FP8 qkv+z] and [BF16 b+a] fused in
    two GEMMs keep the projection order."""
    g = torch.Generator().manual_seed(23 + m)
    x = randn(g, m, 256).to(torch.bfloat16).to(gpu)
    qkv = randint(g, 0, 126, (384, 256)).to(torch.uint8).to(gpu)
    z = randint(g, 0, 126, (128, 256)).to(torch.uint8).to(gpu)
    qs, zs = (torch.rand(384, 2, generator=g) * .01).to(gpu), (torch.rand(128, 2, generator=g) * .01).to(gpu)
    b = randn(g, 4, 256).to(torch.bfloat16).to(gpu)
    a = randn(g, 4, 256).to(torch.bfloat16).to(gpu)
    sep = torch.cat([avi.fp8_linear(x, qkv, qs).float(), avi.fp8_linear(x, z, zs).float(),
                     matmul_ref(x.float(), b.float()).to(gpu), matmul_ref(x.float(), a.float()).to(gpu)], 1)
    grouped = torch.cat([avi.fp8_linear(x, torch.cat([qkv, z]), torch.cat([qs, zs])).float(),
                         matmul_ref(x.float(), torch.cat([b, a]).float()).to(gpu)], 1)
    assert close(sep, grouped, .025, .05)


def test_rms_and_swiglu(avi, gpu):
    """tests/optimized_test.cpp:94-96 and :105-106."""
    g = torch.Generator().manual_seed(24)
    x, w = randn(g, 3, 512).to(torch.bfloat16), randn(g, 512).to(torch.bfloat16)
    f = x.float()
    expected = (f * torch.rsqrt((f * f).mean(-1, keepdim=True) + 1e-6) * (1 + w.float())).to(torch.bfloat16)
    assert close(avi.fused_rms(x.to(gpu), w.to(gpu), 1e-6, True), expected, .02, .02)
    gu = randn(g, 4, 128).to(torch.bfloat16)
    sg = torch.nn.functional.silu(gu[:, :64].float()) * gu[:, 64:].float()
    assert close(avi.fused_swiglu(gu.to(gpu)), sg, .02, .02)


def test_rope(avi, fp8lin, gpu):
    """tests/optimized_test.cpp:139-141 (zero positions give x back), and
    avi::fused_rope equals the library's rotary embedding bit for bit."""
    g = torch.Generator().manual_seed(141)
    x = randn(g, 3, 2, 64).to(torch.bfloat16).to(gpu)
    zero = torch.zeros((3, 3), dtype=torch.int64, device=gpu)
    assert torch.equal(avi.fused_rope(x, zero, 32, 10000., 4, 4), x)
    pos = torch.randint(0, 4096, (3, 3), generator=g).to(gpu)
    assert torch.equal(avi.fused_rope(x, pos, 32, 10000., 4, 4).view(torch.int16),
                       fp8lin.fused_rope(x, pos, 32, 10000., 4, 4).view(torch.int16))


def fp64_w8a16(x, codes, scales):
    """tests/fp8_tensor_test.cpp:10-19: CPU decode with the BF16 rounding of
    W8A16, FP64 product, rounded to BF16."""
    w = host_decode(codes, scales).to(torch.bfloat16).double()
    return (x.cpu().double() @ w.t()).to(torch.bfloat16).float()


@pytest.mark.parametrize("m", range(2, 9))
@pytest.mark.parametrize("k", [128, 384, 5120])
@pytest.mark.parametrize("n", [17, 80, 144])
def test_tensor_small_fp64_oracle(avi, gpu, m, k, n):
    """tests/fp8_tensor_test.cpp:25-35, both splits and the TileLang entry."""
    g = torch.Generator().manual_seed(915 + m * 10000 + k * 10 + n)
    x = (randn(g, m, k) * .1).to(torch.bfloat16).to(gpu)
    codes = randint(g, 0, 256, (n, k))
    codes[(codes == 127) | (codes == 255)] = 0
    codes = codes.to(torch.uint8).to(gpu)
    scales = (torch.rand(n, k // 128, generator=g) * .001 + .0001).to(gpu)
    expected = fp64_w8a16(x, codes, scales)
    for split in (1, 4):
        out = avi.fp8_tensor_small(x, codes, scales, split)
        assert torch.isfinite(out.float()).all() and close(out, expected, .01, .001)
        if n % 16 == 0:
            assert torch.equal(avi.tilelang_fp8_small(x, codes, scales, split), out)


def test_tensor_small_unaligned_views(avi, gpu):
    """Any contiguous x and codes (src/fp8_tensor.cu:54-59), here views at an
    odd element offset (the pattern of tests/optimized_test.cpp:15-21): the
    operator returns the FP64-oracle result instead of throwing."""
    g = torch.Generator().manual_seed(917)
    m, n, k = 4, 19, 384
    x = (randn(g, m * k + 1) * .1).to(torch.bfloat16).to(gpu).narrow(0, 1, m * k).reshape(m, k)
    codes = randint(g, 0, 126, (n * k + 1,)).to(torch.uint8).to(gpu).narrow(0, 1, n * k).reshape(n, k)
    scales = (torch.rand(n, k // 128, generator=g) * .001 + .0001).to(gpu)
    expected = fp64_w8a16(x, codes, scales)
    for split in (1, 4):
        out = avi.fp8_tensor_small(x, codes, scales, split)
        assert torch.isfinite(out.float()).all() and close(out, expected, .01, .001)


def test_tensor_small_graph_replay(avi, gpu):
    """tests/fp8_tensor_test.cpp:37-49."""
    g = torch.Generator().manual_seed(916)
    x = (randn(g, 4, 384) * .1).to(torch.bfloat16).to(gpu)
    codes = torch.full((144, 384), 24, dtype=torch.uint8, device=gpu)
    scales = (torch.rand(144, 3, generator=g) * .1).to(gpu)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        out = avi.fp8_tensor_small(x, codes, scales, 4)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = avi.fp8_tensor_small(x, codes, scales, 4)
    for i in range(3):
        if i:
            x.add_(.015625)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert close(out, fp64_w8a16(x, codes, scales), .01, .001), f"replay {i}"


@pytest.mark.parametrize("m", [1, 4, 33])
@pytest.mark.parametrize("d", [16, 128, 5120])
@pytest.mark.parametrize("centered", [False, True])
def test_residual_rms(avi, gpu, m, d, centered):
    """tests/dual_path_test.cpp:9-17."""
    g = torch.Generator().manual_seed(104 + m + d)
    x = randn(g, m, d).to(torch.bfloat16).to(gpu)
    u = randn(g, m, d).to(torch.bfloat16).to(gpu)
    w = randn(g, d).to(torch.bfloat16).to(gpu)
    res, out = avi.residual_rms(x, u, w, 1e-6, centered)
    s = x + u
    assert torch.equal(res, s)
    ref = s.float()
    ref = ref * torch.rsqrt((ref * ref).mean(-1, keepdim=True) + 1e-6)
    if not centered:
        ref = ref.to(torch.bfloat16).float()
    ref = (ref * (w.float() + (1.0 if centered else 0.0))).to(torch.bfloat16)
    assert close(out, ref, .01, .001)
    assert torch.equal(out, avi.fused_rms(s, w, 1e-6, centered))


@pytest.mark.parametrize("m", [1, 4, 6])
@pytest.mark.parametrize("n", [1, 257, 4096, 4097, 124160])
def test_vocabulary_candidates(avi, gpu, m, n):
    """tests/dual_path_test.cpp:19-28."""
    g = torch.Generator().manual_seed(200 + m + n)
    logits = randn(g, m, n).to(torch.bfloat16)
    logits[:, 0] = 8
    logits[:, n - 1] = 8
    logits = logits.to(gpu)
    cand = avi.vocabulary_candidates(logits, 124160)
    top = logits.float().max(-1)
    assert torch.equal(cand[:, 0], top.values.double())
    assert torch.equal(cand[:, 1], (top.indices + 124160).double())
    lower = cand.clone()
    lower[:, 1] -= 124160
    assert torch.equal(avi.merge_candidates(torch.stack([cand, lower]).contiguous()), top.indices)


def test_shim_matches_python_ops(avi, fp8lin, gpu):
    """The shim and the Python host mirror call the same C ABI: identical bits."""
    codes, scales = fp8lin.gen_weights(1040, 5120, seed=3, tag=1, device=gpu)
    for m in (1, 4, 300):
        x = fp8lin.gen_activations(m, 5120, seed=3, tag=2, device=gpu)
        assert torch.equal(avi.fp8_linear(x, codes, scales, True), fp8lin.fp8_linear(x, codes, scales, True))
    x = fp8lin.gen_activations(4, 5120, seed=3, tag=2, device=gpu)
    assert torch.equal(avi.fp8_tensor_small(x, codes, scales, 4), fp8lin.fp8_tensor_small(x, codes, scales, 4))


def test_shim_rejects_like_reference(avi, gpu):
    """TORCH_CHECK messages of src/optimized.cu:62-65 and src/fp8_tensor.cu:54."""
    x = torch.zeros(2, 256, dtype=torch.bfloat16, device=gpu)
    codes = torch.zeros(16, 256, dtype=torch.uint8, device=gpu)
    with pytest.raises(RuntimeError, match="Invalid FP8 scales"):
        avi.fp8_linear(x, codes, torch.ones(16, 3, device=gpu))
    with pytest.raises(RuntimeError, match="Invalid Ampere FP8 W8A16 geometry/dtype"):
        avi.fp8_tensor_small(x, codes, torch.ones(16, 2, device=gpu), 2)
    with pytest.raises(RuntimeError, match="Invalid TileLang FP8 W8A16 inputs"):
        avi.tilelang_fp8_small(x, codes[:15].contiguous(), torch.ones(15, 2, device=gpu), 1)


def _bits(t):
    import numpy as np
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("m,n,k", [(512, 7168, 5120), (512, 5120, 8704), (64, 17408, 5120)])
def test_shim_fp8_linear_split_k(avi, fp8lin, gpu, oracle, m, n, k):
    """avi::fp8_linear on the prefill projections whose GEMM tiles leave CUs
    idle (the QKV-gate and down projections at a 512-row chunk, the gate/up
    rows at a 64-row chunk tail; down at 64 rows runs the small-M kernel and
    needs none) splits K through its own workspace, as the engine
    branch does (src/engine.cpp:222-224): at the parity bar against the FP64
    oracle on the last 600 columns, equal to the Python mirror's call bit for
    bit, and within the split-order bar of the unsplit call everywhere."""
    from parity import assert_parity, ulp_distance
    assert fp8lin.lib().fp8lin_linear_workspace_bytes(m, n, k) > 0
    codes, scales = fp8lin.gen_weights(n, k, seed=0, tag=31, device=gpu)
    x = fp8lin.gen_activations(m, k, seed=0, tag=32, device=gpu)
    y = avi.fp8_linear(x, codes, scales, True)
    assert torch.equal(y, fp8lin.fp8_linear(x, codes, scales, True))
    got = _bits(y)
    cols = (n - 600, n)
    ref = oracle.linear(_bits(x), codes.cpu().numpy(), scales.cpu().numpy(), rows=cols)
    assert_parity(got[:, cols[0]:], ref[:, cols[0]:], f"shim split-K {m}x{n}x{k}")
    plain = _bits(fp8lin.fp8_linear(x, codes, scales, True, split=False))
    assert_parity(got, plain, f"shim split-K vs unsplit {m}x{n}x{k}", min_exact=0.99)
    assert (ulp_distance(got, plain) > 1).sum() <= max(1, got.size // 10000)


def test_shim_fp8_linear_split_k_graph_replay(avi, fp8lin, gpu):
    """One avi::fp8_linear call with split K, captured in a HIP graph (its
    workspace comes from the capture's private pool) and replayed with
    updated activations, eager work and synchronisations in between: every
    replay equals the eager call on the same input."""
    m, n, k = 512, 5120, 8704
    codes, scales = fp8lin.gen_weights(n, k, seed=0, tag=33, device=gpu)
    x = fp8lin.gen_activations(m, k, seed=0, tag=34, device=gpu)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        out = avi.fp8_linear(x, codes, scales, True)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = avi.fp8_linear(x, codes, scales, True)
    for i in range(3):
        if i:
            x.copy_(fp8lin.gen_activations(m, k, seed=i, tag=34, device=gpu))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, avi.fp8_linear(x, codes, scales, True)), f"replay {i}"
