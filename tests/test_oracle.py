"""Pin the CPU oracle before trusting it (CPU only).

Each oracle function is checked against something it does not share code
with: the reference's known-answer vectors, library routines (torch's
float8_e4m3fn / bfloat16 casts, numpy float64 matmul), published Philox
vectors, closed forms and brute force.  The last group plants plausible
mistakes in copies of the oracle's arithmetic and shows that these checks
catch them.
"""
import math
import os

import numpy as np
import pytest
import torch

from parity import bf16_to_f32, stats, ulp_distance

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def torch_bf16_bits(f32):
    return torch.from_numpy(np.ascontiguousarray(f32, np.float32)).to(torch.bfloat16) \
        .view(torch.int16).numpy().view(np.uint16)


# ---------------------------------------------------------------- decode (A1)
def test_decode_exhaustive_closed_form(oracle):
    """tests/kernel_test.cpp:16-24: ldexp closed form for all 256 codes,
    signed zero, NaN for 0x7f/0xff."""
    t = oracle.decode_table()
    for b in range(256):
        e, m = (b >> 3) & 15, b & 7
        expected = math.ldexp(float(m), -9) if e == 0 else math.ldexp(1 + m / 8, e - 7)
        if b & 128:
            expected = -expected
        if e == 15 and m == 7:
            assert math.isnan(t[b])
        else:
            assert t[b] == expected and (expected != 0 or math.copysign(1, t[b]) == (-1 if b & 128 else 1))


def test_decode_known_answers(oracle):
    """tests/test_format.py:10-11."""
    np.testing.assert_array_equal(oracle.fp8_decode_values([0, 1, 56, 126, 184]),
                                  [0, 2 ** -9, 1, 448, -1])
    assert np.isnan(oracle.fp8_decode_values([127, 255])).all()


def test_decode_matches_torch_and_fixture(oracle):
    t = oracle.decode_table()
    lib_table = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    fixture = np.load(os.path.join(GOLDEN, "decode_table.npy"))
    for ref in (lib_table, fixture):
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(t), nan)
        assert np.array_equal(t[~nan].view(np.uint32), ref[~nan].view(np.uint32))


# ------------------------------------------------------------------ BF16 RNE
def test_bf16_known_answers(oracle):
    """tests/test_format.py:20-23."""
    x = np.array([1., -2., 0., 1 + 2 ** -8, 1 + 3 * 2 ** -8], np.float32)
    np.testing.assert_array_equal(bf16_to_f32(oracle.bf16_rne(x)), [1., -2., 0., 1., 1 + 2 ** -6])


def test_bf16_matches_torch(oracle):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 3.4028235e38, -3.4028235e38, 1e-45, 1.1754942e-38,
                        1.0 + 2 ** -8, 1.0 + 2 ** -7 + 2 ** -8, 65504.0], np.float32)
    vals = np.concatenate([vals[np.isfinite(vals) | np.isinf(vals)], special])
    got = oracle.bf16_rne(vals)
    ref = torch_bf16_bits(vals)
    assert np.array_equal(got, ref)
    nan = oracle.bf16_rne(np.array([np.nan, -np.nan], np.float32))
    assert np.isnan(bf16_to_f32(nan)).all()


# ------------------------------------------------------- E4M3FN RNE encoder
def test_e4m3_encoder_matches_torch(oracle):
    rng = np.random.default_rng(2)
    grid = oracle.decode_table()[:127]
    mids = (grid[:-1] + grid[1:]) / 2                      # exact ties
    vals = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * 40,
        rng.uniform(-470, 470, 50000).astype(np.float32),
        rng.uniform(-0.02, 0.02, 50000).astype(np.float32),
        grid, -grid, mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 1000),
        np.array([448.0, 449.0, 463.99, 464.0, -464.0, 0.0, -0.0, 2 ** -10, 2 ** -9 * 1.5],
                 np.float32)]).astype(np.float32)
    got = oracle.e4m3_from_float(vals)
    ref = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, ref)


# ------------------------------------------------ block quantization (input)
def test_block_quantization_matches_torch_recipe(oracle):
    """tools/make_tiny_fixture.py:56-61 evaluated with torch (fixture)."""
    f = np.load(os.path.join(GOLDEN, "block_quant.npz"))
    w = f["w"]
    n, k = w.shape
    kb = (k + 127) // 128
    codes = np.empty_like(f["codes"])
    for r in range(0, n, 128):
        for c in range(0, k, 128):
            blk = w[r:r + 128, c:c + 128]
            amax = np.float32(np.abs(blk).max())
            scale = np.float32(max(amax, np.float32(1e-12))) / np.float32(448)
            assert scale == f["block_scales"][r // 128, c // 128]
            codes[r:r + 128, c:c + 128] = oracle.e4m3_from_float(blk / scale)
    assert np.array_equal(codes, f["codes"])
    np.testing.assert_array_equal(oracle.expand_block_scales(f["block_scales"], n), f["scales"])
    assert f["scales"].shape == (n, kb)


def test_scale_expansion_equivalence(oracle):
    """tests/test_fp8_import.py:8-18: decode(q) * row-expanded scales equals
    the blockwise dequantization, including a ragged last row block."""
    rng = np.random.default_rng(3)
    for n, k in [(512, 256), (256, 512), (200, 300)]:
        codes = rng.integers(0, 127, (n, k), dtype=np.uint8)
        block = rng.uniform(.01, .1, ((n + 127) // 128, (k + 127) // 128)).astype(np.float32)
        full = oracle.fp8_decode_values(codes) * block.repeat(128, 0)[:n].repeat(128, 1)[:, :k]
        s = oracle.expand_block_scales(block, n)
        got = oracle.fp8_decode_values(codes) * s.repeat(128, 1)[:, :k]
        np.testing.assert_array_equal(got, full)


# ------------------------------------------------------------ Philox + normal
def test_philox_published_vectors(oracle):
    """Random123 known-answer vectors for Philox4x32-10."""
    kat = [
        ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
        ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
        ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
         [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
    ]
    for ctr, key, out in kat:
        assert [int(v) for v in oracle.philox(ctr, key)] == out


def test_normal_statistics(oracle):
    z = oracle.normal(0, 1, 0, 1 << 20).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1) < 5e-3
    # Tail mass against the normal distribution (2 and 3 sigma).
    assert abs((np.abs(z) > 2).mean() - 0.0455) < 2e-3
    assert abs((np.abs(z) > 3).mean() - 0.0027) < 5e-4
    # Kolmogorov-Smirnov distance to the standard normal CDF on the first
    # 2^16 draws: for n = 65536 the 1% critical value is 1.63 / sqrt(n).
    from scipy import stats
    d = stats.kstest(z[:1 << 16], "norm").statistic
    assert d < 1.63 / np.sqrt(1 << 16), d
    # Different tags and seeds give different streams.
    assert not np.array_equal(z[:64], oracle.normal(0, 2, 0, 64))
    assert not np.array_equal(z[:64], oracle.normal(1, 1, 0, 64))


def test_gen_weights_recipe(oracle):
    codes, scales, w = oracle.gen_weights(0, 1, 200, 300, 0.02, want_w=True)
    np.testing.assert_array_equal(w, np.float32(0.02) * oracle.normal(0, 1, 0, 200 * 300).reshape(200, 300))
    for r in range(0, 200, 128):
        for c in range(0, 300, 128):
            blk = w[r:r + 128, c:c + 128]
            s = np.float32(max(np.float32(np.abs(blk).max()), np.float32(1e-12))) / np.float32(448)
            assert (scales[r:r + 128, c // 128] == s).all()
            ref = torch.from_numpy(blk / s).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(codes[r:r + 128, c:c + 128], ref)
    assert not np.isin(codes, [0x7f, 0xff]).any()


# --------------------------------------------------------------- linear (A3-A10)
def numpy_linear(x_bits, codes, scales):
    """Independent evaluation with library routines: torch decode/casts and
    numpy float64 matmul (tests/fp8_tensor_test.cpp:11-22)."""
    k = codes.shape[1]
    dec = torch.from_numpy(codes).view(torch.float8_e4m3fn).float()
    s = torch.from_numpy(scales if scales.ndim == 2 else scales[:, None])
    s = s.repeat_interleave(128, 1)[:, :k] if scales.ndim == 2 else s.expand(-1, k)
    w = (dec * s).to(torch.bfloat16).double().numpy()
    x = bf16_to_f32(x_bits).astype(np.float64)
    return torch_bf16_bits((x @ w.T).astype(np.float32))


def test_linear_fixture(oracle):
    f = np.load(os.path.join(GOLDEN, "linear_case.npz"))
    for m in (1, 2, 3):
        got = oracle.linear(f[f"x{m}"], f["codes"], f["scales"])
        assert np.array_equal(got, f[f"y{m}"])


@pytest.mark.parametrize("m,n,k,blockscale", [
    (1, 19, 17, True), (4, 137, 257, True), (17, 79, 70, False), (8, 64, 5120, True),
    (3, 33, 128, False), (2, 16, 384, True)])
def test_linear_brute_force(oracle, m, n, k, blockscale):
    rng = np.random.default_rng(m * 1000 + n + k)
    codes = rng.integers(0, 256, (n, k), dtype=np.uint8)
    codes[(codes & 0x7f) == 0x7f] = 0
    scales = (rng.random((n, (k + 127) // 128) if blockscale else n) * .01 + .001).astype(np.float32)
    x = torch_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    assert np.array_equal(oracle.linear(x, codes, scales), numpy_linear(x, codes, scales))


def test_linear_row_range_and_bf16w(oracle):
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 126, (40, 256), dtype=np.uint8)
    scales = (rng.random((40, 2)) * .01 + .001).astype(np.float32)
    x = torch_bf16_bits(rng.standard_normal((3, 256)).astype(np.float32))
    full = oracle.linear(x, codes, scales)
    part = oracle.linear(x, codes, scales, rows=(10, 25))
    assert np.array_equal(part[:, 10:25], full[:, 10:25]) and not part[:, :10].any()
    # Decoded-cache path equals the FP8 path (tests/optimized_test.cpp:11-12).
    assert np.array_equal(oracle.linear_bf16w(x, oracle.dequant(codes, scales)), full)


def test_dequant_block_identity(oracle):
    """tests/optimized_test.cpp:78-85: dequant(codes, scales) ==
    bf16(decode(codes, ones) * expanded scales)."""
    rng = np.random.default_rng(6)
    n, k = 137, 257
    codes = rng.integers(0, 126, (n, k), dtype=np.uint8)
    scales = (rng.random((n, 3)) * .01 + .001).astype(np.float32)
    unit = bf16_to_f32(oracle.dequant(codes, np.ones(n, np.float32)))
    expanded = np.repeat(scales, 128, 1)[:, :k]
    ref = torch_bf16_bits(unit * expanded)
    assert np.array_equal(oracle.dequant(codes, scales), ref)


# ----------------------------------------------------------------- SwiGLU (A11)
def test_swiglu_fixture_and_special_values(oracle):
    f = np.load(os.path.join(GOLDEN, "swiglu_case.npz"))
    got = oracle.swiglu(f["gate_up"])
    # torch computes silu as a*sigmoid(a); the reference's a/(1+exp(-a)) may
    # differ in the last FP32 bit, i.e. at most one BF16 ulp after rounding.
    assert ulp_distance(got, f["y"]).max() <= 1
    assert (ulp_distance(got, f["y"]) == 0).mean() > 0.97
    a = np.array([[0.0, -0.0, 20.0, -20.0, 1.0, 1.0, 1.0, 1.0]], np.float32)
    y = bf16_to_f32(oracle.swiglu(torch_bf16_bits(a)))
    assert y[0, 0] == 0 and y[0, 1] == 0 and y[0, 2] == 20.0 and abs(y[0, 3]) < 1e-6


def bf16_rne_f64(v):
    """FP64 values rounded once to BF16 (normal range), as bit patterns."""
    m, e = np.frexp(v)
    r = np.ldexp(np.rint(m * 256.0), e - 8)  # 8 significant bits, ties to even
    return (r.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)


def test_swiglu_against_fp64_exp(oracle):
    """Every normal BF16 gate value a >= -88 with u = 1 (so y = g): the oracle's
    g = bf16(a / (1 + expf(-a))) (src/optimized.cu:73, FP32 expf) against the
    same quotient in FP64 rounded once to BF16.  An FP32 expf and division
    move the quotient by a few FP32 ulp, so the two agree except where the
    FP64 value lies next to a BF16 rounding midpoint, and never by more than
    one ulp.  (Below a = -88.7 expf(-a) overflows and the reference's FP32
    formula returns -0.)  A sign error in the exponent, a dropped "1 +" or
    sigmoid(a) in place of a * sigmoid(a) fail this."""
    a = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    g = np.concatenate([a, np.full(65536, 0x3F80, np.uint16)])[None, :]
    y = oracle.swiglu(g)[0]
    af = bf16_to_f32(a).astype(np.float64)
    keep = np.isfinite(af) & (af >= -88.0) & (np.abs(af) >= 2.0 ** -125)  # g = a/2 stays normal
    af, y = af[keep], y[keep]
    exact = af / (1.0 + np.exp(-af))
    d = ulp_distance(y, bf16_rne_f64(exact))
    assert d.max() <= 1
    assert (d == 0).mean() > 0.999
    # where they differ, the FP64 value is within 2^-8 BF16 ulp of a midpoint
    m, _ = np.frexp(exact[d == 1])
    frac = np.abs(m) * 256.0 - np.floor(np.abs(m) * 256.0)
    assert np.all(np.abs(frac - 0.5) < 2.0 ** -8), frac


# ------------------------------------- decode epilogue and output head (f)
def _torch_rms_reference(r_bits, w_bits, eps, centered):
    """The reference test's own formula (tests/dual_path_test.cpp:13-15) in
    torch float32: r * rsqrt(mean(r^2) + eps), BF16-rounded first when not
    centered, times (w + centered), to BF16."""
    r = torch.from_numpy(bf16_to_f32(r_bits))
    ref = r * torch.rsqrt((r * r).mean(-1, keepdim=True) + eps)
    if not centered:
        ref = ref.to(torch.bfloat16).float()
    w = torch.from_numpy(bf16_to_f32(w_bits))
    return (ref * (w + (1.0 if centered else 0.0))).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("m,d", [(1, 16), (4, 128), (33, 5120)])
@pytest.mark.parametrize("centered", [False, True])
def test_residual_rms_oracle(oracle, m, d, centered):
    """tests/dual_path_test.cpp:8-17: the residual is the BF16 sum bit for bit
    (torch's own float32 add + BF16 cast), and the normalized output matches
    the reference test's torch formula within its allclose(.01, .001)."""
    rng = np.random.default_rng(m * d + centered)
    x = torch_bf16_bits(rng.standard_normal((m, d)).astype(np.float32))
    u = torch_bf16_bits(rng.standard_normal((m, d)).astype(np.float32))
    w = torch_bf16_bits(rng.standard_normal(d).astype(np.float32))
    res, y = oracle.residual_rms(x, u, w, 1e-6, centered)
    want_res = torch_bf16_bits(bf16_to_f32(x) + bf16_to_f32(u))
    assert np.array_equal(res, want_res)
    ref = _torch_rms_reference(res, w, 1e-6, centered)
    assert np.allclose(bf16_to_f32(y), bf16_to_f32(ref), rtol=0.01, atol=0.001)
    assert ulp_distance(y, ref).max() <= 1
    # fused_rms of the sum is the same function (src/optimized.cu:71)
    assert np.array_equal(oracle.rms(res, w, 1e-6, centered), y)


def test_rms_closed_forms(oracle):
    """Constant rows normalize to +-1 (times w + 1 when centered); scaling a
    row by a power of two changes nothing when eps is negligible; the centered
    form with w = 0 equals the uncentered form with w = 1 (both are bf16(v))."""
    d = 256
    c = torch_bf16_bits(np.array([[3.0] * d, [-0.5] * d], np.float32))
    w0 = np.zeros(d, np.uint16)
    y = bf16_to_f32(oracle.rms(c, w0, 1e-6, True))
    assert np.all(y[0] == 1.0) and np.all(y[1] == -1.0)
    rng = np.random.default_rng(3)
    x = torch_bf16_bits(rng.standard_normal((3, d)).astype(np.float32))
    w = torch_bf16_bits(rng.standard_normal(d).astype(np.float32))
    x8 = torch_bf16_bits(bf16_to_f32(x) * 8.0)
    assert np.array_equal(oracle.rms(x, w, 1e-30, True), oracle.rms(x8, w, 1e-30, True))
    one = torch_bf16_bits(np.ones(d, np.float32))
    assert np.array_equal(oracle.rms(x, w0, 1e-6, True), oracle.rms(x, one, 1e-6, False))


@pytest.mark.parametrize("m,n", [(1, 1), (4, 257), (6, 4096), (1, 4097), (4, 124160)])
def test_vocab_candidates_oracle(oracle, m, n):
    """tests/dual_path_test.cpp:19-27: ties across chunks (columns 0 and N-1
    both 8) go to the smaller column, values and columns (+ offset) equal
    numpy's max / first argmax, and the TP merge of a candidate set with a
    shifted copy keeps the smaller id."""
    rng = np.random.default_rng(n)
    lg = torch_bf16_bits(rng.standard_normal((m, n)).astype(np.float32))
    lg[:, 0] = torch_bf16_bits(np.array([8.0], np.float32))[0]
    lg[:, n - 1] = lg[:, 0]
    off = 124160
    cand = oracle.vocab_candidates(lg, off)
    f = bf16_to_f32(lg)
    assert np.array_equal(cand[:, 0], f.max(1).astype(np.float64))
    assert np.array_equal(cand[:, 1], (f.argmax(1) + off).astype(np.float64))
    lower = cand.copy()
    lower[:, 1] -= off
    assert np.array_equal(oracle.merge_candidates(np.stack([cand, lower])), f.argmax(1))


def test_candidates_nonfinite(oracle):
    """tests/dual_path_test.cpp:28-38: an all-NaN or all-inf row is rejected
    (-1); a losing -inf is valid; a NaN anywhere invalidates the row."""
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    for bad in (nan, inf, -inf):
        lg = torch_bf16_bits(np.full((1, 4097), bad, np.float32))
        assert oracle.merge_candidates(oracle.vocab_candidates(lg)[None])[0] == -1
    lg = np.zeros((2, 4097), np.uint16)
    lg[0, 4096] = torch_bf16_bits(np.array([-inf], np.float32))[0]
    lg[1, 4096] = torch_bf16_bits(np.array([nan], np.float32))[0]
    ids = oracle.merge_candidates(oracle.vocab_candidates(lg)[None])
    assert ids[0] == 0 and ids[1] == -1
    # corrupt ids are rejected: negative, fractional, above INT_MAX
    g = np.array([[[1.0, 3.0]], [[0.5, -1.0]]])
    assert oracle.merge_candidates(g)[0] == -1
    g[1, 0, 1] = 2.5
    assert oracle.merge_candidates(g)[0] == -1
    g[1, 0, 1] = 2.0 ** 31
    assert oracle.merge_candidates(g)[0] == -1
    g[1, 0, 1] = 2.0
    assert oracle.merge_candidates(g)[0] == 3


# ------------------------------------------- planted mistakes are caught (CPU)
def _linear_variant(x_bits, codes, scales, mistake):
    k = codes.shape[1]
    dec = torch.from_numpy(codes).view(torch.float8_e4m3fn).float()
    s = torch.from_numpy(np.repeat(scales, 128, 1)[:, :k])
    xd = bf16_to_f32(x_bits).astype(np.float64)
    if mistake == "scale_factored_out":        # BF16 rounding before the scale multiply
        w = (dec.to(torch.bfloat16).float() * s).double().numpy()
    elif mistake == "scale_transposed":        # block index taken from n instead of k
        sc = torch.from_numpy(scales)
        idx = torch.clamp(torch.arange(codes.shape[0]) // 128, max=sc.shape[1] - 1)
        w = (dec * sc[:, idx].T[:, :1]).to(torch.bfloat16).double().numpy()
    elif mistake == "weights_truncated":       # BF16 weights by truncation, not RNE
        prod = (dec * s).numpy()
        w = (prod.view(np.uint32) & 0xffff0000).view(np.float32).astype(np.float64)
    elif mistake == "output_truncated":        # BF16 output by truncation, not RNE
        w = (dec * s).to(torch.bfloat16).double().numpy()
        y = (xd @ w.T).astype(np.float32)
        return (y.view(np.uint32) >> 16).astype(np.uint16)
    return torch_bf16_bits((xd @ w.T).astype(np.float32))


@pytest.mark.parametrize("mistake", ["scale_factored_out", "scale_transposed", "weights_truncated",
                                     "output_truncated"])
def test_planted_mistakes_fail_the_checks(oracle, mistake):
    """The GPU parity gate (max 1 BF16 ulp, and >= 90% of outputs bit-exact
    when the reference rounding point is kept) rejects each planted mistake."""
    codes, scales = oracle.gen_weights(0, 1, 256, 1024, 0.02)
    x = oracle.gen_activations(0, 2, 2, 1024)
    good = oracle.linear(x, codes, scales)
    bad = _linear_variant(x, codes, scales, mistake)
    s = stats(bad, good)
    assert s["max_ulp"] > 1 or s["exact"] < 0.9, s
