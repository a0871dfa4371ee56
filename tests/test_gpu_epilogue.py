"""GPU parity of the decode epilogue and the output head: fused residual add +
RMSNorm, RMSNorm, vocabulary candidates, their cross-rank merge and the head
projection followed by its candidates.

Cases follow the reference's own test (tests/dual_path_test.cpp:7-48) with
numpy's seeded RNG in place of the CUDA RNG.  Residuals, candidates and
merged ids are integer/selection results and must be bit-identical to the
oracle; the normalised output keeps the BF16 parity bar (FP32 block sum here,
FP64 sum in the oracle).
"""
import numpy as np
import pytest
import torch

from parity import assert_parity, bf16_to_f32

pytestmark = pytest.mark.gpu


def up(a, dev):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if a.dtype == np.uint16:
        t = t.view(torch.bfloat16)
    return t.to(dev)


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def rand_bf16(rng, shape, scale=1.0):
    f = (rng.standard_normal(shape) * scale).astype(np.float32)
    return torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bf16_of(values):
    return torch.tensor(values, dtype=torch.float32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def misaligned(t):
    """A contiguous copy of t whose data pointer is 2 bytes past a 16-byte
    boundary (forces the scalar-load kernels)."""
    flat = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    v = flat[1:].view(t.shape)
    v.copy_(t)
    assert v.data_ptr() % 16 != 0
    return v


# ------------------------------------------------------------------ RMSNorm
@pytest.mark.parametrize("m", [1, 4, 33, 512])
@pytest.mark.parametrize("d", [16, 128, 5120])
@pytest.mark.parametrize("centered", [False, True])
def test_residual_rms_reference_grid(fp8lin, gpu, oracle, m, d, centered):
    """tests/dual_path_test.cpp:9-17: residual bit-exact, output at the parity
    bar, and identical to fused_rms of the stored residual."""
    rng = np.random.default_rng(104 + m * 7 + d + centered)
    x, u, w = rand_bf16(rng, (m, d)), rand_bf16(rng, (m, d)), rand_bf16(rng, (d,))
    xt, ut, wt = up(x, gpu), up(u, gpu), up(w, gpu)
    res, y = fp8lin.residual_rms(xt, ut, wt, 1e-6, centered)
    ref_res, ref_y = oracle.residual_rms(x, u, w, 1e-6, centered)
    assert np.array_equal(bits(res), ref_res)
    assert np.array_equal(bits(res), bits(xt + ut))
    assert_parity(bits(y), ref_y, f"residual_rms {m}x{d} c{centered}", min_exact=0.95)
    assert torch.equal(y, fp8lin.fused_rms(res, wt, 1e-6, centered))


@pytest.mark.parametrize("m,d", [(3, 1000), (2, 33), (1, 7168), (5, 16384), (2, 7), (2, 20480), (1, 24584)])
@pytest.mark.parametrize("centered", [False, True])
def test_rms_ragged_and_misaligned(fp8lin, gpu, oracle, m, d, centered):
    """Widths off the 8-element vector, and 2-byte-aligned buffers: the scalar
    kernel gives the same bits as the vector kernel."""
    rng = np.random.default_rng(m * 31 + d)
    x, u, w = rand_bf16(rng, (m, d), 3.0), rand_bf16(rng, (m, d)), rand_bf16(rng, (d,))
    xt, ut, wt = up(x, gpu), up(u, gpu), up(w, gpu)
    y = fp8lin.fused_rms(xt, wt, 1e-5, centered)
    assert_parity(bits(y), oracle.rms(x, w, 1e-5, centered), f"rms {m}x{d}", min_exact=0.95)
    res, y2 = fp8lin.residual_rms(xt, ut, wt, 1e-5, centered)
    assert np.array_equal(bits(res), oracle.residual_rms(x, u, w, 1e-5, centered)[0])
    res_m, y2_m = fp8lin.residual_rms(misaligned(xt), misaligned(ut), misaligned(wt), 1e-5, centered)
    assert torch.equal(res_m, res) and torch.equal(y2_m, y2)
    assert torch.equal(fp8lin.fused_rms(misaligned(xt), misaligned(wt), 1e-5, centered), y)


def test_rms_3d_input(fp8lin, gpu, oracle):
    """fused_rms normalises the last dimension of any shape (src/optimized.cu:72)."""
    rng = np.random.default_rng(5)
    x, w = rand_bf16(rng, (2, 3, 256)), rand_bf16(rng, (256,))
    y = fp8lin.fused_rms(up(x, gpu), up(w, gpu), 1e-6, True)
    assert y.shape == (2, 3, 256)
    assert_parity(bits(y).reshape(6, 256), oracle.rms(x.reshape(6, 256), w, 1e-6, True), "rms 3d",
                  min_exact=0.95)


def test_residual_rms_rejects(fp8lin, gpu):
    x = torch.zeros((2, 64), dtype=torch.bfloat16, device=gpu)
    w = torch.zeros(64, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(fp8lin.Fp8linError):
        fp8lin.residual_rms(x, x[:, :32].contiguous(), w, 1e-6)
    with pytest.raises(fp8lin.Fp8linError):
        fp8lin.residual_rms(x, x, w, 0.0)
    with pytest.raises(fp8lin.Fp8linError):
        fp8lin.residual_rms(x[0], x[0], w, 1e-6)   # dim() >= 2


@pytest.mark.parametrize("ranks", [1, 2, 4, 8])
@pytest.mark.parametrize("m,d", [(1, 5120), (4, 5120), (33, 128), (3, 1000)])
def test_reduce_residual_rms(fp8lin, gpu, oracle, ranks, m, d):
    """Row-parallel reduce folded into residual_rms: the update is bf16 of the
    FP32 sum of the rank partials in rank order (for 2 ranks the reference's
    BF16 all-reduce, tests/tp_reduce_test.cpp:25-32), then the residual is
    bit-exact against the oracle and y equals fused_rms of it."""
    rng = np.random.default_rng(ranks * 100 + m + d)
    x, w = rand_bf16(rng, (m, d)), rand_bf16(rng, (d,))
    parts = np.stack([rand_bf16(rng, (m, d), 0.5) for _ in range(ranks)])
    acc = bf16_to_f32(parts[0]).astype(np.float32)
    for r in range(1, ranks):
        acc = (acc + bf16_to_f32(parts[r])).astype(np.float32)
    update = torch.from_numpy(acc).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    xt, pt, wt = up(x, gpu), up(parts, gpu), up(w, gpu)
    res, y = fp8lin.reduce_residual_rms(xt, pt, wt, 1e-6, True)
    ref_res, ref_y = oracle.residual_rms(x, update, w, 1e-6, True)
    assert np.array_equal(bits(res), ref_res)
    assert_parity(bits(y), ref_y, f"reduce+rms r={ranks} {m}x{d}", min_exact=0.95)
    assert torch.equal(y, fp8lin.fused_rms(res, wt, 1e-6, True))
    if ranks == 2:
        ref2 = (pt[0].float() + pt[1].float()).to(torch.bfloat16)
        assert torch.equal(fp8lin.residual_rms(xt, ref2, wt, 1e-6, True)[0], res)
    # the scalar kernel on 2-byte-aligned buffers gives the same bits
    res_m, y_m = fp8lin.reduce_residual_rms(misaligned(xt), misaligned(pt), misaligned(wt), 1e-6, True)
    assert torch.equal(res_m, res) and torch.equal(y_m, y)


# ------------------------------------------------------ vocabulary candidates
@pytest.mark.parametrize("m", [1, 4, 6])
@pytest.mark.parametrize("n", [1, 257, 4096, 4097, 124160])
def test_vocab_candidates_reference_grid(fp8lin, gpu, oracle, m, n):
    """tests/dual_path_test.cpp:19-28: ties across chunks at columns 0 and
    N-1, offset 124160, and the merge with a copy shifted down by it."""
    rng = np.random.default_rng(m * 1000 + n)
    logits = rand_bf16(rng, (m, n))
    logits[:, 0] = bf16_of([8.0])[0]
    logits[:, n - 1] = bf16_of([8.0])[0]
    lt = up(logits, gpu)
    cand = fp8lin.vocabulary_candidates(lt, 124160)
    ref = oracle.vocab_candidates(logits, 124160)
    assert np.array_equal(cand.cpu().numpy(), ref)
    top = lt.float().max(-1)
    assert torch.equal(cand[:, 0], top.values.double())
    assert torch.equal(cand[:, 1], (top.indices + 124160).double())
    lower = cand.clone()
    lower[:, 1] -= 124160
    ids = fp8lin.merge_candidates(torch.stack([cand, lower]).contiguous())
    assert torch.equal(ids, top.indices)
    # 2-byte-aligned rows take the scalar-load kernel: same result
    assert torch.equal(fp8lin.vocabulary_candidates(misaligned(lt), 124160), cand)


@pytest.mark.parametrize("invalid", [float("nan"), float("inf"), float("-inf")])
def test_nonfinite_vocabulary_rejected(fp8lin, gpu, oracle, invalid):
    """tests/dual_path_test.cpp:29-33."""
    logits = torch.full((1, 4097), invalid, device=gpu).to(torch.bfloat16)
    cand = fp8lin.vocabulary_candidates(logits)
    assert np.array_equal(cand.cpu().numpy(), oracle.vocab_candidates(bits(logits)), equal_nan=True)
    assert fp8lin.merge_candidates(cand.unsqueeze(0).contiguous()).item() == -1


def test_nan_invalidates_losing_neg_inf_does_not(fp8lin, gpu):
    """tests/dual_path_test.cpp:34-38."""
    logits = torch.zeros((2, 4097), device=gpu).to(torch.bfloat16)
    logits[0, 4096] = float("-inf")
    logits[1, 4096] = float("nan")
    ids = fp8lin.merge_candidates(fp8lin.vocabulary_candidates(logits).unsqueeze(0).contiguous()).cpu()
    assert ids.tolist() == [0, -1]


def test_merge_candidates_vs_oracle(fp8lin, gpu, oracle):
    """Random candidates over 1..8 ranks with value ties across ranks and
    corrupt entries (NaN/inf values, negative, fractional, > INT_MAX ids)."""
    rng = np.random.default_rng(77)
    for ranks in range(1, 9):
        rows = 300
        g = np.empty((ranks, rows, 2))
        g[..., 0] = rng.integers(-4, 4, (ranks, rows)) * 0.5
        g[..., 1] = rng.integers(0, 1 << 20, (ranks, rows))
        bad = rng.random((ranks, rows)) < 0.02
        kinds = rng.integers(0, 6, (ranks, rows))
        g[..., 0] = np.where(bad & (kinds == 0), np.nan, g[..., 0])
        g[..., 0] = np.where(bad & (kinds == 1), np.inf, g[..., 0])
        g[..., 1] = np.where(bad & (kinds == 2), -1.0, g[..., 1])
        g[..., 1] = np.where(bad & (kinds == 3), 2.5, g[..., 1])
        g[..., 1] = np.where(bad & (kinds == 4), 2.0 ** 31, g[..., 1])
        g[..., 1] = np.where(bad & (kinds == 5), np.nan, g[..., 1])
        got = fp8lin.merge_candidates(up(g, gpu)).cpu().numpy()
        assert np.array_equal(got, oracle.merge_candidates(g)), f"ranks={ranks}"


def test_epilogue_graph_replay(fp8lin, gpu, oracle):
    """tests/dual_path_test.cpp:39-47: residual RMS -> candidates -> merge
    captured once, replayed after the input changes."""
    rng = np.random.default_rng(9)
    x = up(rand_bf16(rng, (4, 128)), gpu)
    u = up(rand_bf16(rng, (4, 128)), gpu)
    w = torch.zeros(128, dtype=torch.bfloat16, device=gpu)

    def invoke():
        y = fp8lin.residual_rms(x, u, w, 1e-6)[1]
        return fp8lin.merge_candidates(fp8lin.vocabulary_candidates(y).unsqueeze(0).contiguous())

    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        out = invoke()
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = invoke()
    for i in range(3):
        if i:
            x[:, 37 + i] = 100.0
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        expected = fp8lin.fused_rms(x + u, w, 1e-6, True).argmax(-1)
        assert torch.equal(out, expected), f"replay {i}"


# ----------------------------------------------- head projection + candidates
def _head(fp8lin, gpu, m, n, k, seed):
    codes, scales = fp8lin.gen_weights(n, k, seed=seed, tag=1, device=gpu)
    x = fp8lin.gen_activations(m, k, seed=seed, tag=2, device=gpu)
    return x, codes, scales


@pytest.mark.parametrize("m", [1, 2, 3, 4, 8, 9, 16, 24, 64])
@pytest.mark.parametrize("n,k", [(1000, 256), (4097, 5120), (31040, 4096), (777, 10240), (300, 6144)])
def test_linear_candidates_equals_unfused(fp8lin, gpu, oracle, m, n, k):
    """The head in one call (src/speculative.cpp:25-27) is bit-identical to
    vocabulary_candidates(fp8_linear(x, W), offset) on the GEMV paths (128-bit
    and byte loads), the small-M row-range kernel's candidate form (9..32
    rows against 31040 rows) and the M > 8 GEMM path."""
    x, codes, scales = _head(fp8lin, gpu, m, n, k, seed=m + n)
    offset = 124160
    want = fp8lin.vocabulary_candidates(fp8lin.fp8_linear(x, codes, scales, True), offset)
    got = fp8lin.linear_candidates(x, codes, scales, offset)
    assert torch.equal(got, want), f"{m}x{n}x{k}"
    if m <= 8:
        got_b = fp8lin.linear_candidates(misaligned(x), codes, scales, offset)
        assert torch.equal(got_b, want), f"byte loads {m}x{n}x{k}"


def test_linear_candidates_vs_oracle(fp8lin, gpu, oracle):
    """Against the oracle's logits: the chosen id's logit is the oracle's row
    maximum to within the GEMV's 1-ulp bar, and the value is that logit."""
    m, n, k = 4, 4097, 5120
    x, codes, scales = _head(fp8lin, gpu, m, n, k, seed=3)
    logits = oracle.linear(bits(x), codes.cpu().numpy(), scales.cpu().numpy())
    got = fp8lin.linear_candidates(x, codes, scales, 0).cpu().numpy()
    lf = bf16_to_f32(logits).astype(np.float64)
    for r in range(m):
        i = int(got[r, 1])
        assert abs(got[r, 0] - lf[r, i]) <= abs(lf[r, i]) * 2 ** -7
        assert lf[r].max() - lf[r, i] <= abs(lf[r].max()) * 2 ** -7


@pytest.mark.parametrize("m", [2, 3])
def test_linear_candidates_ties_and_nan(fp8lin, gpu, oracle, m):
    """Equal weight rows give exactly tied logits: the smallest row id wins,
    across row groups and across activation rows; a NaN scale makes its row
    +inf, which the merge rejects.  M = 2 takes the GEMV's candidate
    epilogue (ties across workgroups), M = 3 the two-stage kernels."""
    n, k = 1030, 512
    rng = np.random.default_rng(12)
    codes_np = (rng.integers(0, 127, (n, k)) | (rng.integers(0, 2, (n, k)) << 7)).astype(np.uint8)
    codes_np[[5, 6, 700, 1029]] = codes_np[900]
    scales_np = (rng.random((n, k // 128)) * 0.01 + 0.001).astype(np.float32)
    scales_np[[5, 6, 700, 1029]] = scales_np[900] = 1.0
    x_np = rand_bf16(rng, (m, k))
    x_np[1] = x_np[0] ^ 0x8000          # one of rows 0 and 1 sees the tied rows as its maximum
    x = up(x_np, gpu)
    codes, scales = up(codes_np, gpu), up(scales_np, gpu)
    want = fp8lin.vocabulary_candidates(fp8lin.fp8_linear(x, codes, scales), 0)
    got = fp8lin.linear_candidates(x, codes, scales, 0)
    assert torch.equal(got, want)
    assert 5 in got[:2, 1].long().tolist()
    logits = oracle.linear(bits(x), codes_np, scales_np)
    assert np.array_equal(got.cpu().numpy(), oracle.vocab_candidates(logits, 0))
    scales_np[17, 0] = np.nan
    got = fp8lin.linear_candidates(x, codes, up(scales_np, gpu), 0)
    assert torch.isinf(got[:, 0]).all()
    assert (fp8lin.merge_candidates(got.unsqueeze(0).contiguous()) == -1).all()


@pytest.mark.parametrize("m", [3, 8, 16, 17, 32])
def test_small_m_candidates_ties_and_nan(fp8lin, gpu, oracle, m):
    """3..32 rows against a wide head (8208 rows: the small-M row-range
    kernel, 33 rows per workgroup in pieces of 11) take that kernel's candidate
    form: per workgroup and activation row one pair, then one finishing
    workgroup per row.
    Equal weight rows in different workgroups give tied logits and the
    smallest row id wins; the result equals vocabulary_candidates of
    fp8_linear and the oracle's candidates; a NaN scale makes every row's
    candidate +inf.  Engine::local_candidates on the tensor-small branch
    (3 and 8 rows) takes the same candidate form."""
    n, k = 8208, 4096
    rng = np.random.default_rng(40 + m)
    codes_np = (rng.integers(0, 127, (n, k)) | (rng.integers(0, 2, (n, k)) << 7)).astype(np.uint8)
    tied = [7, 3300, 6001, 8207]
    codes_np[tied] = codes_np[4500]
    scales_np = (rng.random((n, k // 128)) * 0.01 + 0.001).astype(np.float32)
    scales_np[tied] = scales_np[4500] = 1.0
    x_np = rand_bf16(rng, (m, k))
    x_np[1] = x_np[0] ^ 0x8000          # one of rows 0 and 1 sees the tied rows as its maximum
    x = up(x_np, gpu)
    codes, scales = up(codes_np, gpu), up(scales_np, gpu)
    assert fp8lin.lib().fp8lin_linear_candidates_workspace_bytes(m, n, k) > 0
    want = fp8lin.vocabulary_candidates(fp8lin.fp8_linear(x, codes, scales), 0)
    got = fp8lin.linear_candidates(x, codes, scales, 0)
    assert torch.equal(got, want)
    assert 7 in got[:2, 1].long().tolist()
    logits = oracle.linear(bits(x), codes_np, scales_np)
    assert np.array_equal(got.cpu().numpy(), oracle.vocab_candidates(logits, 0))
    if m <= 8:
        # Engine::local_candidates on the tensor-small branch: the same kernel's
        # candidate form, the same result
        eng = fp8lin.LinearEngine(fp8lin.LinearOptions(fp8_tensor_small=True))
        eng.add("lm_head.weight", codes, scales)
        ec, path = eng.local_candidates(x, "lm_head", 0, return_path=True)
        assert path == fp8lin.PATH_TENSOR_SMALL
        assert torch.equal(ec, got)
        assert torch.equal(ec, fp8lin.vocabulary_candidates(eng.linear(x, "lm_head"), 0))
    scales_np[5000, 3] = np.nan
    got = fp8lin.linear_candidates(x, codes, up(scales_np, gpu), 0)
    assert torch.isinf(got[:, 0]).all()


@pytest.mark.parametrize("m", [1, 4])
def test_linear_candidates_graph_replay(fp8lin, gpu, m):
    """Captured head: every replay matches the eager call on the new input
    (M = 1: the GEMV candidate form; M = 4: the small-M row-range form)."""
    x, codes, scales = _head(fp8lin, gpu, m, 31040, 4096, seed=21)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        out = fp8lin.linear_candidates(x, codes, scales, 62080)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = fp8lin.linear_candidates(x, codes, scales, 62080)
    for i in range(4):
        if i:
            x.copy_(fp8lin.gen_activations(m, 4096, seed=100 + i, tag=2, device=gpu))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = fp8lin.linear_candidates(x, codes, scales, 62080)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"


@pytest.mark.parametrize("rows", [1, 4, 9])
@pytest.mark.parametrize("opts", ["default", "tensor_small", "cached"])
def test_engine_local_candidates(fp8lin, gpu, rows, opts):
    """Engine::local_candidates (src/speculative.cpp:25-27) through the engine's
    dispatch: bit-identical to vocabulary_candidates of Engine::linear's output
    on every branch the options select."""
    n, k = 4112, 5120
    codes, scales = fp8lin.gen_weights(n, k, seed=31, tag=1, device=gpu)
    opt = fp8lin.LinearOptions(fp8_tensor_small=(opts == "tensor_small"))
    eng = fp8lin.LinearEngine(opt, weight_cache_bytes=(1 << 30) if opts == "cached" else 0)
    eng.add("lm_head.weight", codes, scales)
    if opts == "cached":
        eng.build_cache()
    x = fp8lin.gen_activations(rows, k, seed=rows, tag=2, device=gpu)
    got, path = eng.local_candidates(x, "lm_head", 62080, return_path=True)
    y, path2 = eng.linear(x, "lm_head", return_path=True)
    assert path == path2
    if opts == "tensor_small" and rows == 4:
        assert path == fp8lin.PATH_TENSOR_SMALL
    if opts == "cached" and rows > 1:
        assert path == fp8lin.PATH_CACHED_BF16
    assert torch.equal(got, fp8lin.vocabulary_candidates(y, 62080))
    if opts == "default":
        assert torch.equal(got, fp8lin.linear_candidates(x, codes, scales, 62080))


# ------------------------------------------------------ rotary embedding
ROPE_CASES = [
    ((1, 12, 256), 64, 1e7, 11, 10),     # decode token, the model's query heads per TP=2 rank
    ((300, 2, 256), 64, 1e7, 11, 10),    # prefill, key heads
    ((7, 3, 128), 128, 1e4, 4, 2),       # full rotation; section bounds inside the pairs
    ((5, 3, 100), 30, 5e5, 2, 5),        # ragged head and rotary sizes
    ((2, 1, 4096), 4096, 1e4, 11, 10),   # largest head the kernel takes (2048 pairs)
    ((3, 5, 128), 30, 1e4, 4, 2),        # odd pair count with 16-byte rows
    ((1024, 9, 136), 64, 1e7, 11, 10),   # long input: each workgroup loops over its token's heads
    ((1050, 6, 100), 30, 5e5, 2, 5),     # the same loop on the scalar path
]


def assert_rope_parity(got, ref, rotary, what, min_exact):
    """The BF16 bar over the whole output (rel_l2 <= 1e-2, cos >= 0.9999,
    the given bit-exact fraction), and per rotated element an error within
    2^-6 of its pair's norm: a rotation keeps the pair's norm, and a one-ulp
    difference of the BF16 cos or sin (device against host math library)
    moves an output by about 2^-8 of it, which near a cancelling sum is many
    ulps of the result."""
    assert_parity(got, ref, what, min_exact=min_exact, elementwise=False)
    half = rotary // 2
    g = bf16_to_f32(got[..., :rotary]).astype(np.float64)
    r = bf16_to_f32(ref[..., :rotary]).astype(np.float64)
    partner = np.concatenate([r[..., half:], r[..., :half]], -1)
    bound = 2.0 ** -6 * np.sqrt(r * r + partner * partner) + 1e-30
    worst = np.max(np.abs(g - r) / bound)
    assert worst <= 1.0, f"{what}: rotated error {worst:.3f} of the pair bound"


@pytest.mark.parametrize("shape,rotary,theta,hs,ws", ROPE_CASES)
def test_rope_oracle(fp8lin, gpu, oracle, shape, rotary, theta, hs, ws):
    """fused_rope (src/optimized.cu:77-78) against the oracle: the part past
    `rotary` bit for bit; the rotated part at the BF16 bar, with >= 99% of it
    bit-exact (cos/sin of the device math library against the host's, both
    rounded to BF16)."""
    rng = np.random.default_rng(sum(shape) + rotary)
    x = rand_bf16(rng, shape)
    pos = rng.integers(0, 4096, size=(3, shape[0]), dtype=np.int64)
    got = bits(fp8lin.fused_rope(up(x, gpu), torch.from_numpy(pos).to(gpu), rotary, theta, hs, ws))
    ref = oracle.rope(x, pos, rotary, theta, hs, ws)
    assert np.array_equal(got[..., rotary:], x[..., rotary:])
    assert_rope_parity(got, ref, rotary, f"rope {shape}", 0.99)


def test_rope_large_positions(fp8lin, gpu, oracle):
    """Positions up to 2^20 (angles up to 1e6 rad): the BF16 bar and the
    pair bound, no bit-exact fraction (the FP32 angle's cos/sin differ by an
    ulp between math libraries often enough at this range)."""
    rng = np.random.default_rng(20)
    x = rand_bf16(rng, (64, 12, 256))
    pos = rng.integers(0, 1 << 20, size=(3, 64), dtype=np.int64)
    got = bits(fp8lin.fused_rope(up(x, gpu), torch.from_numpy(pos).to(gpu), 64, 1e7, 11, 10))
    assert_rope_parity(got, oracle.rope(x, pos, 64, 1e7, 11, 10), 64, "rope large positions", None)


def test_rope_zero_positions(fp8lin, gpu):
    """tests/optimized_test.cpp:139-141: zero positions return x."""
    rng = np.random.default_rng(141)
    x = rand_bf16(rng, (3, 2, 64))
    pos = torch.zeros((3, 3), dtype=torch.int64, device=gpu)
    assert np.array_equal(bits(fp8lin.fused_rope(up(x, gpu), pos, 32, 1e4, 4, 4)), x)


QK_CASES = [
    (1, 12, 2, 256, 64, 0),      # decode, the model's rank shape (QKV-gate width 7168)
    (33, 12, 2, 256, 64, 0),
    (300, 12, 2, 256, 64, 40),   # prefill; projected is a column slice of a wider buffer
    (5, 4, 1, 100, 30, 0),       # D not a multiple of 8 (scalar path of fused_rms)
    (3, 2, 2, 512, 128, 8),      # largest fused head
    (3, 2, 1, 512, 512, 8),      # 256 pairs: the idle fourth wave still fills its part of the table
    (4, 3, 1, 128, 30, 0),       # odd pair count with 16-byte rows
    (2, 5, 3, 64, 64, 3),        # row stride not a multiple of 8 (scalar path), full rotation
    (1100, 12, 2, 256, 64, 0),   # long prefill: one wave per token, all 14 heads
    (1030, 5, 3, 100, 30, 3),    # long input on the scalar path: workgroups loop over a token's heads
    (520, 16, 4, 256, 64, 0),    # one wave per token, 20 heads: two rounds of 8 loads
    (513, 7, 3, 64, 16, 0),      # 8 heads per load, the second load half past the last head; T % 4 != 0
    (512, 3, 1, 128, 32, 8),     # 4 heads per load, two rotary lanes per half
    (516, 2, 2, 512, 512, 0),    # one head per load, full rotation (32 lanes per half)
    (600, 2, 2, 128, 48, 0),     # long input, R / 16 not a power of two: the head-parallel kernel
]


@pytest.mark.parametrize("T,H,HK,D,R,pad", QK_CASES)
def test_qk_norm_rope(fp8lin, gpu, oracle, T, H, HK, D, R, pad):
    """The Q/K epilogue of src/engine.cpp:279-287 in one launch: bit-identical
    to fused_rms of the query (key) heads followed by fused_rope, and at the
    BF16 bar against the oracle's composition."""
    rng = np.random.default_rng(T * 31 + D + pad)
    W = 2 * (H + HK) * D
    buf = rand_bf16(rng, (T, W + pad))
    qw, kw = rand_bf16(rng, (D,), 0.1), rand_bf16(rng, (D,), 0.1)
    pos = rng.integers(0, 8192, size=(3, T), dtype=np.int64)
    args = (R, 1e7, 11, 10)
    proj = up(buf, gpu)[:, :W]
    posd = torch.from_numpy(pos).to(gpu)
    q, k = fp8lin.qk_norm_rope(proj, up(qw, gpu), up(kw, gpu), posd, H, HK, D, *args, 1e-6)
    qv, _, kv, _ = fp8lin.LinearEngine.qkv_gate_views(proj, H, HK, D)
    q2 = fp8lin.fused_rope(fp8lin.fused_rms(qv.contiguous(), up(qw, gpu), 1e-6, True), posd, *args)
    k2 = fp8lin.fused_rope(fp8lin.fused_rms(kv.contiguous(), up(kw, gpu), 1e-6, True), posd, *args)
    assert torch.equal(q.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(k.view(torch.int16), k2.view(torch.int16))
    rq, rk = oracle.qk_norm_rope(buf[:, :W], qw, kw, pos, H, HK, D, *args, eps=1e-6)
    assert_rope_parity(bits(q), rq, R, "qk_norm_rope q", 0.98)
    assert_rope_parity(bits(k), rk, R, "qk_norm_rope k", 0.98)
    assert_parity(bits(q)[..., R:], rq[..., R:], "qk_norm_rope q pass-through", min_exact=0.98)


def test_engine_full_attention_inputs(fp8lin, gpu):
    """LinearEngine.full_attention_inputs (src/engine.cpp:276-287, optimized
    branch): the fused QKV-gate projection, then the Q/K epilogue; gate and v
    are the projection's own columns."""
    H, HK, D, K, T = 12, 2, 256, 5120, 3
    eng = fp8lin.LinearEngine(fp8lin.LinearOptions())
    p = "model.language_model.layers.3.self_attn"
    for i, (name, n) in enumerate((("q_proj", H * 2 * D), ("k_proj", HK * D), ("v_proj", HK * D))):
        c, s = fp8lin.gen_weights(n, K, seed=5, tag=10 + i, device=gpu)
        eng.add(f"{p}.{name}.weight", c, s)
    eng.fuse_weights(p + ".qkv_gate", [p + ".q_proj", p + ".k_proj", p + ".v_proj"])
    rng = np.random.default_rng(3)
    qw, kw = up(rand_bf16(rng, (D,), 0.1), gpu), up(rand_bf16(rng, (D,), 0.1), gpu)
    pos = torch.from_numpy(rng.integers(0, 4096, size=(3, T), dtype=np.int64)).to(gpu)
    rope = {"partial_rotary_factor": 0.25, "mrope_section": [11, 11, 10], "rope_theta": 10000000}
    x = fp8lin.gen_activations(T, K, seed=9, tag=2, device=gpu)
    q, gate, k, v = eng.full_attention_inputs(x, p, pos, qw, kw, H, HK, D, rope, 1e-6)
    proj = eng.linear(x, p + ".qkv_gate")
    q2, k2 = fp8lin.qk_norm_rope(proj, qw, kw, pos, H, HK, D, 64, 1e7, 11, 10, 1e-6)
    _, gate2, _, v2 = fp8lin.LinearEngine.qkv_gate_views(proj, H, HK, D)
    for a, b in ((q, q2), (k, k2), (gate, gate2), (v, v2)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_qk_norm_rope_graph_replay(fp8lin, gpu):
    """The decode step's Q/K epilogue captured once: each replay, after the
    projection and the positions change in place (with eager work between
    replays), equals the eager call on the new inputs."""
    rng = np.random.default_rng(287)
    H, HK, D = 12, 2, 256
    proj = up(rand_bf16(rng, (1, 2 * (H + HK) * D)), gpu)
    qw, kw = up(rand_bf16(rng, (D,), 0.1), gpu), up(rand_bf16(rng, (D,), 0.1), gpu)
    pos = torch.from_numpy(rng.integers(0, 4096, size=(3, 1), dtype=np.int64)).to(gpu)
    args = (H, HK, D, 64, 1e7, 11, 10, 1e-6)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        q, k = fp8lin.qk_norm_rope(proj, qw, kw, pos, *args)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            q, k = fp8lin.qk_norm_rope(proj, qw, kw, pos, *args)
    for i in range(4):
        proj.copy_(up(rand_bf16(rng, tuple(proj.shape)), gpu))
        pos += 17 * (i + 1)
        q_eager, k_eager = fp8lin.qk_norm_rope(proj, qw, kw, pos, *args)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(q.view(torch.int16), q_eager.view(torch.int16)), f"replay {i}"
        assert torch.equal(k.view(torch.int16), k_eager.view(torch.int16)), f"replay {i}"
