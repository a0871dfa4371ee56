"""GPU parity at every shape the benchmark times, the way
the reference's linear benchmark checks each shape it times
(tests/linear_benchmark.cpp:22-23,35-47):

- decode gate/up + SwiGLU at M = 1, 2 on 17408 x 5120 (all 8704 outputs), and
  the K = 8704 SwiGLU GEMV forms;
- prefill gate/up + SwiGLU at M = 512 and 1024 on every row, and at the real
  prompt length M = 3913 (a partial last 256-row tile) on a row sample plus
  every row of that tile;
- the vocab-sharded output head 75968 x 5120 at M = 1 (every logit and the
  candidates) and at M = 512 (a row sample, plus the 192-column tail of the
  last 256-row weight tile on every row);
- the GDN in_proj_all mixed group, 8192 FP8 rows + 48 BF16 rows at K = 5120
  (src/engine.cpp:198-199, tests/linear_benchmark.cpp:22), at M = 1, 4, 512;
- fp8_tensor_small on unaligned contiguous views (the reference accepts any
  contiguous tensor, src/fp8_tensor.cu:54-59).

Inputs are the benchmark's seeded device-generated weights and activations
(bit-identical to the oracle's generator).
"""
import numpy as np
import pytest
import torch

from parity import assert_parity, ulp_distance

pytestmark = pytest.mark.gpu


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def weights(fp8lin, dev, n, k, tag=1):
    codes, scales = fp8lin.gen_weights(n, k, seed=0, tag=tag, device=dev)
    return codes, scales, codes.cpu().numpy(), scales.cpu().numpy()


def check_swiglu(fp8lin, oracle, x, codes, scales, c_np, s_np, rows, what):
    """Fused gate/up + SwiGLU on the x rows `rows`: the unfused gate/up at the
    parity bar against the oracle; the fused output bit-equal to
    fused_swiglu(fp8_linear) (the same per-row sums, the same epilogue
    helper), within 1 ulp of the oracle SwiGLU of the device's own gate/up,
    and at the bar against the oracle composition."""
    fused = fp8lin.linear_swiglu(x, codes, scales, split=False)
    gate_up = fp8lin.fp8_linear(x, codes, scales, True, split=False)
    assert torch.equal(fused, fp8lin.fused_swiglu(gate_up)), f"{what}: fused != unfused"
    ref_gu = oracle.linear(bits(x)[rows], c_np, s_np)
    gu = bits(gate_up)[rows]
    assert_parity(gu, ref_gu, f"{what} gate/up")
    f = bits(fused)[rows]
    assert ulp_distance(f, oracle.swiglu(gu)).max() <= 1, what
    assert_parity(f, oracle.swiglu(ref_gu), f"{what} swiglu", elementwise=False)
    # the workspace form (K split on the tail tiles at M = 1024, 3913):
    # only the FP32 summation order of those tiles differs
    split = bits(fp8lin.linear_swiglu(x, codes, scales))[rows]
    assert_parity(split, oracle.swiglu(ref_gu), f"{what} swiglu, split K", elementwise=False)


@pytest.mark.parametrize("m", [1, 2])
def test_decode_gate_up_swiglu(fp8lin, gpu, oracle, m):
    """Config 5, M = 1 link and config 3 M = 2: gemv_ring_kernel<M,2,5,SWIGLU>."""
    n, k = 17408, 5120
    codes, scales, c_np, s_np = weights(fp8lin, gpu, n, k)
    x = fp8lin.gen_activations(m, k, seed=0, tag=2, device=gpu)
    check_swiglu(fp8lin, oracle, x, codes, scales, c_np, s_np, np.arange(m), f"gate/up M={m}")


@pytest.mark.parametrize("m", [1, 2])
def test_swiglu_gemv_k8704(fp8lin, gpu, oracle, m):
    """K = 8704: the nine-step ring kernel at M = 1, the general kernel at
    M = 2."""
    n, k = 2048, 8704
    codes, scales, c_np, s_np = weights(fp8lin, gpu, n, k, tag=3)
    x = fp8lin.gen_activations(m, k, seed=0, tag=4, device=gpu)
    check_swiglu(fp8lin, oracle, x, codes, scales, c_np, s_np, np.arange(m), f"swiglu K=8704 M={m}")


@pytest.mark.parametrize("m", [512, 1024])
def test_prefill_swiglu_all_rows(fp8lin, gpu, oracle, m):
    """Config 4 chunks, every row against the oracle."""
    n, k = 17408, 5120
    codes, scales, c_np, s_np = weights(fp8lin, gpu, n, k)
    x = fp8lin.gen_activations(m, k, seed=0, tag=2, device=gpu)
    check_swiglu(fp8lin, oracle, x, codes, scales, c_np, s_np, np.arange(m), f"prefill M={m}")


def test_prefill_swiglu_prompt_length(fp8lin, gpu, oracle):
    """M = 3913 (text + image tokens): the last 256-row M tile holds 73 rows."""
    n, k, m = 17408, 5120, 3913
    codes, scales, c_np, s_np = weights(fp8lin, gpu, n, k)
    x = fp8lin.gen_activations(m, k, seed=0, tag=2, device=gpu)
    rng = np.random.default_rng(m)
    rows = np.unique(np.concatenate([rng.choice(m - 73, 24, replace=False), np.arange(m - 73, m)]))
    check_swiglu(fp8lin, oracle, x, codes, scales, c_np, s_np, rows, "prefill M=3913")


@pytest.fixture(scope="module")
def head(fp8lin, gpu):
    n, k = 75968, 5120
    return weights(fp8lin, gpu, n, k, tag=5)


def test_head_m1(fp8lin, gpu, oracle, head):
    """Config 5 head at decode: every logit; candidates equal the oracle's
    candidates of the device logits, and the fused call equals
    vocabulary_candidates(fp8_linear) bit for bit."""
    codes, scales, c_np, s_np = head
    x = fp8lin.gen_activations(1, 5120, seed=0, tag=6, device=gpu)
    logits = fp8lin.fp8_linear(x, codes, scales, True)
    lb = bits(logits)
    assert_parity(lb, oracle.linear(bits(x), c_np, s_np), "head M=1")
    offset = 75968
    cand = fp8lin.vocabulary_candidates(logits, offset)
    assert np.array_equal(cand.cpu().numpy(), oracle.vocab_candidates(lb, offset))
    fused = fp8lin.linear_candidates(x, codes, scales, offset)
    assert torch.equal(fused, cand)


def test_head_m512(fp8lin, gpu, oracle, head):
    """Config 5 head at the prefill chunk: a sample of 8 rows on every column,
    and every row on the 192 columns past the last full 256-row weight tile
    (75776..75967)."""
    codes, scales, c_np, s_np = head
    m, n = 512, 75968
    x = fp8lin.gen_activations(m, 5120, seed=0, tag=6, device=gpu)
    y = bits(fp8lin.fp8_linear(x, codes, scales, split=False))
    xb = bits(x)
    rows = np.array([0, 1, 100, 255, 256, 300, 510, 511])
    assert_parity(y[rows], oracle.linear(xb[rows], c_np, s_np), "head M=512 rows")
    tail = (75776, n)
    ref = oracle.linear(xb, c_np, s_np, rows=tail)
    assert_parity(y[:, tail[0]:], ref[:, tail[0]:], "head M=512 column tail")
    # Through Engine::linear (with a workspace): 594 tiles = 2 rounds of 256
    # + 82, whose tiles (weight rows 65536..75967 of both row tiles) split K
    # three ways; only their FP32 summation order differs from fp8_linear.
    eng = fp8lin.LinearEngine()
    eng.add("lm_head.weight", codes, scales)
    ys, path = eng.linear(x, "lm_head", return_path=True)
    assert path == fp8lin.PATH_FP8_GEMM
    ys = bits(ys)
    split = (65536, n)
    assert np.array_equal(ys[:, :split[0]], y[:, :split[0]])
    ref = oracle.linear(xb[rows], c_np, s_np, rows=split)
    assert_parity(ys[rows, split[0]:], ref[:, split[0]:], "head M=512 split tiles")
    assert_parity(ys, y, "head M=512 split vs unsplit", min_exact=0.99)
    assert (ulp_distance(ys, y) > 1).sum() <= max(1, ys.size // 10000)


@pytest.mark.parametrize("m", [1, 4, 512])
def test_gdn_in_proj_all(fp8lin, gpu, oracle, m):
    """The GDN in_proj_all group at one rank's size: FP8 qkv (5120 rows) + z
    (3072) fused into 8192 rows, then BF16 b + a (24 + 24); the output is the
    column concatenation of the four projections (src/engine.cpp:198-199)."""
    F, k = fp8lin, 5120
    eng = F.LinearEngine(F.LinearOptions(fp8_tensor_small=m in (2, 4, 8)))
    parts = []
    for i, (name, rows) in enumerate([("in_proj_qkv", 5120), ("in_proj_z", 3072)]):
        codes, scales, c_np, s_np = weights(F, gpu, rows, k, tag=10 + i)
        eng.add(f"l.{name}.weight", codes, scales)
        parts.append(("fp8", c_np, s_np))
    for i, name in enumerate(["in_proj_b", "in_proj_a"]):
        w = (F.gen_activations(24, k, seed=1, tag=20 + i, device=gpu).float() * 0.02).to(torch.bfloat16)
        eng.add(f"l.{name}.weight", w.contiguous())
        parts.append(("bf16", bits(w), None))
    eng.fuse_weights("l.in_proj_all", ["l.in_proj_qkv", "l.in_proj_z", "l.in_proj_b", "l.in_proj_a"])
    assert eng.mixed_projections["l.in_proj_all"] == ["l.in_proj_all.group0", "l.in_proj_all.group1"]
    x = F.gen_activations(m, k, seed=0, tag=7, device=gpu)
    y = bits(eng.linear(x, "l.in_proj_all"))
    assert y.shape == (m, 8240)
    sample = np.arange(m) if m <= 8 else np.array([0, 7, 255, 256, 400, 511])
    xb = bits(x)[sample]
    ref = np.concatenate([oracle.linear(xb, c, s) if kind == "fp8" else oracle.linear_bf16w(xb, c)
                          for kind, c, s in parts], axis=1)
    assert_parity(y[sample], ref, f"in_proj_all M={m}")
    if m == 4:
        assert eng.cache_stats()["fp8_tensor_calls"] == 1
    # M = 1: one launch for both groups (the FP8 ring GEMV's rows, then the
    # BF16 rows); more rows: one launch per group.  Either way the bits of the
    # groups' own calls.
    sep = np.concatenate([bits(eng.linear(x, f"l.in_proj_all.group{i}")) for i in (0, 1)], axis=1)
    assert np.array_equal(y, sep)


@pytest.mark.parametrize("m", [4, 300])
def test_mixed_group_under_capture(fp8lin, gpu, m):
    """A mixed FP8 + BF16 group at several rows captured in a HIP graph:
    every replay (with eager calls of other sizes on the capture stream and
    on the default stream in between) equals the eager call."""
    F, k = fp8lin, 5120
    eng = F.LinearEngine()
    codes, scales, _, _ = weights(F, gpu, 8192, k, tag=50)
    eng.add("l.q.weight", codes, scales)
    w = (F.gen_activations(48, k, seed=1, tag=51, device=gpu).float() * 0.02).to(torch.bfloat16).contiguous()
    eng.add("l.b.weight", w)
    eng.fuse_weights("l.g", ["l.q", "l.b"])
    x = F.gen_activations(m, k, seed=0, tag=52, device=gpu)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        eng.linear(x, "l.g")
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = eng.linear(x, "l.g")
    for i in range(3):
        x.copy_(F.gen_activations(m, k, seed=0, tag=60 + i, device=gpu))
        other = F.gen_activations(m + 3, k, seed=0, tag=70 + i, device=gpu)
        with torch.cuda.stream(stream):
            eng.linear(other, "l.g")
        eng.linear(other, "l.g")
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = eng.linear(x, "l.g")
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"


@pytest.mark.parametrize("na,nb,k", [(2049, 7, 4096), (1025, 1, 2304), (16383, 1024, 5120), (3000, 48, 128)])
def test_fp8_bf16_pair_one_row(fp8lin, gpu, oracle, na, nb, k):
    """An FP8 weight and a BF16 weight in one group call at one activation
    row run in one launch (odd row counts, the row limits of both parts,
    K = 4096's four steps and a one-step K): every output against the oracle
    and bit-equal to each weight's own call."""
    F = fp8lin
    eng = F.LinearEngine()
    codes, scales, c_np, s_np = weights(F, gpu, na, k, tag=40)
    eng.add("l.a.weight", codes, scales)
    wb = (F.gen_activations(nb, k, seed=2, tag=41, device=gpu).float() * 0.02).to(torch.bfloat16).contiguous()
    eng.add("l.b.weight", wb)
    eng.fuse_weights("l.ab", ["l.a", "l.b"])
    assert eng.mixed_projections["l.ab"] == ["l.a", "l.b"]
    x = F.gen_activations(1, k, seed=0, tag=42, device=gpu)
    y = bits(eng.linear(x, "l.ab"))
    xb = bits(x)
    ref = np.concatenate([oracle.linear(xb, c_np, s_np), oracle.linear_bf16w(xb, bits(wb))], axis=1)
    assert_parity(y, ref, f"pair {na}+{nb} K={k}")
    sep = np.concatenate([bits(eng.linear(x, "l.a")), bits(eng.linear(x, "l.b"))], axis=1)
    assert np.array_equal(y, sep)


def test_split_k_into_unaligned_column_slice(fp8lin, gpu, oracle):
    """A K-split FP8 group (7168 rows at M=512: 56 tiles x 4 K ranges) written
    into the column slice that starts 6 columns into a 7174-column output,
    after a 6-row BF16 group: with a row stride of 7174 elements the tail
    reduce stores every other row with 8-byte stores and the others with
    2-byte stores.  The slice equals the same projection on its own (column
    0, every row aligned) bit for bit, and both groups meet the parity bar."""
    F, k, m = fp8lin, 5120, 512
    codes, scales, c_np, s_np = weights(F, gpu, 7168, k, tag=31)
    w = (F.gen_activations(6, k, seed=1, tag=32, device=gpu).float() * 0.02).to(torch.bfloat16).contiguous()
    eng = F.LinearEngine()
    eng.add("l.b.weight", w)
    eng.add("l.q.weight", codes, scales)
    eng.fuse_weights("l.mix", ["l.b", "l.q"])
    assert eng.mixed_projections["l.mix"] == ["l.b", "l.q"]
    alone = F.LinearEngine()
    alone.add("q.weight", codes, scales)
    x = F.gen_activations(m, k, seed=0, tag=33, device=gpu)
    y = bits(eng.linear(x, "l.mix"))
    assert y.shape == (m, 7174)
    ya, path = alone.linear(x, "q", return_path=True)
    assert path == F.PATH_FP8_GEMM
    assert np.array_equal(y[:, 6:], bits(ya))
    rows = np.array([0, 1, 2, 255, 256, 511])
    xb = bits(x)[rows]
    assert_parity(y[rows, 6:], oracle.linear(xb, c_np, s_np), "split slice")
    assert_parity(y[rows, :6], oracle.linear_bf16w(xb, bits(w)), "bf16 group")


@pytest.mark.parametrize("m,k", [(2, 256), (4, 5120), (8, 384)])
def test_tensor_small_unaligned_views(fp8lin, gpu, oracle, m, k):
    """An unaligned contiguous view of x or of the codes (the reference's own
    pattern, tests/optimized_test.cpp:15-21) is served, not refused: the
    multi-row GEMV runs instead, bit-equal to fp8_linear on the same views,
    and at the parity bar against the oracle."""
    rng = np.random.default_rng(m * k)
    n = 19
    codes_np = rng.integers(0, 126, (n, k), dtype=np.uint8)
    scales_np = (rng.random((n, k // 128)) * .01 + .001).astype(np.float32)
    x32 = rng.standard_normal(m * k).astype(np.float32)
    xflat = torch.zeros(m * k + 1, dtype=torch.bfloat16, device=gpu)
    xflat[1:] = torch.from_numpy(x32).to(torch.bfloat16).to(gpu)
    xu = xflat.narrow(0, 1, m * k).reshape(m, k)
    cflat = torch.zeros(n * k + 1, dtype=torch.uint8, device=gpu)
    cflat[1:] = torch.from_numpy(codes_np.reshape(-1)).to(gpu)
    cu = cflat.narrow(0, 1, n * k).reshape(n, k)
    ca = torch.from_numpy(codes_np).to(gpu)
    s = torch.from_numpy(scales_np).to(gpu)
    ref = oracle.linear(bits(xu), codes_np, scales_np)
    for xx, cc, what in [(xu, ca, "x"), (xu.clone(), cu, "codes"), (xu, cu, "both")]:
        for split in (1, 4):
            y = fp8lin.fp8_tensor_small(xx, cc, s, split)
            assert_parity(bits(y), ref, f"unaligned {what} m={m} k={k} split={split}")
            assert torch.equal(y, fp8lin.fp8_linear(xx, cc, s)), what


@pytest.fixture(scope="module")
def head124160(fp8lin, gpu):
    return weights(fp8lin, gpu, 124160, 5120, tag=41)


@pytest.mark.parametrize("m", [2, 4, 8])
@pytest.mark.parametrize("shape", ["5120x5120", "124160x5120"])
def test_reference_benchmark_shapes(fp8lin, gpu, oracle, head124160, shape, m):
    """The reference benchmark's remaining shapes (tests/linear_benchmark.cpp:
    22-23): 5120 x 5120 and the full-vocabulary TP = 2 head 124160 x 5120 at
    M = 2, 4, 8 through fp8_linear and fp8_tensor_small with split 1 and 4,
    every output against the FP64 oracle; split 1 and 4 give the same bits
    (the kernel's own K partition).  fp8_linear takes the small-M kernel, bit
    for bit, except at 2 rows against 5120 x 5120 (20 rows per CU), which
    stay on the two-row GEMV; the head's 485 rows per CU take it at M = 2
    too."""
    if shape == "5120x5120":
        codes, scales, c_np, s_np = weights(fp8lin, gpu, 5120, 5120, tag=40)
    else:
        codes, scales, c_np, s_np = head124160
    k = 5120
    x = fp8lin.gen_activations(m, k, seed=0, tag=42, device=gpu)
    ref = oracle.linear(bits(x), c_np, s_np)
    y = fp8lin.fp8_linear(x, codes, scales, True)
    assert_parity(bits(y), ref, f"{shape} fp8_linear M={m}")
    s1 = fp8lin.fp8_tensor_small(x, codes, scales, 1)
    assert_parity(bits(s1), ref, f"{shape} fp8_tensor_small M={m}")
    assert torch.equal(fp8lin.fp8_tensor_small(x, codes, scales, 4), s1)
    if m > 2 or shape == "124160x5120":
        assert torch.equal(y, s1)
