"""Tensor-level host mirror of the reference's linear-path operators.

Same names, argument meaning and error behaviour as the reference's ATen
functions (laoyin/a100-vision-infer include/avi/ops.h:6-8,10,11,18-20 and
include/avi/engine.h:13): inputs are device tensors, the output is allocated
on the input's device, work is enqueued on torch's current stream, and a
violated precondition raises (Fp8linError, a RuntimeError, where the
reference's TORCH_CHECK raises c10::Error).  All arithmetic runs in the HIP
library through the C ABI; torch only provides memory and the stream.
"""
import ctypes

import torch

from ._lib import (ERR_ARGUMENT, ERR_SHAPE, Fp8linError, LinearOptions, Weight, check, lib)


def _fail(code, msg):
    raise Fp8linError(code, msg)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


_ready_devices = set()


def _stream(t):
    """torch's current stream on t's device, as a hipStream_t.  The first
    time a device is seen, fp8lin_init runs with that device current, so the
    library's one-time device queries never happen inside a graph capture
    that starts later."""
    idx = t.device.index if t.device.index is not None else torch.cuda.current_device()
    if idx not in _ready_devices:
        with torch.cuda.device(idx):
            check(lib().fp8lin_init())
        _ready_devices.add(idx)
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _is_dev(t):
    return isinstance(t, torch.Tensor) and t.is_cuda


def _scale_cols(scales, codes_rows, k, what="Invalid FP8 scales"):
    # src/optimized.cu:64
    ok = (_is_dev(scales) and scales.dtype == torch.float32 and scales.is_contiguous() and
          ((scales.dim() == 1 and scales.numel() == codes_rows) or
           (scales.dim() == 2 and scales.size(0) == codes_rows and scales.size(1) == (k + 127) // 128)))
    if not ok:
        _fail(ERR_ARGUMENT, what)
    return 1 if scales.dim() == 1 else scales.size(1)


def _check_x(x, what):
    if not (_is_dev(x) and x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous()):
        _fail(ERR_ARGUMENT, what)


def _check_codes(codes, x, what="Invalid FP8 weights"):
    if not (_is_dev(codes) and codes.device == x.device and codes.dtype == torch.uint8 and
            codes.dim() == 2 and codes.is_contiguous() and codes.size(1) == x.size(1)):
        _fail(ERR_ARGUMENT, what)


def fp8_decode(codes, scales):
    """`Tensor fp8_decode(Tensor codes, Tensor scales)` -- src/kernels.cu:17-27."""
    if not (_is_dev(codes) and codes.dtype == torch.uint8 and codes.dim() == 2 and
            codes.is_contiguous()):
        _fail(ERR_ARGUMENT, "FP8 codes must be contiguous CUDA uint8 matrix")
    sc = _scale_cols(scales, codes.size(0), codes.size(1), "Invalid FP8 row scales")
    y = torch.empty(codes.shape, dtype=torch.bfloat16, device=codes.device)
    if codes.numel():
        check(lib().fp8lin_decode(_ptr(codes), _ptr(scales), sc, _ptr(y), codes.size(0),
                                  codes.size(1), _stream(codes)))
    return y


def fp8_linear(x, codes, scales, vector_gemv=False, split=True):
    """`at::Tensor fp8_linear(x, codes, scales, bool vector_gemv=false)` --
    src/optimized.cu:61-70.  split: give the prefill GEMM a workspace (allocated
    here, on the input's stream, as the reference allocates its operators'
    partials, src/fp8_tensor.cu:65) so it may split K where whole tiles would
    leave CUs idle (fp8lin_linear_ws); False runs every tile whole
    (fp8lin_linear)."""
    _check_x(x, "FP8 linear expects CUDA BF16 [M,K]")
    _check_codes(codes, x)
    sc = _scale_cols(scales, codes.size(0), codes.size(1))
    M, N, K = x.size(0), codes.size(0), codes.size(1)
    if not (M > 0 and N > 0 and K > 0):
        _fail(ERR_SHAPE, "Empty GEMM")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    need = lib().fp8lin_linear_workspace_bytes(M, N, K) if split else 0
    if need:
        ws = torch.empty(need, dtype=torch.uint8, device=x.device)
        check(lib().fp8lin_linear_ws(_ptr(x), _ptr(codes), _ptr(scales), sc, _ptr(y), M, N, K,
                                     int(bool(vector_gemv)), _ptr(ws), need, _stream(x)))
    else:
        check(lib().fp8lin_linear(_ptr(x), _ptr(codes), _ptr(scales), sc, _ptr(y), M, N, K,
                                  int(bool(vector_gemv)), _stream(x)))
    return y


def linear_swiglu(x, codes, scales, split=True):
    """Fused `fused_swiglu(fp8_linear(x, gate_up))` (src/engine.cpp:415).
    split: give the prefill GEMM a workspace so it may split K where whole
    tiles would leave CUs idle (fp8lin_linear_swiglu_ws); False runs every
    tile whole (fp8lin_linear_swiglu)."""
    _check_x(x, "FP8 linear expects CUDA BF16 [M,K]")
    _check_codes(codes, x)
    sc = _scale_cols(scales, codes.size(0), codes.size(1))
    M, N, K = x.size(0), codes.size(0), codes.size(1)
    if not (M > 0 and N > 0 and K > 0) or N % 2:
        _fail(ERR_SHAPE, "Invalid gate/up geometry")
    y = torch.empty((M, N // 2), dtype=torch.bfloat16, device=x.device)
    need = lib().fp8lin_linear_swiglu_workspace_bytes(M, N, K) if split else 0
    if need:
        ws = torch.empty(need, dtype=torch.uint8, device=x.device)
        check(lib().fp8lin_linear_swiglu_ws(_ptr(x), _ptr(codes), _ptr(scales), sc, _ptr(y), M, N, K, _ptr(ws),
                                            need, _stream(x)))
    else:
        check(lib().fp8lin_linear_swiglu(_ptr(x), _ptr(codes), _ptr(scales), sc, _ptr(y), M, N, K,
                                         _stream(x)))
    return y


def fused_swiglu(gate_up):
    """`at::Tensor fused_swiglu(at::Tensor gate_up)` -- src/optimized.cu:73-74."""
    if not (_is_dev(gate_up) and gate_up.is_contiguous() and gate_up.dim() == 2 and
            gate_up.dtype == torch.bfloat16 and gate_up.size(1) % 2 == 0):
        _fail(ERR_ARGUMENT, "Invalid SwiGLU input")
    M, D = gate_up.size(0), gate_up.size(1) // 2
    y = torch.empty((M, D), dtype=torch.bfloat16, device=gate_up.device)
    check(lib().fp8lin_swiglu(_ptr(gate_up), _ptr(y), M, D, _stream(gate_up)))
    return y


def add_bias(y, bias):
    """In place y = y + bias for BF16 y [..., N] and bias [N]: the BF16 sum of
    src/engine.cpp:240 (FP32 add, one rounding), for a caller that reduces an
    output across ranks before adding its bias."""
    if not (_is_dev(y) and _is_dev(bias) and y.dtype == torch.bfloat16 and bias.dtype == torch.bfloat16 and
            y.dim() >= 1 and bias.dim() == 1 and bias.numel() == y.size(-1) and bias.is_contiguous() and
            y.stride(-1) == 1 and (y.dim() == 1 or y.is_contiguous())):
        _fail(ERR_ARGUMENT, "Invalid bias add")
    N = y.size(-1)
    rows = y.numel() // N if N else 0
    check(lib().fp8lin_add_bias(_ptr(y), N, _ptr(bias), rows, N, _stream(y)))
    return y


def small_linear_shared(x, weight, scales=None):
    """`at::Tensor small_linear_shared(x, weight, scales={})` --
    src/deep_kernels.cu:134-157."""
    if not (_is_dev(x) and x.dim() == 2 and x.is_contiguous() and x.dtype == torch.bfloat16 and
            _is_dev(weight) and weight.dim() == 2 and weight.is_contiguous() and
            weight.device == x.device and x.size(1) == weight.size(1)):
        _fail(ERR_ARGUMENT, "Invalid shared GEMV inputs")
    M, N, K = x.size(0), weight.size(0), x.size(1)
    if not (1 <= M <= 8 and N > 0 and K > 0):
        _fail(ERR_SHAPE, "Shared GEMV requires 1..8 rows")
    if scales is not None:
        if weight.dtype != torch.uint8:
            _fail(ERR_ARGUMENT, "Invalid shared FP8 scales")
        sc = _scale_cols(scales, N, K, "Invalid shared FP8 scales")
    else:
        if weight.dtype != torch.bfloat16:
            _fail(ERR_ARGUMENT, "Shared GEMV expects BF16 or FP8 weights")
        sc = 1
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    check(lib().fp8lin_linear_shared(_ptr(x), _ptr(weight), _ptr(scales), sc, _ptr(y), M, N, K,
                                     _stream(x)))
    return y


def _tensor_small_checks(x, codes, scales, split, what, n16=False):
    ok = (_is_dev(x) and x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous() and
          _is_dev(codes) and codes.device == x.device and codes.dtype == torch.uint8 and
          codes.dim() == 2 and codes.is_contiguous() and
          _is_dev(scales) and scales.device == x.device and scales.dtype == torch.float32 and
          scales.dim() == 2 and scales.is_contiguous() and
          2 <= x.size(0) <= 8 and x.size(1) > 0 and x.size(1) == codes.size(1) and
          x.size(1) % 128 == 0 and codes.size(0) > 0 and scales.size(0) == codes.size(0) and
          scales.size(1) == x.size(1) // 128 and split in (1, 4) and
          (not n16 or codes.size(0) % 16 == 0))
    if not ok:
        _fail(ERR_ARGUMENT, what)


def fp8_tensor_small(x, codes, scales, split=1):
    """`at::Tensor fp8_tensor_small(x, codes, scales, int split=1)` --
    src/fp8_tensor.cu:53-71."""
    _tensor_small_checks(x, codes, scales, split, "Invalid Ampere FP8 W8A16 geometry/dtype")
    return _run_tensor_small(x, codes, scales, split)


def tilelang_fp8_small(x, codes, scales, split):
    """`at::Tensor tilelang_fp8_small(x, codes, scales, int split)` --
    src/tilelang.cpp:94-107 (same contract plus N % 16 == 0; served by the
    same matrix-core kernel)."""
    _tensor_small_checks(x, codes, scales, split, "Invalid TileLang FP8 W8A16 inputs", n16=True)
    return _run_tensor_small(x, codes, scales, split)


def _run_tensor_small(x, codes, scales, split):
    M, N, K = x.size(0), codes.size(0), x.size(1)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    nbytes = lib().fp8lin_tensor_small_workspace_bytes(M, N, split)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device) if nbytes else None
    check(lib().fp8lin_tensor_small(_ptr(x), _ptr(codes), _ptr(scales), _ptr(y), M, N, K, split,
                                    _ptr(ws), nbytes, _stream(x)))
    return y


def gemm_bf16(x, w, out=None):
    """BF16 `at::matmul(x, w.t())` (src/engine.cpp:221,236) on the HIP GEMM."""
    _check_x(x, "BF16 GEMM expects CUDA BF16 [M,K]")
    if not (_is_dev(w) and w.dtype == torch.bfloat16 and w.dim() == 2 and w.is_contiguous() and
            w.size(1) == x.size(1)):
        _fail(ERR_ARGUMENT, "Invalid BF16 weights")
    M, N, K = x.size(0), w.size(0), x.size(1)
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    check(lib().fp8lin_gemm_bf16(_ptr(x), _ptr(w), _ptr(y), y.stride(0), M, N, K, _stream(x)))
    return y


def fused_rms(x, weight, eps, one_center):
    """`at::Tensor fused_rms(x, weight, double eps, bool one_center)` --
    src/optimized.cu:71-72 (RMSNorm over the last dimension)."""
    if not (_is_dev(x) and _is_dev(weight) and weight.device == x.device and
            x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and x.dim() >= 1 and
            weight.numel() == x.size(-1)):
        _fail(ERR_ARGUMENT, "Invalid RMS input")
    x, weight = x.contiguous(), weight.contiguous()
    y = torch.empty_like(x)
    D = x.size(-1)
    rows = x.numel() // D if D else 0
    check(lib().fp8lin_rms(_ptr(x), _ptr(weight), _ptr(y), rows, D, float(eps),
                           int(bool(one_center)), _stream(x)))
    return y


def residual_rms(x, update, weight, eps, centered=True):
    """`std::pair<Tensor,Tensor> residual_rms(residual, update, weight, eps,
    centered=true)` -- src/dual_path.cu:68-78.  Returns (bf16(x + update),
    RMSNorm of that sum)."""
    ok = (_is_dev(x) and x.dim() >= 2 and x.dtype == torch.bfloat16 and x.is_contiguous() and
          x.numel() > 0 and _is_dev(update) and update.device == x.device and
          update.dtype == x.dtype and update.shape == x.shape and update.is_contiguous() and
          _is_dev(weight) and weight.device == x.device and weight.dtype == x.dtype and
          weight.is_contiguous() and weight.numel() == x.size(-1))
    if not ok:
        _fail(ERR_ARGUMENT, "Invalid fused residual RMS input")
    residual, y = torch.empty_like(x), torch.empty_like(x)
    D = x.size(-1)
    check(lib().fp8lin_residual_rms(_ptr(x), _ptr(update), _ptr(weight), _ptr(residual), _ptr(y),
                                    x.numel() // D, D, float(eps), int(bool(centered)), _stream(x)))
    return residual, y


def reduce_residual_rms(x, partials, weight, eps, centered=True):
    """Row-parallel reduce folded into residual_rms: partials [ranks, *x.shape]
    are per-rank outputs of a row-parallel projection; update =
    bf16(sum over ranks in order, FP32), then (bf16(x + update), RMSNorm of
    it) as residual_rms (src/engine.cpp:183-195 with src/dual_path.cu:68-78)."""
    ok = (_is_dev(x) and x.dim() >= 2 and x.dtype == torch.bfloat16 and x.is_contiguous() and
          x.numel() > 0 and _is_dev(partials) and partials.device == x.device and
          partials.dtype == x.dtype and partials.is_contiguous() and partials.dim() == x.dim() + 1 and
          partials.shape[1:] == x.shape and 1 <= partials.size(0) <= 8 and
          _is_dev(weight) and weight.device == x.device and weight.dtype == x.dtype and
          weight.is_contiguous() and weight.numel() == x.size(-1))
    if not ok:
        _fail(ERR_ARGUMENT, "Invalid reduce + residual RMS input")
    residual, y = torch.empty_like(x), torch.empty_like(x)
    D = x.size(-1)
    check(lib().fp8lin_reduce_residual_rms(_ptr(x), _ptr(partials), partials.size(0), _ptr(weight), _ptr(residual),
                                           _ptr(y), x.numel() // D, D, float(eps), int(bool(centered)), _stream(x)))
    return residual, y


def _positions_ok(positions, x, T):
    return (_is_dev(positions) and positions.device == x.device and positions.dtype == torch.int64 and
            positions.dim() == 2 and positions.size(0) == 3 and positions.size(1) == T)


def fused_rope(x, positions, rotary, theta, height_section, width_section):
    """`at::Tensor fused_rope(x, positions, int rotary, double theta,
    int height_section, int width_section)` -- src/optimized.cu:77-78: the
    interleaved multi-axis rotary embedding of x [T, H, D] at positions
    [3, T] (int64), first `rotary` dimensions of each head."""
    ok = (_is_dev(x) and x.dim() == 3 and x.dtype == torch.bfloat16 and _positions_ok(positions, x, x.size(0)) and
          rotary > 0 and rotary % 2 == 0 and rotary <= x.size(2))
    if not ok:
        _fail(ERR_ARGUMENT, "Invalid RoPE input")
    x, positions = x.contiguous(), positions.contiguous()
    y = torch.empty_like(x)
    T, H, D = x.shape
    check(lib().fp8lin_rope(_ptr(x), _ptr(positions), _ptr(y), T, H, D, int(rotary), float(theta),
                            int(height_section), int(width_section), _stream(x)))
    return y


def qk_norm_rope(projected, q_norm, k_norm, positions, heads, kv_heads, head_dim, rotary, theta, height_section,
                 width_section, eps):
    """The optimized branch of src/engine.cpp:279-287 on the QKV-gate output
    projected [T, H*2D + 2*HK*D] (row stride may be wider): returns q
    [T, H, D] = rope(rms(query heads, q_norm)) and k [T, HK, D] =
    rope(rms(key heads, k_norm)) with the centered RMSNorm, in one launch.
    Equal bit for bit to fused_rms of the query (key) heads followed by
    fused_rope."""
    H, HK, D = int(heads), int(kv_heads), int(head_dim)
    ok = (_is_dev(projected) and projected.dim() == 2 and projected.dtype == torch.bfloat16 and
          projected.stride(1) == 1 and H > 0 and HK > 0 and 0 < D <= 512 and
          projected.size(1) == 2 * (H + HK) * D and _positions_ok(positions, projected, projected.size(0)) and
          rotary > 0 and rotary % 2 == 0 and rotary <= D)
    for w in (q_norm, k_norm):
        ok = ok and (_is_dev(w) and w.device == projected.device and w.dtype == torch.bfloat16 and
                     w.is_contiguous() and w.numel() == D)
    if not ok:
        _fail(ERR_ARGUMENT, "Invalid Q/K norm + RoPE input")
    positions = positions.contiguous()
    T = projected.size(0)
    q = torch.empty((T, H, D), dtype=torch.bfloat16, device=projected.device)
    k = torch.empty((T, HK, D), dtype=torch.bfloat16, device=projected.device)
    check(lib().fp8lin_qk_norm_rope(_ptr(projected), projected.stride(0), _ptr(q_norm), _ptr(k_norm),
                                    _ptr(positions), _ptr(q), _ptr(k), T, H, HK, D, int(rotary), float(theta),
                                    int(height_section), int(width_section), float(eps), _stream(projected)))
    return q, k


def _workspace(nbytes, device):
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device) if nbytes else None


def vocabulary_candidates(logits, offset=0):
    """`at::Tensor vocabulary_candidates(logits, int64_t offset=0)` --
    src/dual_path.cu:79-85: per row {max value, argmax + offset} as doubles."""
    if not (_is_dev(logits) and logits.dtype == torch.bfloat16 and logits.dim() == 2 and
            logits.is_contiguous()):
        _fail(ERR_ARGUMENT, "Invalid vocabulary candidates")
    M, N = logits.shape
    out = torch.empty((M, 2), dtype=torch.float64, device=logits.device)
    nbytes = lib().fp8lin_vocab_candidates_workspace_bytes(M, N)
    ws = _workspace(nbytes, logits.device)
    check(lib().fp8lin_vocab_candidates(_ptr(logits), M, N, int(offset), _ptr(out), _ptr(ws), nbytes,
                                        _stream(logits)))
    return out


def merge_candidates(gathered):
    """`at::Tensor merge_candidates(at::Tensor gathered)` --
    src/dual_path.cu:86-92: [ranks, rows, 2] doubles -> [rows] int64 ids
    (-1 where a rank's candidate is not finite or not a valid id)."""
    if not (_is_dev(gathered) and gathered.dtype == torch.float64 and gathered.is_contiguous() and
            gathered.dim() == 3 and gathered.size(2) == 2):
        _fail(ERR_ARGUMENT, "Invalid gathered candidates")
    out = torch.empty(gathered.size(1), dtype=torch.int64, device=gathered.device)
    check(lib().fp8lin_merge_candidates(_ptr(gathered), gathered.size(0), gathered.size(1),
                                        _ptr(out), _stream(gathered)))
    return out


def linear_candidates(x, codes, scales, offset=0):
    """`vocabulary_candidates(fp8_linear(x, codes, scales), offset)` in one call
    (Engine::local_candidates, src/speculative.cpp:25-27)."""
    _check_x(x, "FP8 linear expects CUDA BF16 [M,K]")
    _check_codes(codes, x)
    sc = _scale_cols(scales, codes.size(0), codes.size(1))
    M, N, K = x.size(0), codes.size(0), codes.size(1)
    if not (M > 0 and N > 0 and K > 0):
        _fail(ERR_SHAPE, "Empty GEMM")
    out = torch.empty((M, 2), dtype=torch.float64, device=x.device)
    nbytes = lib().fp8lin_linear_candidates_workspace_bytes(M, N, K)
    ws = _workspace(nbytes, x.device)
    check(lib().fp8lin_linear_candidates(_ptr(x), _ptr(codes), _ptr(scales), sc, M, N, K,
                                         int(offset), _ptr(out), _ptr(ws), nbytes, _stream(x)))
    return out


def gen_weights(n, k, seed=0, tag=1, std=0.02, device="cuda"):
    """Synthetic block-FP8 weights on the device (codes [n,k] u8, scales
    [n, ceil(k/128)] f32)."""
    codes = torch.empty((n, k), dtype=torch.uint8, device=device)
    scales = torch.empty((n, (k + 127) // 128), dtype=torch.float32, device=device)
    check(lib().fp8lin_gen_weights(seed, tag, n, k, float(std), _ptr(codes), _ptr(scales),
                                   _stream(codes)))
    return codes, scales


def gen_activations(m, k, seed=0, tag=2, device="cuda"):
    x = torch.empty((m, k), dtype=torch.bfloat16, device=device)
    check(lib().fp8lin_gen_activations(seed, tag, m, k, _ptr(x), _stream(x)))
    return x


def gen_normal(n, seed=0, tag=1, first=0, device="cuda"):
    out = torch.empty(n, dtype=torch.float32, device=device)
    check(lib().fp8lin_gen_normal(seed, tag, first, n, _ptr(out), _stream(out)))
    return out


def stream_read(src, sink):
    check(lib().fp8lin_stream_read(_ptr(src), src.numel() * src.element_size(), _ptr(sink),
                                   _stream(src)))


def mfma_ceiling(iters, sink, clocks):
    """MFMA-ceiling probe: sink float32 [>=1], clocks int64 [2] (shader-clock
    and 100 MHz ticks of workgroup 0), both on the device."""
    check(lib().fp8lin_mfma_ceiling(int(iters), _ptr(sink), _ptr(clocks), _stream(sink)))


def decode_chain_workspace(nlinks, device):
    """A zeroed workspace for decode_chain with `nlinks` links (64-bit
    counters that never reset: word 0 counts waits that gave up, word 1 the
    chain's shape); one serves any number of calls of one chain shape on one
    stream.  Zero it again (or take another) for a chain of another shape."""
    return torch.zeros(lib().fp8lin_decode_chain_workspace_bytes(int(nlinks)), dtype=torch.uint8, device=device)


def decode_chain(links, workspace=None):
    """The one-row projections of one decode step in one launch
    (fp8lin_decode_chain; Engine::step's linear calls at one token,
    src/engine.cpp:401-421).  links: a sequence of
    (x, codes, scales, swiglu, after): x a BF16 [1, K] tensor, or the index of
    an earlier link whose output it is (then `after` defaults to that index);
    after: an earlier link to wait for before x is read, or -1.  Returns the
    outputs, each equal to fp8_linear (linear_swiglu with swiglu) of its link
    bit for bit."""
    from ._lib import CHAIN_MAX_LINKS, ChainLink
    n = len(links)
    if not 1 <= n <= CHAIN_MAX_LINKS:
        _fail(ERR_SHAPE, f"decode chain: 1 to {CHAIN_MAX_LINKS} links")
    recs = (ChainLink * n)()
    outs = []
    for i, link in enumerate(links):
        x, codes, scales = link[0], link[1], link[2]
        swiglu = bool(link[3]) if len(link) > 3 else False
        after = link[4] if len(link) > 4 and link[4] is not None else (x if isinstance(x, int) else -1)
        if isinstance(x, int):
            if not 0 <= x < i:
                _fail(ERR_ARGUMENT, "decode chain: x must name an earlier link")
            x = outs[x]
        _check_x(x, "decode chain: x must be a CUDA BF16 [1,K] tensor")
        _check_codes(codes, x)
        sc = _scale_cols(scales, codes.size(0), codes.size(1))
        if x.size(0) != 1:
            _fail(ERR_SHAPE, "decode chain: one activation row per link")
        N = codes.size(0)
        y = torch.empty((1, N // 2 if swiglu else N), dtype=torch.bfloat16, device=x.device)
        outs.append(y)
        r = recs[i]
        r.codes, r.scales, r.scale_cols = codes.data_ptr(), scales.data_ptr(), sc
        r.N, r.K = N, codes.size(1)
        r.x, r.y = x.data_ptr(), y.data_ptr()
        r.swiglu, r.after = int(swiglu), int(after)
    dev = outs[0].device
    if workspace is None:
        workspace = decode_chain_workspace(n, dev)
    check(lib().fp8lin_decode_chain(recs, n, _ptr(workspace), workspace.numel(), _stream(outs[0])))
    return outs
