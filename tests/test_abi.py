"""C ABI checks that need no GPU: the library loads, exports every function
include/fp8lin.h declares, rejects bad arguments with the documented status
codes before touching a device, and chooses Engine::linear's branch in the
reference's order (src/engine.cpp:206-237)."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "fp8lin.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fp8lin_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported(fp8lin):
    names = header_functions()
    assert len(names) >= 20
    L = fp8lin.lib()
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/fp8lin.h but not exported"
    assert sorted(set(fp8lin.EXPORTED) | {"fp8lin_engine_linear_path"}) == names


def test_version_and_error_string(fp8lin):
    L = fp8lin.lib()
    assert L.fp8lin_version() == 200
    assert isinstance(L.fp8lin_last_error(), bytes)


# Fake, 16-byte aligned, never dereferenced: every call below fails validation
# before any device access.
P = ctypes.c_void_p(0x10000)


@pytest.mark.parametrize("args,code", [
    ((None, P, P, 1, P, 1, 8, 8, 0, None), 2),            # null x
    ((P, P, P, 1, P, 0, 8, 8, 0, None), 1),               # M == 0 ("Empty GEMM")
    ((P, P, P, 1, P, 1, 8, -1, 0, None), 1),              # K < 0
    ((P, P, P, 3, P, 1, 8, 256, 0, None), 2),             # scale_cols not in {1, 2}
    ((P, P, None, 1, P, 1, 8, 256, 0, None), 2),          # null scales
])
def test_linear_validation(fp8lin, args, code):
    L = fp8lin.lib()
    assert L.fp8lin_linear(*args) == code
    assert L.fp8lin_last_error()


@pytest.mark.parametrize("m,n,k,split,ws,code", [
    (1, 16, 128, 1, None, 1),      # M < 2
    (9, 16, 128, 1, None, 1),      # M > 8
    (4, 16, 130, 1, None, 1),      # K % 128 != 0
    (4, 16, 128, 2, None, 2),      # split not in {1, 4}
])
def test_tensor_small_validation(fp8lin, m, n, k, split, ws, code):
    L = fp8lin.lib()
    assert L.fp8lin_tensor_small(P, P, P, P, m, n, k, split, ws, 0, None) == code


def test_workspace_sizes(fp8lin):
    L = fp8lin.lib()
    assert L.fp8lin_tensor_small_workspace_bytes(4, 100, 1) == 0
    assert L.fp8lin_tensor_small_workspace_bytes(4, 100, 4) == 0  # split 4 sums in-kernel


def test_shared_and_swiglu_validation(fp8lin):
    L = fp8lin.lib()
    assert L.fp8lin_linear_shared(P, P, None, 1, P, 9, 8, 8, None) == 1   # 1..8 rows
    assert L.fp8lin_linear_shared(P, P, P, 5, P, 2, 8, 300, None) == 2    # bad scale cols
    assert L.fp8lin_linear_swiglu(P, P, P, 1, P, 1, 7, 8, None) == 1      # odd N
    assert L.fp8lin_swiglu(P, P, -1, 4, None) == 1
    assert L.fp8lin_swiglu(P, P, 0, 4, None) == 0                         # empty: no-op
    assert L.fp8lin_decode(P, P, 1, P, 0, 5, None) == 0                   # empty: no-op
    assert L.fp8lin_decode(P, P, 7, P, 4, 256, None) == 2


def test_rope_validation(fp8lin):
    """src/optimized.cu:78 preconditions (rotary even, 0 < rotary <= D) and the
    kernels' own limits (D <= 4096; D <= 512 and a row stride covering the
    head layout for the fused Q/K epilogue) as status codes."""
    L = fp8lin.lib()
    assert L.fp8lin_rope(P, P, P, 0, 12, 256, 64, 1e7, 11, 10, None) == 0          # no tokens: no-op
    assert L.fp8lin_rope(None, P, P, 1, 12, 256, 64, 1e7, 11, 10, None) == 2
    assert L.fp8lin_rope(P, None, P, 1, 12, 256, 64, 1e7, 11, 10, None) == 2
    assert L.fp8lin_rope(P, P, P, 1, 12, 256, 63, 1e7, 11, 10, None) == 2          # odd rotary
    assert L.fp8lin_rope(P, P, P, 1, 12, 256, 0, 1e7, 11, 10, None) == 2
    assert L.fp8lin_rope(P, P, P, 1, 12, 256, 258, 1e7, 11, 10, None) == 2         # rotary > D
    assert L.fp8lin_rope(P, P, P, 1, 12, 4098, 64, 1e7, 11, 10, None) == 1         # D limit
    assert L.fp8lin_rope(P, P, P, 1, 0, 256, 64, 1e7, 11, 10, None) == 1
    assert L.fp8lin_rope(P, P, P, 1 << 20, 1 << 12, 8, 8, 1e7, 11, 10, None) == 1  # 2^31 rows
    assert L.fp8lin_rope(P, P, P, 1, 4 * 65535 + 1, 8, 8, 1e7, 11, 10, None) == 1  # heads: 65535 groups of 4
    args = (12, 2, 256, 64, 1e7, 11, 10, 1e-6, None)
    ld = 2 * 14 * 256
    assert L.fp8lin_qk_norm_rope(P, ld, P, P, P, P, P, 0, *args) == 0              # no tokens: no-op
    assert L.fp8lin_qk_norm_rope(P, ld, None, P, P, P, P, 1, *args) == 2
    assert L.fp8lin_qk_norm_rope(P, ld, P, P, P, P, None, 1, *args) == 2
    assert L.fp8lin_qk_norm_rope(P, ld - 1, P, P, P, P, P, 1, *args) == 1          # stride below the layout
    assert L.fp8lin_qk_norm_rope(P, ld, P, P, P, P, P, 1, 12, 0, *args[2:]) == 1   # key heads
    assert L.fp8lin_qk_norm_rope(P, 4 * 14 * 576, P, P, P, P, P, 1, 12, 2, 576, 64, 1e7, 11, 10, 1e-6,
                                 None) == 1                                        # D <= 512
    assert L.fp8lin_qk_norm_rope(P, ld, P, P, P, P, P, 1, 12, 2, 256, 65, 1e7, 11, 10, 1e-6, None) == 2
    # query heads: H = -1 with H + HK > 0 must not reach the kernel
    assert L.fp8lin_qk_norm_rope(P, ld, P, P, P, P, P, 1, -1, 5, *args[2:]) == 1
    assert L.fp8lin_qk_norm_rope(P, ld, P, P, P, P, P, 1, 0, 2, *args[2:]) == 1


def test_epilogue_validation(fp8lin):
    """src/dual_path.cu:69-72,73-75,86-88 preconditions as status codes."""
    L = fp8lin.lib()
    assert L.fp8lin_rms(P, P, P, 0, 64, 1e-6, 1, None) == 0                 # no rows: no-op
    assert L.fp8lin_rms(None, P, P, 2, 64, 1e-6, 1, None) == 2
    assert L.fp8lin_rms(P, P, P, 2, 0, 1e-6, 1, None) == 1
    assert L.fp8lin_rms(P, P, P, 1 << 22, 64, 1e-6, 1, None) == 1          # grid rows
    assert L.fp8lin_rms(P, P, P, 0, 64, 0.0, 1, None) == 0                  # no rows: no-op, any eps
    assert L.fp8lin_residual_rms(P, P, P, P, P, 0, 64, 1e-6, 1, None) == 1  # numel() > 0
    assert L.fp8lin_residual_rms(P, None, P, P, P, 2, 64, 1e-6, 1, None) == 2
    assert L.fp8lin_residual_rms(P, P, P, P, P, 2, 64, 0.0, 1, None) == 2   # eps > 0
    assert L.fp8lin_residual_rms(P, P, P, P, P, 2, 64, float("nan"), 1, None) == 2
    assert L.fp8lin_residual_rms(P, P, P, P, P, 2, 64, float("inf"), 0, None) == 2
    ws = L.fp8lin_vocab_candidates_workspace_bytes(3, 10000)
    assert ws == 3 * 5 * 8                                                  # 5 chunks of 2048
    assert L.fp8lin_vocab_candidates(P, 0, 10, 0, P, P, ws, None) == 1      # M > 0
    assert L.fp8lin_vocab_candidates(P, 65536, 10, 0, P, P, 1 << 30, None) == 1
    assert L.fp8lin_vocab_candidates(P, 3, 10000, -1, P, P, ws, None) == 1  # offset >= 0
    assert L.fp8lin_vocab_candidates(P, 3, 10000, 2**31 - 10000, P, P, ws, None) == 1
    assert L.fp8lin_vocab_candidates(P, 3, 10000, 0, P, P, ws - 8, None) == 4
    assert L.fp8lin_vocab_candidates(P, 3, 10000, 0, P, None, ws, None) == 4
    assert L.fp8lin_vocab_candidates(P, 3, 10000, 0, None, P, ws, None) == 2
    assert L.fp8lin_vocab_candidates(None, 3, 10000, 0, P, P, ws, None) == 2
    assert L.fp8lin_merge_candidates(P, 9, 4, P, None) == 1                 # ranks <= 8
    assert L.fp8lin_merge_candidates(P, 0, 4, P, None) == 1
    assert L.fp8lin_merge_candidates(P, 2, 65536, P, None) == 1
    assert L.fp8lin_merge_candidates(None, 2, 4, P, None) == 2
    assert L.fp8lin_reduce_residual_rms(P, P, 0, P, P, P, 2, 64, 1e-6, 1, None) == 1   # 1..8 ranks
    assert L.fp8lin_reduce_residual_rms(P, P, 9, P, P, P, 2, 64, 1e-6, 1, None) == 1
    assert L.fp8lin_reduce_residual_rms(P, None, 2, P, P, P, 2, 64, 1e-6, 1, None) == 2
    assert L.fp8lin_reduce_residual_rms(P, P, 2, P, P, P, 2, 64, -1.0, 1, None) == 2


def test_linear_candidates_validation(fp8lin):
    L = fp8lin.lib()
    # The larger of the two candidate forms: the BF16 logits [M, N] padded to
    # 256 bytes, then one pair per 2048-column chunk; or, at M <= 2 (the GEMV
    # epilogue form), the workgroup pairs, at most one per 4 columns in 8 XCD
    # runs, padded to 256 bytes, then 16 slice pairs and a counter per row.
    def want(m, n):
        two_stage = (m * n * 2 + 255) // 256 * 256 + m * ((n + 2047) // 2048) * 8
        gemv = (m * ((n + 3) // 4 + 7) * 8 + 255) // 256 * 256 + m * 16 * 8 + m * 4
        return max(two_stage, gemv) if m <= 2 else two_stage
    assert L.fp8lin_linear_candidates_workspace_bytes(1, 1000, 256) == want(1, 1000) == 2304 + 132
    assert L.fp8lin_linear_candidates_workspace_bytes(16, 1000, 256) == want(16, 1000) == 32000 + 16 * 8
    assert L.fp8lin_linear_candidates_workspace_bytes(2, 75968, 5120) == want(2, 75968) == 303872 + 2 * 38 * 8
    assert L.fp8lin_linear_candidates_workspace_bytes(0, 1000, 256) == 0
    ws = L.fp8lin_linear_candidates_workspace_bytes(2, 1000, 256)
    assert L.fp8lin_linear_candidates(P, P, P, 1, 2, 1000, 256, 0, P, P, ws - 1, None) == 4
    assert L.fp8lin_linear_candidates(P, P, P, 3, 2, 1000, 256, 0, P, P, ws, None) == 2
    assert L.fp8lin_linear_candidates(P, P, P, 1, 2, 1000, 256, -5, P, P, ws, None) == 1
    assert L.fp8lin_linear_candidates(P, P, P, 1, 2, 1000, 256, 0, None, P, ws, None) == 2
    assert L.fp8lin_linear_candidates(P, P, P, 1, 0, 1000, 256, 0, P, P, ws, None) == 1


def test_linear_candidates_static_validation(fp8lin):
    """The allocation-free head + candidates: the checks of
    fp8lin_linear_candidates, and sizes beyond the static scratch
    (FP8LIN_STATIC_SCRATCH_BYTES = 4 MiB of logits and pairs) refused before
    any device work."""
    L = fp8lin.lib()
    assert L.fp8lin_linear_candidates_static(None, P, P, 1, 2, 1000, 256, 0, P, None) == 2
    assert L.fp8lin_linear_candidates_static(P, P, P, 3, 2, 1000, 256, 0, P, None) == 2
    assert L.fp8lin_linear_candidates_static(P, P, P, 1, 2, 1000, 256, -5, P, None) == 1
    assert L.fp8lin_linear_candidates_static(P, P, P, 1, 2, 1000, 256, 0, None, None) == 2
    assert L.fp8lin_linear_candidates_static(P, P, P, 1, 0, 1000, 256, 0, P, None) == 1
    limit = 4 << 20
    assert L.fp8lin_linear_candidates_workspace_bytes(8, 261632, 256) == limit
    assert L.fp8lin_linear_candidates_workspace_bytes(8, 261633, 256) > limit
    assert L.fp8lin_linear_candidates_static(P, P, P, 1, 8, 261633, 256, 0, P, None) == fp8lin.ERR_UNSUPPORTED
    assert L.fp8lin_linear_candidates_static(P, P, P, 1, 1, 2093057, 256, 0, P, None) == fp8lin.ERR_UNSUPPORTED
    assert b"FP8LIN_STATIC_SCRATCH_BYTES" in L.fp8lin_last_error()


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device error path")
def test_no_device_is_reported(fp8lin):
    L = fp8lin.lib()
    assert L.fp8lin_init() == fp8lin.ERR_DEVICE


def _weight(fp8lin, n=256, k=512, scales=True, scale_cols=None, cached=False):
    w = fp8lin.Weight()
    w.data = 0x10000
    w.scales = 0x20000 if scales else None
    w.scale_cols = scale_cols if scale_cols is not None else (k + 127) // 128
    w.cached_bf16 = 0x30000 if cached else None
    w.N, w.K = n, k
    return w


def _path(fp8lin, opt, w, rows):
    return fp8lin.lib().fp8lin_engine_linear_path(ctypes.byref(opt), ctypes.byref(w), rows)


def test_engine_decision_table(fp8lin):
    F, O = fp8lin, fp8lin.LinearOptions
    w = _weight(F)
    assert _path(F, O(), w, 1) == F.PATH_FP8_GEMV
    assert _path(F, O(), w, 8) == F.PATH_FP8_GEMV
    assert _path(F, O(), w, 9) == F.PATH_FP8_GEMM
    assert _path(F, O(cublas_prefill=True), w, 9) == F.PATH_DEQUANT_GEMM
    assert _path(F, O(cublas_prefill=True), w, 8) == F.PATH_FP8_GEMV
    assert _path(F, O(optimized=False), w, 1) == F.PATH_DEQUANT_GEMM
    # tensor-small precedes everything for rows 2..8 with block scales, K%128 == 0
    assert _path(F, O(fp8_tensor_small=True, multi_token_gemv=True), w, 4) == F.PATH_TENSOR_SMALL
    assert _path(F, O(fp8_tensor_small=True), w, 1) == F.PATH_FP8_GEMV
    assert _path(F, O(fp8_tensor_small=True), _weight(F, k=500), 4) == F.PATH_FP8_GEMV
    assert _path(F, O(fp8_tensor_small=True), _weight(F, scale_cols=1), 4) == F.PATH_FP8_GEMV
    assert _path(F, O(tilelang_fp8=True), _weight(F, n=250), 4) == F.PATH_FP8_GEMV
    assert _path(F, O(tilelang_fp8=True), _weight(F, n=256), 4) == F.PATH_TENSOR_SMALL
    # multi-token GEMV for rows 2..8, then the cache for rows > 1
    assert _path(F, O(multi_token_gemv=True), w, 2) == F.PATH_SHARED_GEMV
    assert _path(F, O(multi_token_gemv=True), w, 9) == F.PATH_FP8_GEMM
    wc = _weight(F, cached=True)
    assert _path(F, O(), wc, 2) == F.PATH_CACHED_BF16
    assert _path(F, O(), wc, 1) == F.PATH_FP8_GEMV
    assert _path(F, O(), _weight(F, scales=False), 4) == F.PATH_BF16


SLOT = 256 * 256 * 4  # one FP32 partial of a 256-row tile
SLOT128 = 128 * 256 * 4  # of a 128-row tile (M <= 128)


def test_engine_splitk_workspace(fp8lin):
    """FP8 GEMM branch on a 256-CU device: K-split partials (one BM x 256 FP32
    slot per split tile and K range; BM = 128 rows for M <= 128, else 256) when the tiles number at most half the
    CUs (every tile, min(256 / T, K / 256, 8) ranges) or leave a last round
    on at most half of them (those tiles, min(256 / R, K / 256, 8))."""
    F, O = fp8lin, fp8lin.LinearOptions

    def ws(n, k, rows, **kw):
        w = _weight(F, n=n, k=k, **kw)
        return F.lib().fp8lin_engine_linear_workspace_bytes(ctypes.byref(O()), ctypes.byref(w), rows)
    assert ws(7168, 5120, 512) == 56 * 4 * SLOT          # QKV-gate, 56 tiles
    assert ws(5120, 8704, 512) == 40 * 6 * SLOT          # down, 40 tiles
    assert ws(7168, 5120, 1024) == 112 * 2 * SLOT        # 112 tiles
    assert ws(17408, 5120, 512) == 0                     # 136 tiles: no split
    assert ws(17408, 5120, 1024) == 16 * 8 * SLOT        # 272 = 256 + 16: the 16 tail tiles
    assert ws(17408, 5120, 4096) == 64 * 4 * SLOT        # 1088 = 4 * 256 + 64
    assert ws(17408, 5120, 2560) == 0                    # 680 = 2 * 256 + 168: last round over half
    assert ws(75968, 5120, 512) == 82 * 3 * SLOT         # output head: 594 = 2 * 256 + 82
    assert ws(22784, 512, 1024) == 100 * 2 * SLOT        # 356 = 256 + 100, K / 256 = 2
    assert ws(384, 512, 20) == 2 * 2 * SLOT128           # K / 256 = 2 caps the splits; 128-row tiles
    assert ws(7168, 5120, 128) == 28 * 8 * SLOT128       # M <= 128: one row of 128-row tiles
    assert ws(7168, 5120, 129) == 28 * 8 * SLOT          # M > 128: 256-row tiles
    assert ws(384, 256, 20) == 0                         # one 256-K chunk
    assert ws(384, 640, 20) == 0                         # K % 256 != 0: general GEMM
    assert ws(7168, 5120, 8) == 0                        # GEMV rows
    assert ws(256, 5120, 512) == 0                       # 256 weight rows or fewer: the GEMV's prefill form


def test_linear_swiglu_workspace(fp8lin):
    """The fused gate/up + SwiGLU splits by SwiGLU tiles (128 output pairs)."""
    L = fp8lin.lib()
    assert L.fp8lin_linear_swiglu_workspace_bytes(8, 17408, 5120) == 0        # GEMV rows
    assert L.fp8lin_linear_swiglu_workspace_bytes(512, 17408, 5120) == 0      # 136 tiles
    assert L.fp8lin_linear_swiglu_workspace_bytes(1024, 17408, 5120) == 16 * 8 * SLOT
    assert L.fp8lin_linear_swiglu_workspace_bytes(4096, 17408, 5120) == 64 * 4 * SLOT
    assert L.fp8lin_linear_swiglu_workspace_bytes(3913, 17408, 5120) == 64 * 4 * SLOT
    assert L.fp8lin_linear_swiglu_workspace_bytes(64, 512, 512) == 2 * 2 * SLOT128
    assert L.fp8lin_linear_swiglu_workspace_bytes(64, 511, 512) == 0          # odd N
    n = L.fp8lin_linear_swiglu_workspace_bytes(1024, 17408, 5120)
    assert L.fp8lin_linear_swiglu_ws(P, P, P, 40, P, 1024, 17408, 5120, P, n - 16, None) == 4
    assert L.fp8lin_linear_swiglu_ws(P, P, P, 40, P, 1024, 17407, 5120, P, n, None) == 1


def test_engine_option_consistency(fp8lin):
    """The option combinations the reference's Engine constructor rejects
    (src/engine.cpp:78,81) are argument errors; the queries return 0."""
    F, O = fp8lin, fp8lin.LinearOptions
    L = F.lib()
    w = _weight(F)
    for opt in (O(fp8_tensor_small=True, tilelang_fp8=True), O(fp8_tensor_small=True, optimized=False),
                O(tilelang_fp8=True, optimized=False), O(fp8_tensor_split=2)):
        assert _path(F, opt, w, 4) == 0
        assert L.fp8lin_engine_linear_workspace_bytes(ctypes.byref(opt), ctypes.byref(w), 512) == 0
        assert L.fp8lin_engine_linear_candidates_workspace_bytes(ctypes.byref(opt), ctypes.byref(w), 4) == 0
        rc = L.fp8lin_engine_linear(ctypes.byref(opt), ctypes.byref(w), P, 4, P, 256, None, 0, None, None)
        assert rc == F.ERR_ARGUMENT
        rc = L.fp8lin_engine_linear_candidates(ctypes.byref(opt), ctypes.byref(w), P, 4, 0, P, P, 1 << 20,
                                               None, None)
        assert rc == F.ERR_ARGUMENT
    # optimized=False alone stays valid (the dequant-then-GEMM branch)
    assert _path(F, O(optimized=False), w, 4) == F.PATH_DEQUANT_GEMM


def test_bias_validation(fp8lin):
    L = fp8lin.lib()
    assert L.fp8lin_add_bias(P, 8, P, 0, 8, None) == 0      # no rows: no-op
    assert L.fp8lin_add_bias(P, 8, P, 4, 0, None) == 0      # no columns: no-op
    assert L.fp8lin_add_bias(None, 8, P, 4, 8, None) == 2
    assert L.fp8lin_add_bias(P, 8, None, 4, 8, None) == 2
    assert L.fp8lin_add_bias(P, 7, P, 4, 8, None) == 1      # ldy < N
    assert L.fp8lin_add_bias(P, 8, P, -1, 8, None) == 1


def test_engine_validation(fp8lin):
    F = fp8lin
    L = F.lib()
    opt = F.LinearOptions(fp8_tensor_split=3)
    w = _weight(F)
    rc = L.fp8lin_engine_linear(ctypes.byref(opt), ctypes.byref(w), P, 2, P, 256, None, 0, None, None)
    assert rc == F.ERR_ARGUMENT
    opt = F.LinearOptions()
    rc = L.fp8lin_engine_linear(ctypes.byref(opt), ctypes.byref(w), P, 2, P, 100, None, 0, None, None)
    assert rc == F.ERR_SHAPE   # ldy < N
    w.scale_cols = 3
    rc = L.fp8lin_engine_linear(ctypes.byref(opt), ctypes.byref(w), P, 2, P, 256, None, 0, None, None)
    assert rc == F.ERR_ARGUMENT


def splitk_plan_bytes(m, n, k, cus=256):
    """K-split partials of the prefill GEMM plan (bm x 256 tiles, bm = 128 for
    m <= 128): every tile when the tiles number at most half the CUs, else
    the tiles of a last round on at most half of them; min(CUs / tiles,
    K / 256, 8) K ranges of one bm x 256 FP32 partial each."""
    bm = 128 if m <= 128 else 256
    tiles = -(-m // bm) * -(-n // 256)
    split = tiles if 2 * tiles <= cus else tiles % cus if tiles > cus and 2 * (tiles % cus) <= cus else 0
    s = min(cus // split, k // 256, 8) if split else 0
    return split * s * bm * 256 * 4 if s > 1 else 0


@pytest.mark.parametrize("m,n,k", [(512, 7168, 5120), (512, 5120, 8704), (64, 17408, 5120), (1024, 17408, 5120),
                                   (4096, 17408, 5120), (512, 17408, 5120), (512, 75968, 5120)])
def test_linear_workspace_bytes(fp8lin, m, n, k):
    """fp8lin_linear_ws's partials follow the engine branch's split plan (no
    GPU here: the plan assumes 256 CUs)."""
    L = fp8lin.lib()
    assert L.fp8lin_linear_workspace_bytes(m, n, k) == splitk_plan_bytes(m, n, k)


@pytest.mark.parametrize("m,n,k", [(1, 7168, 5120), (8, 5120, 8704), (16, 5120, 8704), (32, 7168, 5120),
                                   (64, 5120, 8704), (48, 7168, 5120), (512, 48, 5120), (0, 16, 16), (512, 7168, 0)])
def test_linear_workspace_bytes_none(fp8lin, m, n, k):
    """No partials where fp8_linear runs no GEMM tile (the decode GEMV, the
    small-M kernel for 9..32 rows and for 33..64 on weights of up to 32 rows
    per CU, the skinny kernel) or on empty shapes."""
    assert fp8lin.lib().fp8lin_linear_workspace_bytes(m, n, k) == 0


def test_linear_ws_validation(fp8lin):
    """fp8lin_linear_ws checks its workspace before touching a device."""
    L = fp8lin.lib()
    need = L.fp8lin_linear_workspace_bytes(512, 7168, 5120)
    assert need > 0
    assert L.fp8lin_linear_ws(P, P, P, 40, P, 512, 7168, 5120, 0, None, need, None) == fp8lin.ERR_WORKSPACE
    assert L.fp8lin_linear_ws(P, P, P, 40, P, 512, 7168, 5120, 0, P, need - 16, None) == fp8lin.ERR_WORKSPACE
    assert L.fp8lin_linear_ws(P, P, P, 40, P, 512, 7168, 5120, 0, ctypes.c_void_p(0x10008), need,
                              None) == fp8lin.ERR_WORKSPACE
    assert L.fp8lin_linear_ws(None, P, P, 40, P, 512, 7168, 5120, 0, P, need, None) == fp8lin.ERR_ARGUMENT
    assert L.fp8lin_linear_ws(P, P, P, 40, P, 0, 7168, 5120, 0, P, need, None) == fp8lin.ERR_SHAPE


def _chain(fp8lin, specs):
    """ChainLink records with fake (never dereferenced) pointers:
    specs = [(N, K, scale_cols, swiglu, after)]."""
    recs = (fp8lin._lib.ChainLink * len(specs))()
    for r, (n, k, sc, sw, after) in zip(recs, specs):
        r.codes = r.scales = r.x = r.y = 0x10000
        r.scale_cols, r.N, r.K, r.swiglu, r.after = sc, n, k, sw, after
    return recs


@pytest.mark.parametrize("specs,ws,code", [
    ([], 256, 1),                                                # no links
    ([(16, 16, 1, 0, -1)] * 9, 256, 1),                          # more than FP8LIN_CHAIN_MAX_LINKS
    ([(16, 16, 1, 0, 0)], 256, 2),                               # a link waits for itself
    ([(16, 16, 1, 0, -1), (16, 16, 1, 0, 1)], 256, 2),           # ... or a later link
    ([(16, 16, 1, 0, -1), (16, 16, 1, 0, -2)], 256, 2),          # after < -1
    ([(16, 16, 3, 0, -1)], 256, 2),                              # scale_cols not in {1, ceil(K/128)}
    ([(16, 24, 1, 0, -1)], 256, 3),                              # K % 16 != 0
    ([(16, 9232, 1, 0, -1)], 256, 3),                            # K > 9216
    ([(16, 5136, 1, 1, -1)], 256, 3),                            # SwiGLU with K > 5120
    ([(15, 512, 4, 1, -1)], 256, 3),                             # SwiGLU with N odd
    ([(0, 512, 4, 0, -1)], 256, 1),                              # N == 0
    ([(16, 512, 4, 0, -1)], 0, 4),                               # no workspace
    ([(16, 512, 4, 0, -1)] * 4, 256, 4),                         # workspace too small for 4 links
])
def test_decode_chain_validation(fp8lin, specs, ws, code):
    """fp8lin_decode_chain rejects bad chains before touching a device."""
    L = fp8lin.lib()
    recs = _chain(fp8lin, specs) if specs else (fp8lin._lib.ChainLink * 1)()
    assert L.fp8lin_decode_chain(recs, len(specs), P if ws else None, ws, None) == code
    assert L.fp8lin_last_error()


def test_decode_chain_workspace_bytes(fp8lin):
    L = fp8lin.lib()
    assert L.fp8lin_decode_chain_workspace_bytes(0) == 0
    assert L.fp8lin_decode_chain_workspace_bytes(9) == 0
    for n in range(1, 9):  # a 128-byte line for the timeouts, 256 lines of slot counters and 8 XCD words per link
        assert L.fp8lin_decode_chain_workspace_bytes(n) == (128 + n * (256 * 128 + 8 * 256) + 255) // 256 * 256
