"""ctypes loader for libfp8lin.so (the C ABI of include/fp8lin.h).

The library is built in-tree by a100-vision-infer_amd/build.py (or
__graft_entry__.build()).  There is no fallback: if the library is missing,
every entry point raises.
"""
import ctypes
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libfp8lin.so")

OK = 0
ERR_SHAPE = 1
ERR_ARGUMENT = 2
ERR_UNSUPPORTED = 3
ERR_WORKSPACE = 4
ERR_LAUNCH = 5
ERR_DEVICE = 6

PATH_TENSOR_SMALL = 1
PATH_SHARED_GEMV = 2
PATH_CACHED_BF16 = 3
PATH_FP8_GEMV = 4
PATH_FP8_GEMM = 5
PATH_DEQUANT_GEMM = 6
PATH_BF16 = 7

EXPORTED = [
    "fp8lin_version", "fp8lin_last_error", "fp8lin_init", "fp8lin_decode", "fp8lin_linear",
    "fp8lin_linear_ld", "fp8lin_linear_swiglu", "fp8lin_swiglu", "fp8lin_linear_shared",
    "fp8lin_tensor_small_workspace_bytes", "fp8lin_tensor_small", "fp8lin_gemm_bf16",
    "fp8lin_engine_linear_workspace_bytes", "fp8lin_engine_linear",
    "fp8lin_engine_linear_groups", "fp8lin_gen_weights", "fp8lin_gen_activations",
    "fp8lin_gen_normal", "fp8lin_stream_read", "fp8lin_mfma_ceiling",
    "fp8lin_rms", "fp8lin_residual_rms", "fp8lin_vocab_candidates_workspace_bytes",
    "fp8lin_vocab_candidates", "fp8lin_merge_candidates",
    "fp8lin_linear_candidates_workspace_bytes", "fp8lin_linear_candidates",
    "fp8lin_engine_linear_candidates_workspace_bytes", "fp8lin_engine_linear_candidates",
    "fp8lin_reduce_residual_rms",
    "fp8lin_rope",
    "fp8lin_qk_norm_rope",
    "fp8lin_add_bias",
    "fp8lin_linear_candidates_static",
    "fp8lin_linear_swiglu_workspace_bytes", "fp8lin_linear_swiglu_ws",
    "fp8lin_linear_workspace_bytes", "fp8lin_linear_ws",
    "fp8lin_decode_chain_workspace_bytes", "fp8lin_decode_chain",
]


class Fp8linError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"fp8lin error {code}: {message}")
        self.code = code


class Weight(ctypes.Structure):
    """struct fp8lin_weight"""
    _fields_ = [("data", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("scale_cols", ctypes.c_int64), ("cached_bf16", ctypes.c_void_p),
                ("N", ctypes.c_int64), ("K", ctypes.c_int64), ("bias", ctypes.c_void_p)]


class ChainLink(ctypes.Structure):
    """struct fp8lin_chain_link"""
    _fields_ = [("codes", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("scale_cols", ctypes.c_int64),
                ("N", ctypes.c_int64), ("K", ctypes.c_int64), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("swiglu", ctypes.c_int), ("after", ctypes.c_int)]


CHAIN_MAX_LINKS = 8


class LinearOptions(ctypes.Structure):
    """struct fp8lin_linear_options (the EngineOptions linear flags,
    include/avi/engine.h:16 of the reference)."""
    _fields_ = [("optimized", ctypes.c_int), ("vector_gemv", ctypes.c_int),
                ("cublas_prefill", ctypes.c_int), ("fp8_tensor_small", ctypes.c_int),
                ("fp8_tensor_split", ctypes.c_int), ("tilelang_fp8", ctypes.c_int),
                ("multi_token_gemv", ctypes.c_int), ("shared_gemv_fp8", ctypes.c_int)]

    def __init__(self, optimized=True, vector_gemv=False, cublas_prefill=False,
                 fp8_tensor_small=False, fp8_tensor_split=1, tilelang_fp8=False,
                 multi_token_gemv=False, shared_gemv_fp8=False):
        super().__init__(int(optimized), int(vector_gemv), int(cublas_prefill),
                         int(fp8_tensor_small), int(fp8_tensor_split), int(tilelang_fp8),
                         int(multi_token_gemv), int(shared_gemv_fp8))


_lib = None


def lib():
    """Load libfp8lin.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"fp8lin native library not built ({LIB_PATH}); run "
                           "`python a100-vision-infer_amd/build.py`")
    L = ctypes.CDLL(LIB_PATH)
    vp, i64, i32, u64, u32 = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                              ctypes.c_uint64, ctypes.c_uint32)
    sz = ctypes.c_size_t
    sig = {
        "fp8lin_version": (i32, []),
        "fp8lin_last_error": (ctypes.c_char_p, []),
        "fp8lin_init": (i32, []),
        "fp8lin_decode": (i32, [vp, vp, i64, vp, i64, i64, vp]),
        "fp8lin_linear": (i32, [vp, vp, vp, i64, vp, i64, i64, i64, i32, vp]),
        "fp8lin_linear_ld": (i32, [vp, vp, vp, i64, vp, i64, i64, i64, i64, i32, vp]),
        "fp8lin_linear_workspace_bytes": (sz, [i64, i64, i64]),
        "fp8lin_decode_chain_workspace_bytes": (sz, [i32]),
        "fp8lin_decode_chain": (i32, [ctypes.POINTER(ChainLink), i32, vp, sz, vp]),
        "fp8lin_linear_ws": (i32, [vp, vp, vp, i64, vp, i64, i64, i64, i32, vp, sz, vp]),
        "fp8lin_linear_swiglu": (i32, [vp, vp, vp, i64, vp, i64, i64, i64, vp]),
        "fp8lin_swiglu": (i32, [vp, vp, i64, i64, vp]),
        "fp8lin_linear_swiglu_workspace_bytes": (sz, [i64, i64, i64]),
        "fp8lin_linear_swiglu_ws": (i32, [vp, vp, vp, i64, vp, i64, i64, i64, vp, sz, vp]),
        "fp8lin_add_bias": (i32, [vp, i64, vp, i64, i64, vp]),
        "fp8lin_linear_shared": (i32, [vp, vp, vp, i64, vp, i64, i64, i64, vp]),
        "fp8lin_tensor_small_workspace_bytes": (sz, [i64, i64, i32]),
        "fp8lin_tensor_small": (i32, [vp, vp, vp, vp, i64, i64, i64, i32, vp, sz, vp]),
        "fp8lin_gemm_bf16": (i32, [vp, vp, vp, i64, i64, i64, i64, vp]),
        "fp8lin_engine_linear_workspace_bytes": (sz, [ctypes.POINTER(LinearOptions),
                                                      ctypes.POINTER(Weight), i64]),
        "fp8lin_engine_linear": (i32, [ctypes.POINTER(LinearOptions), ctypes.POINTER(Weight), vp,
                                       i64, vp, i64, vp, sz, ctypes.POINTER(ctypes.c_int), vp]),
        "fp8lin_engine_linear_groups": (i32, [ctypes.POINTER(LinearOptions),
                                              ctypes.POINTER(Weight), i32, vp, i64, vp, i64, vp,
                                              sz, vp]),
        "fp8lin_gen_weights": (i32, [u64, u32, i64, i64, ctypes.c_float, vp, vp, vp]),
        "fp8lin_gen_activations": (i32, [u64, u32, i64, i64, vp, vp]),
        "fp8lin_gen_normal": (i32, [u64, u32, u64, i64, vp, vp]),
        "fp8lin_stream_read": (i32, [vp, sz, vp, vp]),
        "fp8lin_mfma_ceiling": (i32, [i64, vp, vp, vp]),
        "fp8lin_rms": (i32, [vp, vp, vp, i64, i64, ctypes.c_double, i32, vp]),
        "fp8lin_residual_rms": (i32, [vp, vp, vp, vp, vp, i64, i64, ctypes.c_double, i32, vp]),
        "fp8lin_reduce_residual_rms": (i32, [vp, vp, i64, vp, vp, vp, i64, i64, ctypes.c_double, i32, vp]),
        "fp8lin_rope": (i32, [vp, vp, vp, i64, i64, i64, i64, ctypes.c_double, i64, i64, vp]),
        "fp8lin_qk_norm_rope": (i32, [vp, i64, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ctypes.c_double, i64,
                                      i64, ctypes.c_double, vp]),
        "fp8lin_vocab_candidates_workspace_bytes": (sz, [i64, i64]),
        "fp8lin_vocab_candidates": (i32, [vp, i64, i64, i64, vp, vp, sz, vp]),
        "fp8lin_merge_candidates": (i32, [vp, i64, i64, vp, vp]),
        "fp8lin_linear_candidates_workspace_bytes": (sz, [i64, i64, i64]),
        "fp8lin_linear_candidates": (i32, [vp, vp, vp, i64, i64, i64, i64, i64, vp, vp, sz, vp]),
        "fp8lin_linear_candidates_static": (i32, [vp, vp, vp, i64, i64, i64, i64, i64, vp, vp]),
        "fp8lin_engine_linear_candidates_workspace_bytes": (sz, [ctypes.POINTER(LinearOptions),
                                                                 ctypes.POINTER(Weight), i64]),
        "fp8lin_engine_linear_candidates": (i32, [ctypes.POINTER(LinearOptions), ctypes.POINTER(Weight), vp,
                                                  i64, i64, vp, vp, sz, ctypes.POINTER(ctypes.c_int), vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    # Prepare the current device now (its properties and the device address
    # of the library's static scratch), outside any graph capture a caller
    # may start later.  Without a GPU (or on another architecture) this fails
    # here without effect, and every entry point reports it when called.
    L.fp8lin_init()
    _lib = L
    return L


def check(rc):
    if rc != OK:
        msg = lib().fp8lin_last_error().decode(errors="replace")
        raise Fp8linError(rc, msg)
    return rc
