"""fp8lin: MI355X (gfx950) block-FP8 linear layers.

Python host mirror over the C ABI of include/fp8lin.h.  The kernels live in
a100-vision-infer_amd/csrc (HIP); this package only validates tensors, allocates
outputs and passes pointers and torch's current stream.
"""
from ._lib import (EXPORTED, LIB_PATH, Fp8linError, LinearOptions, Weight, check, lib)  # noqa: F401
from ._lib import (ERR_ARGUMENT, ERR_DEVICE, ERR_LAUNCH, ERR_SHAPE, ERR_UNSUPPORTED,  # noqa: F401
                   ERR_WORKSPACE, OK)
from ._lib import (PATH_BF16, PATH_CACHED_BF16, PATH_DEQUANT_GEMM, PATH_FP8_GEMM,  # noqa: F401
                   PATH_FP8_GEMV, PATH_SHARED_GEMV, PATH_TENSOR_SMALL)
from .ops import (add_bias, decode_chain, decode_chain_workspace, fp8_decode, fp8_linear, fp8_tensor_small, fused_rms, fused_rope, fused_swiglu,  # noqa: F401
                  gemm_bf16, gen_activations, gen_normal, gen_weights, linear_candidates,
                  linear_swiglu, merge_candidates, mfma_ceiling, qk_norm_rope, reduce_residual_rms, residual_rms,
                  small_linear_shared, stream_read, tilelang_fp8_small, vocabulary_candidates)
from .engine import LinearEngine, StoredWeight  # noqa: F401
from .artifact import load_linear_engine, read_manifest, read_tensor  # noqa: F401
