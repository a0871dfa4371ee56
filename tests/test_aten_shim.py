"""The compiled LibTorch shim (a100-vision-infer_amd/aten/avi_ops.cpp) loads
without a GPU, exports the reference's avi:: linear-path operators and
rejects host tensors with the reference's TORCH_CHECK messages
(src/optimized.cu:62,72-74, src/kernels.cu:18, src/fp8_tensor.cu:54,
src/deep_kernels.cu:135, src/dual_path.cu:69,80,87, src/optimized.cu:78)."""
import pytest
import torch

NAMES = ["fp8_decode", "fp8_linear", "fp8_tensor_small", "tilelang_fp8_small", "small_linear_shared",
         "fused_swiglu", "fused_rms", "fused_rope", "residual_rms", "vocabulary_candidates", "merge_candidates"]


@pytest.fixture(scope="module")
def avi(fp8lin):
    from fp8lin import aten
    return aten.load()


def test_exports(avi):
    for n in NAMES:
        assert callable(getattr(avi, n)), n


@pytest.mark.parametrize("call,msg", [
    (lambda a, t: a.fp8_decode(t["codes"], t["scales"]), "FP8 codes must be contiguous CUDA uint8 matrix"),
    (lambda a, t: a.fp8_linear(t["x"], t["codes"], t["scales"]), "FP8 linear expects CUDA BF16 [M,K]"),
    (lambda a, t: a.fp8_tensor_small(t["x"], t["codes"], t["scales"], 1), "Invalid Ampere FP8 W8A16 geometry/dtype"),
    (lambda a, t: a.tilelang_fp8_small(t["x"], t["codes"], t["scales"], 1), "Invalid TileLang FP8 W8A16 inputs"),
    (lambda a, t: a.small_linear_shared(t["x"], t["codes"], t["scales"]), "Invalid shared GEMV inputs"),
    (lambda a, t: a.fused_swiglu(t["x"]), "Invalid SwiGLU input"),
    (lambda a, t: a.fused_rms(t["x"], t["w"], 1e-6, True), "Invalid RMS input"),
    (lambda a, t: a.fused_rope(t["x"].view(2, 4, 64), t["p"], 32, 1e4, 4, 4), "Invalid RoPE input"),
    (lambda a, t: a.residual_rms(t["x"], t["x"], t["w"], 1e-6), "Invalid fused residual RMS input"),
    (lambda a, t: a.vocabulary_candidates(t["x"], 0), "Invalid vocabulary candidates"),
    (lambda a, t: a.merge_candidates(t["g"]), "Invalid gathered candidates"),
])
def test_rejects_host_tensors(avi, call, msg):
    t = {"x": torch.zeros(2, 256, dtype=torch.bfloat16), "codes": torch.zeros(16, 256, dtype=torch.uint8),
         "scales": torch.ones(16, 2), "w": torch.zeros(256, dtype=torch.bfloat16),
         "g": torch.zeros(2, 3, 2, dtype=torch.float64), "p": torch.zeros(3, 2, dtype=torch.int64)}
    with pytest.raises(RuntimeError) as e:
        call(avi, t)
    assert msg in str(e.value)
