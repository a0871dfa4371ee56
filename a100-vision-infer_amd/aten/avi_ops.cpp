// The reference's linear-path operators (namespace avi, include/avi/ops.h,
// include/avi/engine.h:13, include/avi/tilelang.h:11) implemented on ROCm
// LibTorch over the fp8lin C ABI: the binding a maintainer of the reference
// engine would link in place of optimized.cu, kernels.cu, fp8_tensor.cu,
// deep_kernels.cu and dual_path.cu's kernels.  Same names, argument meaning,
// output allocation and TORCH_CHECK preconditions; work goes to the current
// HIP stream of the input's device.  A pybind11 module exposes the same
// functions so tests can call them.
#include <torch/extension.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <climits>
#include <optional>
#include <cmath>
#include <utility>

#include "../../include/fp8lin.h"

namespace avi {
namespace {

// ROCm LibTorch reports HIP devices as device type "cuda"; its guards and
// streams for them are the ...MasqueradingAsCUDA forms.
using Guard = c10::hip::HIPGuardMasqueradingAsCUDA;
void* stream_of(const at::Tensor& t) {
    return reinterpret_cast<void*>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}
const uint16_t* bf(const at::Tensor& t) { return reinterpret_cast<const uint16_t*>(t.data_ptr<at::BFloat16>()); }
uint16_t* bf_out(at::Tensor& t) { return reinterpret_cast<uint16_t*>(t.data_ptr<at::BFloat16>()); }
void check(int rc) { TORCH_CHECK(rc == FP8LIN_OK, fp8lin_last_error()); }

// src/optimized.cu:64, src/kernels.cu:19
bool scales_ok(const at::Tensor& s, const at::Tensor& codes) {
    return s.is_cuda() && s.device() == codes.device() && s.scalar_type() == at::kFloat && s.is_contiguous() &&
           (s.dim() == 1 ? s.numel() == codes.size(0)
                         : (s.dim() == 2 && s.size(0) == codes.size(0) && s.size(1) == (codes.size(1) + 127) / 128));
}
int64_t scale_cols(const at::Tensor& s) { return s.dim() == 1 ? 1 : s.size(1); }

// src/fp8_tensor.cu:54-60 and src/tilelang.cpp:95-99
void check_tensor_small(const at::Tensor& x, const at::Tensor& codes, const at::Tensor& scales, int split, bool n16,
                        const char* what) {
    TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kBFloat16 && x.dim() == 2 && x.is_contiguous() &&
                    codes.is_cuda() && codes.device() == x.device() && codes.scalar_type() == at::kByte &&
                    codes.dim() == 2 && codes.is_contiguous() && scales.is_cuda() && scales.device() == x.device() &&
                    scales.scalar_type() == at::kFloat && scales.dim() == 2 && scales.is_contiguous() &&
                    x.size(0) >= 2 && x.size(0) <= 8 && x.size(1) > 0 && x.size(1) == codes.size(1) &&
                    x.size(1) % 128 == 0 && codes.size(0) > 0 && scales.size(0) == codes.size(0) &&
                    scales.size(1) == x.size(1) / 128 && (split == 1 || split == 4) &&
                    (!n16 || codes.size(0) % 16 == 0),
                what);
}

at::Tensor run_tensor_small(const at::Tensor& x, const at::Tensor& codes, const at::Tensor& scales, int split) {
    Guard guard(x.device());
    const int64_t M = x.size(0), N = codes.size(0), K = x.size(1);
    auto y = at::empty({M, N}, x.options());
    const size_t ws = fp8lin_tensor_small_workspace_bytes(M, N, split);
    at::Tensor work;
    if (ws) work = at::empty({(int64_t)ws}, x.options().dtype(at::kByte));
    check(fp8lin_tensor_small(bf(x), codes.data_ptr<uint8_t>(), scales.data_ptr<float>(), bf_out(y), M, N, K, split,
                              ws ? work.data_ptr() : nullptr, ws, stream_of(x)));
    return y;
}

}  // namespace

// include/avi/engine.h:13, src/kernels.cu:17-27
at::Tensor fp8_decode(at::Tensor q, at::Tensor s) {
    TORCH_CHECK(q.is_cuda() && q.scalar_type() == at::kByte && q.dim() == 2 && q.is_contiguous(),
                "FP8 codes must be contiguous CUDA uint8 matrix");
    TORCH_CHECK(scales_ok(s, q), "Invalid FP8 row scales");
    Guard guard(q.device());
    auto y = at::empty(q.sizes(), q.options().dtype(at::kBFloat16));
    if (q.numel())
        check(fp8lin_decode(q.data_ptr<uint8_t>(), s.data_ptr<float>(), scale_cols(s), bf_out(y), q.size(0),
                            q.size(1), stream_of(q)));
    return y;
}

// include/avi/ops.h:18, src/optimized.cu:61-70
at::Tensor fp8_linear(at::Tensor x, at::Tensor w, at::Tensor s, bool vector_gemv) {
    TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kBFloat16 && x.dim() == 2 && x.is_contiguous(),
                "FP8 linear expects CUDA BF16 [M,K]");
    TORCH_CHECK(w.is_cuda() && w.device() == x.device() && w.scalar_type() == at::kByte && w.dim() == 2 &&
                    w.is_contiguous() && x.size(1) == w.size(1),
                "Invalid FP8 weights");
    TORCH_CHECK(scales_ok(s, w), "Invalid FP8 scales");
    const int64_t M = x.size(0), N = w.size(0), K = w.size(1);
    TORCH_CHECK(M > 0 && N > 0 && K > 0, "Empty GEMM");
    Guard guard(x.device());
    auto y = at::empty({M, N}, x.options());
    // The prefill GEMM's K-split partials, allocated by the operator on the
    // input's stream as the reference allocates its own (src/fp8_tensor.cu:65).
    const size_t ws = fp8lin_linear_workspace_bytes(M, N, K);
    at::Tensor work;
    if (ws) work = at::empty({(int64_t)ws}, x.options().dtype(at::kByte));
    check(fp8lin_linear_ws(bf(x), w.data_ptr<uint8_t>(), s.data_ptr<float>(), scale_cols(s), bf_out(y), M, N, K,
                           vector_gemv ? 1 : 0, ws ? work.data_ptr() : nullptr, ws, stream_of(x)));
    return y;
}

// include/avi/ops.h:10, src/fp8_tensor.cu:53-71
at::Tensor fp8_tensor_small(at::Tensor x, at::Tensor codes, at::Tensor scales, int split) {
    check_tensor_small(x, codes, scales, split, false, "Invalid Ampere FP8 W8A16 geometry/dtype");
    return run_tensor_small(x, codes, scales, split);
}

// include/avi/tilelang.h:11, src/tilelang.cpp:94-107 (same contract plus
// N % 16 == 0; served by the same matrix-core kernel)
at::Tensor tilelang_fp8_small(at::Tensor x, at::Tensor codes, at::Tensor scales, int split) {
    check_tensor_small(x, codes, scales, split, true, "Invalid TileLang FP8 W8A16 inputs");
    return run_tensor_small(x, codes, scales, split);
}

// include/avi/ops.h:11, src/deep_kernels.cu:134-157
at::Tensor small_linear_shared(at::Tensor x, at::Tensor weight, at::Tensor scales) {
    TORCH_CHECK(x.is_cuda() && x.dim() == 2 && x.is_contiguous() && x.scalar_type() == at::kBFloat16 &&
                    weight.is_cuda() && weight.dim() == 2 && weight.is_contiguous() && weight.device() == x.device() &&
                    x.size(1) == weight.size(1),
                "Invalid shared GEMV inputs");
    const int64_t M = x.size(0), N = weight.size(0), K = x.size(1);
    TORCH_CHECK(M >= 1 && M <= 8 && N > 0 && K > 0, "Shared GEMV requires 1..8 rows");
    const bool fp8 = scales.defined();
    if (fp8) {
        TORCH_CHECK(weight.scalar_type() == at::kByte && scales_ok(scales, weight), "Invalid shared FP8 scales");
    } else {
        TORCH_CHECK(weight.scalar_type() == at::kBFloat16, "Shared GEMV expects BF16 or FP8 weights");
    }
    Guard guard(x.device());
    auto y = at::empty({M, N}, x.options());
    check(fp8lin_linear_shared(bf(x), weight.data_ptr(), fp8 ? scales.data_ptr<float>() : nullptr,
                               fp8 ? scale_cols(scales) : 1, bf_out(y), M, N, K, stream_of(x)));
    return y;
}

// include/avi/ops.h:20, src/optimized.cu:73-74
at::Tensor fused_swiglu(at::Tensor x) {
    TORCH_CHECK(x.is_contiguous() && x.dim() == 2 && x.scalar_type() == at::kBFloat16 && x.is_cuda() &&
                    x.size(1) % 2 == 0,
                "Invalid SwiGLU input");
    Guard guard(x.device());
    auto y = at::empty({x.size(0), x.size(1) / 2}, x.options());
    check(fp8lin_swiglu(bf(x), bf_out(y), x.size(0), x.size(1) / 2, stream_of(x)));
    return y;
}

// include/avi/ops.h:19, src/optimized.cu:71-72
at::Tensor fused_rms(at::Tensor x, at::Tensor w, double eps, bool one_center) {
    x = x.contiguous();
    w = w.contiguous();
    TORCH_CHECK(x.is_cuda() && w.device() == x.device() && x.scalar_type() == at::kBFloat16 &&
                    w.scalar_type() == at::kBFloat16 && w.numel() == x.size(-1),
                "Invalid RMS input");
    Guard guard(x.device());
    auto y = at::empty_like(x);
    const int64_t D = x.size(-1);
    check(fp8lin_rms(bf(x), bf(w), bf_out(y), D ? x.numel() / D : 0, D, eps, one_center ? 1 : 0, stream_of(x)));
    return y;
}

// include/avi/ops.h:25, src/optimized.cu:77-78
at::Tensor fused_rope(at::Tensor x, at::Tensor pos, int64_t r, double theta, int64_t hs, int64_t ws) {
    x = x.contiguous();
    pos = pos.contiguous();
    TORCH_CHECK(x.dim() == 3 && x.is_cuda() && x.scalar_type() == at::kBFloat16 && pos.device() == x.device() &&
                    pos.scalar_type() == at::kLong && pos.dim() == 2 && pos.size(0) == 3 &&
                    pos.size(1) == x.size(0) && r > 0 && r % 2 == 0 && r <= x.size(2),
                "Invalid RoPE input");
    Guard guard(x.device());
    auto y = at::empty_like(x);
    check(fp8lin_rope(bf(x), pos.data_ptr<int64_t>(), bf_out(y), x.size(0), x.size(1), x.size(2), r, theta, hs, ws,
                      stream_of(x)));
    return y;
}

// include/avi/ops.h:6, src/dual_path.cu:68-78
std::pair<at::Tensor, at::Tensor> residual_rms(at::Tensor x, at::Tensor update, at::Tensor weight, double eps,
                                               bool centered) {
    TORCH_CHECK(x.is_cuda() && x.dim() >= 2 && x.scalar_type() == at::kBFloat16 && x.is_contiguous() &&
                    x.numel() > 0 && update.device() == x.device() && update.scalar_type() == x.scalar_type() &&
                    update.sizes() == x.sizes() && update.is_contiguous() && weight.device() == x.device() &&
                    weight.scalar_type() == x.scalar_type() && weight.is_contiguous() &&
                    weight.numel() == x.size(-1) && x.size(-1) > 0 && x.size(-1) <= INT_MAX &&
                    x.numel() / x.size(-1) <= INT_MAX && std::isfinite(eps) && eps > 0,
                "Invalid fused residual RMS input");
    Guard guard(x.device());
    auto residual = at::empty_like(x), out = at::empty_like(x);
    check(fp8lin_residual_rms(bf(x), bf(update), bf(weight), bf_out(residual), bf_out(out), x.numel() / x.size(-1),
                              x.size(-1), eps, centered ? 1 : 0, stream_of(x)));
    return {residual, out};
}

// include/avi/ops.h:7, src/dual_path.cu:79-85
at::Tensor vocabulary_candidates(at::Tensor logits, int64_t offset) {
    TORCH_CHECK(logits.is_cuda() && logits.scalar_type() == at::kBFloat16 && logits.dim() == 2 &&
                    logits.is_contiguous() && logits.size(0) > 0 && logits.size(0) <= 65535 && logits.size(1) > 0 &&
                    offset >= 0 && offset <= INT_MAX - logits.size(1),
                "Invalid vocabulary candidates");
    Guard guard(logits.device());
    const int64_t M = logits.size(0), N = logits.size(1);
    auto out = at::empty({M, 2}, logits.options().dtype(at::kDouble));
    const size_t ws = fp8lin_vocab_candidates_workspace_bytes(M, N);
    auto work = at::empty({(int64_t)ws}, logits.options().dtype(at::kByte));
    check(fp8lin_vocab_candidates(bf(logits), M, N, offset, out.data_ptr<double>(), work.data_ptr(), ws,
                                  stream_of(logits)));
    return out;
}

// include/avi/ops.h:8, src/dual_path.cu:86-92
at::Tensor merge_candidates(at::Tensor gathered) {
    TORCH_CHECK(gathered.is_cuda() && gathered.scalar_type() == at::kDouble && gathered.is_contiguous() &&
                    gathered.dim() == 3 && gathered.size(0) > 0 && gathered.size(0) <= 8 && gathered.size(1) > 0 &&
                    gathered.size(1) <= 65535 && gathered.size(2) == 2,
                "Invalid gathered candidates");
    Guard guard(gathered.device());
    auto out = at::empty({gathered.size(1)}, gathered.options().dtype(at::kLong));
    check(fp8lin_merge_candidates(gathered.data_ptr<double>(), gathered.size(0), gathered.size(1),
                                  out.data_ptr<int64_t>(), stream_of(gathered)));
    return out;
}

}  // namespace avi

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "The reference's avi:: linear-path operators on ROCm LibTorch over the fp8lin C ABI";
    m.def("fp8_decode", &avi::fp8_decode);
    m.def("fp8_linear", &avi::fp8_linear, py::arg("x"), py::arg("codes"), py::arg("scales"),
          py::arg("vector_gemv") = false);
    m.def("fp8_tensor_small", &avi::fp8_tensor_small, py::arg("x"), py::arg("codes"), py::arg("scales"),
          py::arg("split") = 1);
    m.def("tilelang_fp8_small", &avi::tilelang_fp8_small);
    m.def(
        "small_linear_shared",
        [](at::Tensor x, at::Tensor weight, std::optional<at::Tensor> scales) {
            return avi::small_linear_shared(x, weight, scales ? *scales : at::Tensor());
        },
        py::arg("x"), py::arg("weight"), py::arg("scales") = py::none());
    m.def("fused_swiglu", &avi::fused_swiglu);
    m.def("fused_rms", &avi::fused_rms);
    m.def("fused_rope", &avi::fused_rope);
    m.def("residual_rms", &avi::residual_rms, py::arg("residual"), py::arg("update"), py::arg("weight"),
          py::arg("eps"), py::arg("centered") = true);
    m.def("vocabulary_candidates", &avi::vocabulary_candidates, py::arg("logits"), py::arg("offset") = 0);
    m.def("merge_candidates", &avi::merge_candidates);
}
