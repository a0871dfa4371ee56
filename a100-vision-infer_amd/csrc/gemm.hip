// Prefill GEMM dispatch.  FP8 weights with K % 256 == 0 (every benchmark
// shape) run gemm_fp8_kernel (gemm_fp8.hpp); other K, unaligned operands and
// BF16 weights run the general template of gemm_kernel.hpp.
//
// General template, as measured on MI355X at the prefill shapes (M =
// 512..4096, N = 17408, K = 5120, fused SwiGLU): a 256x256 workgroup tile of 8 waves
// (2 along M x 4 along N, 128x64 per wave as 4x2 accumulators of
// v_mfma_f32_32x32x16_bf16), K step 64, global loads issued two K steps ahead,
// the next stage's FP8 dequantization and LDS store placed after the second
// MFMA group, and the scheduler's MFMA/LDS interleave strategy 1.
#include "gemm_fp8.hpp"
#include "gemm_kernel.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

using Tile = gemm::Cfg<256, 256, 64, 2, 4>;
constexpr int kGroupM = 8;   // XCD-local tile patch height
constexpr int kIglp = 1;     // MFMA / LDS interleave strategy
constexpr int kPrefetch = 2; // global loads two K steps ahead
constexpr int kStoreAt = 1;  // next-stage store after MFMA sub-step 1

template <bool FP8, bool SWIGLU>
hipError_t run(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
               int64_t ldy, int M, int N, int K, hipStream_t stream) {
    return gemm::launch<Tile, FP8, SWIGLU, kGroupM, kIglp, kPrefetch, kStoreAt>(x, w, scales, S, y, ldy,
                                                                             M, N, K, stream);
}

}  // namespace

template <bool SWIGLU>
hipError_t run_fp8(const uint16_t* x, const uint8_t* w, const float* scales, int S, uint16_t* y,
                   int64_t ldy, int M, int N, int K, hipStream_t stream) {
    using namespace gemm_fp8;
    const int mtiles = (M + BM - 1) / BM;
    const int ntiles = SWIGLU ? ((N >> 1) + BN / 2 - 1) / (BN / 2) : (N + BN - 1) / BN;
    const int per_xcd = (mtiles * ntiles + kXcds - 1) / kXcds;
    auto kern = gemm_fp8_kernel<SWIGLU>;
    static const hipError_t attr = gemm::allow_lds(reinterpret_cast<const void*>(kern), LDS_BYTES);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kern, dim3(per_xcd * kXcds), dim3(THREADS), LDS_BYTES, stream, x, w, scales, S, y,
                       (int)ldy, M, N, K, mtiles, ntiles);
    return hipGetLastError();
}

hipError_t launch_gemm(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
                       int64_t ldy, int M, int N, int K, bool swiglu, hipStream_t stream) {
    const bool fp8 = scales != nullptr;
    if (fp8 && gemm_fp8::supported(x, w, S, ldy, M, N, K)) {
        const uint8_t* codes = static_cast<const uint8_t*>(w);
        return swiglu ? run_fp8<true>(x, codes, scales, S, y, ldy, M, N, K, stream)
                      : run_fp8<false>(x, codes, scales, S, y, ldy, M, N, K, stream);
    }
    if (fp8)
        return swiglu ? run<true, true>(x, w, scales, S, y, ldy, M, N, K, stream)
                      : run<true, false>(x, w, scales, S, y, ldy, M, N, K, stream);
    return swiglu ? run<false, true>(x, w, nullptr, 1, y, ldy, M, N, K, stream)
                  : run<false, false>(x, w, nullptr, 1, y, ldy, M, N, K, stream);
}

}  // namespace fp8lin
