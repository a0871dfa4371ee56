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
#include <algorithm>

#include "gemm_fp8.hpp"
#include "gemm_kernel.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

using Tile = gemm::Cfg<256, 256, 64, 2, 4>;
// Split-K: used when the output has at most half as many 256x256 tiles as
// there are CUs; the splits fill up to kSplitCus workgroups.
constexpr int kSplitCus = 256;
constexpr int kMaxSplits = 8;
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

// Split-K reduction: out[m][c] = bf16(sum over s in order of part[s][m][c])
// for c < N, or with SWIGLU y[m][j] = swiglu(bf16(gate sum), bf16(up sum))
// from weight-row columns j and N/2 + j -- the rounding points of the
// unsplit epilogue.  Four columns per thread when the row widths allow it.
template <bool SWIGLU, bool VEC>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int splits, int M, int N,
                                                            uint16_t* __restrict__ y, int64_t ldy) {
    const int cols = SWIGLU ? N / 2 : N;
    const int per_row = VEC ? cols / 4 : cols;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)M * per_row) return;
    const int m = (int)(idx / per_row), c = (int)(idx % per_row) * (VEC ? 4 : 1);
    const int64_t slice = (int64_t)M * N;
    const float* p = part + (int64_t)m * N + c;
    auto sum = [&](int off) __attribute__((always_inline)) -> f32x4 {
        f32x4 t;
        if constexpr (VEC) {
            t = *reinterpret_cast<const f32x4*>(p + off);
            for (int s = 1; s < splits; ++s) t += *reinterpret_cast<const f32x4*>(p + s * slice + off);
        } else {
            t = f32x4{p[off], 0.0f, 0.0f, 0.0f};
            for (int s = 1; s < splits; ++s) t[0] += p[s * slice + off];
        }
        return t;
    };
    uint16_t out[4];
    const f32x4 a = sum(0);
    if constexpr (SWIGLU) {
        const f32x4 u = sum(N / 2);
#pragma unroll
        for (int q = 0; q < (VEC ? 4 : 1); ++q)
            out[q] = swiglu_bf16_bits(f32_to_bf16_bits(a[q]), f32_to_bf16_bits(u[q]));
    } else {
#pragma unroll
        for (int q = 0; q < (VEC ? 4 : 1); ++q) out[q] = f32_to_bf16_bits(a[q]);
    }
    uint16_t* dst = y + (int64_t)m * ldy + c;
#pragma unroll
    for (int q = 0; q < (VEC ? 4 : 1); ++q) dst[q] = out[q];
}

template <bool SWIGLU, bool PARTIAL>
hipError_t run_fp8(const uint16_t* x, const uint8_t* w, const float* scales, int S, uint16_t* y,
                   int64_t ldy, int M, int N, int K, float* part, int splits, hipStream_t stream) {
    using namespace gemm_fp8;
    const int mtiles = (M + BM - 1) / BM;
    const int ntiles = SWIGLU ? ((N >> 1) + BN / 2 - 1) / (BN / 2) : (N + BN - 1) / BN;
    const int per_xcd = (mtiles * ntiles + kXcds - 1) / kXcds;
    auto kern = gemm_fp8_kernel<SWIGLU, PARTIAL>;
    static const hipError_t attr = gemm::allow_lds(reinterpret_cast<const void*>(kern), LDS_BYTES);
    if (attr != hipSuccess) return attr;
    uint16_t* out = PARTIAL ? reinterpret_cast<uint16_t*>(part) : y;
    hipLaunchKernelGGL(kern, dim3(per_xcd * kXcds, PARTIAL ? splits : 1), dim3(THREADS), LDS_BYTES, stream, x, w,
                       scales, S, out, (int)ldy, M, N, K, mtiles, ntiles, splits);
    hipError_t e = hipGetLastError();
    if (!PARTIAL || e != hipSuccess) return e;
    const int cols = SWIGLU ? N / 2 : N;
    const bool vec = cols % 4 == 0 && (!SWIGLU || (N / 2) % 4 == 0) && N % 4 == 0;
    const int64_t threads = (int64_t)M * (vec ? cols / 4 : cols);
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (vec)
        hipLaunchKernelGGL((splitk_reduce_kernel<SWIGLU, true>), grid, dim3(256), 0, stream, part, splits, M, N, y, ldy);
    else
        hipLaunchKernelGGL((splitk_reduce_kernel<SWIGLU, false>), grid, dim3(256), 0, stream, part, splits, M, N, y,
                           ldy);
    return hipGetLastError();
}

int gemm_splits(int S, int64_t ldy, int M, int N, int K, bool swiglu) {
    using namespace gemm_fp8;
    // the FP8 kernel's shape requirements (pointer alignment is the caller's)
    if (!supported(nullptr, nullptr, S, ldy, M, N, K) || ((int64_t)M + BM) * N * 4 >= ((int64_t)1 << 31)) return 1;
    const int64_t tiles = (int64_t)((M + BM - 1) / BM) * (swiglu ? ((N >> 1) + BN / 2 - 1) / (BN / 2)
                                                                  : (N + BN - 1) / BN);
    if (tiles * 2 > kSplitCus) return 1;
    const int chunks = K / 256;
    return std::min<int64_t>(std::min<int64_t>(kSplitCus / tiles, chunks), kMaxSplits);
}

hipError_t launch_gemm_split(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
                             int64_t ldy, int M, int N, int K, bool swiglu, float* part, int splits,
                             hipStream_t stream) {
    const uint8_t* codes = static_cast<const uint8_t*>(w);
    if (splits <= 1 || !gemm_fp8::supported(x, w, S, ldy, M, N, K))
        return launch_gemm(x, w, scales, S, y, ldy, M, N, K, swiglu, stream);
    return swiglu ? run_fp8<true, true>(x, codes, scales, S, y, ldy, M, N, K, part, splits, stream)
                  : run_fp8<false, true>(x, codes, scales, S, y, ldy, M, N, K, part, splits, stream);
}

hipError_t launch_gemm(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
                       int64_t ldy, int M, int N, int K, bool swiglu, hipStream_t stream) {
    const bool fp8 = scales != nullptr;
    if (fp8 && gemm_fp8::supported(x, w, S, ldy, M, N, K)) {
        const uint8_t* codes = static_cast<const uint8_t*>(w);
        return swiglu ? run_fp8<true, false>(x, codes, scales, S, y, ldy, M, N, K, nullptr, 1, stream)
                      : run_fp8<false, false>(x, codes, scales, S, y, ldy, M, N, K, nullptr, 1, stream);
    }
    if (fp8)
        return swiglu ? run<true, true>(x, w, scales, S, y, ldy, M, N, K, stream)
                      : run<true, false>(x, w, scales, S, y, ldy, M, N, K, stream);
    return swiglu ? run<false, true>(x, w, nullptr, 1, y, ldy, M, N, K, stream)
                  : run<false, false>(x, w, nullptr, 1, y, ldy, M, N, K, stream);
}

}  // namespace fp8lin
