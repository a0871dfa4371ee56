// Prefill GEMM: y[M,N] = x[M,K] * W^T on the BF16 matrix cores.
//
// W is either E4M3FN codes with FP32 block scales -- each 64-wide K slice of a
// weight tile is loaded as FP8 bytes, converted in registers with the
// reference rounding point bf16(decode(c) * s) (src/optimized.cu:32) and
// stored to LDS as BF16 -- or plain BF16 (decoded-weight cache, dequant-then-
// GEMM slabs, unquantized weights: src/engine.cpp:221,232,236).
//
// Tiling (gfx950): a 512-thread workgroup computes a 256x256 output tile;
// 8 waves in a 2 (M) x 4 (N) grid each own a 128x64 sub-tile held as 8x4
// v_mfma_f32_16x16x32_bf16 accumulators (128 FP32 per lane).  K advances 64 per
// step through a double-buffered LDS ring (A and B tiles, rows padded to 72
// BF16 = 144 bytes so the 16 rows read by one MFMA fragment fall in distinct
// banks); the next step's global loads are issued before the current step's
// MFMAs.  LDS use: 2 x (256 + 256) x 144 B = 144 KiB of the 160 KiB per CU.
//
// Fused gate/up + SwiGLU (src/engine.cpp:415): the B tile's 256 rows are 128
// gate rows and the 128 matching up rows, interleaved so that each wave's
// 64 columns are 32 gate columns followed by their 32 up columns.  A lane then
// holds gate and up for the same output element in accumulators (mt, nt) and
// (mt, nt+2), and the epilogue applies SwiGLU in registers, writing the
// [M, N/2] output only.
#include "device.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

constexpr int kThreads = 512;
constexpr int BM = 256, BN = 256, BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // BF16 elements per LDS row
constexpr int WAVE_M = 128, WAVE_N = 64;
constexpr int MT = WAVE_M / 16, NT = WAVE_N / 16;
constexpr int A_CHUNKS = BM * BK / 8 / kThreads;   // 16-byte BF16 chunks per thread (4)
constexpr int B8_CHUNKS = BN * BK / 16 / kThreads; // 16-byte FP8 chunks per thread (2)
constexpr int B16_CHUNKS = BN * BK / 8 / kThreads; // 16-byte BF16 chunks per thread (4)

struct Smem {
    uint16_t a[2][BM * LDS_STRIDE];
    uint16_t b[2][BN * LDS_STRIDE];
};

// Weight row held by row `b` of the B tile (or -1 when out of range).
template <bool SWIGLU>
__device__ __forceinline__ int64_t b_tile_row(int tile, int b, int N) {
    if constexpr (SWIGLU) {
        const int D = N >> 1;
        const int q = b >> 6, w = b & 63;
        const int j = tile * (BN / 2) + 32 * q + (w & 31);
        if (j >= D) return -1;
        return w < 32 ? j : (int64_t)D + j;
    } else {
        const int64_t n = (int64_t)tile * BN + b;
        return n < N ? n : -1;
    }
}

template <bool FP8, bool GUARD, bool SWIGLU>
struct Loader {
    u32x4 a[A_CHUNKS];
    u32x4 b[FP8 ? B8_CHUNKS : B16_CHUNKS];
    float s[FP8 ? B8_CHUNKS : 1];

    __device__ __forceinline__ void load(const uint16_t* __restrict__ x, const void* __restrict__ w,
                                         const float* __restrict__ scales, int S, int M, int N, int K,
                                         int m0, int ntile, int k0) {
        const int t = threadIdx.x;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const int q = t + kThreads * i;
            const int row = q >> 3, kc = (q & 7) * 8;
            const int m = m0 + row;
            const uint16_t* src = x + (int64_t)(m < M ? m : 0) * K + k0 + kc;
            if constexpr (!GUARD) {
                a[i] = m < M ? load_u32x4(src) : u32x4{0, 0, 0, 0};
            } else {
                uint32_t v[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const int k = k0 + kc + 2 * d;
                    uint32_t lo = (m < M && k < K) ? (uint32_t)src[2 * d] : 0u;
                    uint32_t hi = (m < M && k + 1 < K) ? (uint32_t)src[2 * d + 1] : 0u;
                    v[d] = lo | (hi << 16);
                }
                a[i] = u32x4{v[0], v[1], v[2], v[3]};
            }
        }
        if constexpr (FP8) {
            const uint8_t* codes = static_cast<const uint8_t*>(w);
#pragma unroll
            for (int i = 0; i < B8_CHUNKS; ++i) {
                const int q = t + kThreads * i;
                const int row = q >> 2, kc = (q & 3) * 16;
                const int64_t n = b_tile_row<SWIGLU>(ntile, row, N);
                const uint8_t* src = codes + (n >= 0 ? n : 0) * (int64_t)K + k0 + kc;
                const bool in_k = GUARD ? (k0 + kc < K) : true;
                s[i] = (n >= 0 && in_k) ? scales[n * S + (S == 1 ? 0 : (k0 + kc) >> 7)] : 0.0f;
                if constexpr (!GUARD) {
                    b[i] = n >= 0 ? load_u32x4(src) : u32x4{0, 0, 0, 0};
                } else {
                    uint32_t v[4];
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        uint32_t word = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int k = k0 + kc + 4 * d + e;
                            uint32_t byte = (n >= 0 && k < K) ? (uint32_t)src[4 * d + e] : 0u;
                            word |= byte << (8 * e);
                        }
                        v[d] = word;
                    }
                    b[i] = u32x4{v[0], v[1], v[2], v[3]};
                }
            }
        } else {
            const uint16_t* wb = static_cast<const uint16_t*>(w);
#pragma unroll
            for (int i = 0; i < B16_CHUNKS; ++i) {
                const int q = t + kThreads * i;
                const int row = q >> 3, kc = (q & 7) * 8;
                const int64_t n = b_tile_row<SWIGLU>(ntile, row, N);
                const uint16_t* src = wb + (n >= 0 ? n : 0) * (int64_t)K + k0 + kc;
                if constexpr (!GUARD) {
                    b[i] = n >= 0 ? load_u32x4(src) : u32x4{0, 0, 0, 0};
                } else {
                    uint32_t v[4];
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const int k = k0 + kc + 2 * d;
                        uint32_t lo = (n >= 0 && k < K) ? (uint32_t)src[2 * d] : 0u;
                        uint32_t hi = (n >= 0 && k + 1 < K) ? (uint32_t)src[2 * d + 1] : 0u;
                        v[d] = lo | (hi << 16);
                    }
                    b[i] = u32x4{v[0], v[1], v[2], v[3]};
                }
            }
        }
    }

    __device__ __forceinline__ void store(uint16_t* __restrict__ sa, uint16_t* __restrict__ sb) const {
        const int t = threadIdx.x;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const int q = t + kThreads * i;
            const int row = q >> 3, kc = (q & 7) * 8;
            *reinterpret_cast<u32x4*>(sa + row * LDS_STRIDE + kc) = a[i];
        }
        if constexpr (FP8) {
#pragma unroll
            for (int i = 0; i < B8_CHUNKS; ++i) {
                const int q = t + kThreads * i;
                const int row = q >> 2, kc = (q & 3) * 16;
                uint32_t wv[8];
                dequant4(b[i].x, s[i], wv[0], wv[1]);
                dequant4(b[i].y, s[i], wv[2], wv[3]);
                dequant4(b[i].z, s[i], wv[4], wv[5]);
                dequant4(b[i].w, s[i], wv[6], wv[7]);
                u32x4* dst = reinterpret_cast<u32x4*>(sb + row * LDS_STRIDE + kc);
                dst[0] = u32x4{wv[0], wv[1], wv[2], wv[3]};
                dst[1] = u32x4{wv[4], wv[5], wv[6], wv[7]};
            }
        } else {
#pragma unroll
            for (int i = 0; i < B16_CHUNKS; ++i) {
                const int q = t + kThreads * i;
                const int row = q >> 3, kc = (q & 7) * 8;
                *reinterpret_cast<u32x4*>(sb + row * LDS_STRIDE + kc) = b[i];
            }
        }
    }
};

template <bool FP8, bool GUARD, bool SWIGLU>
__global__ __launch_bounds__(kThreads) void gemm_kernel(const uint16_t* __restrict__ x,
                                                        const void* __restrict__ w,
                                                        const float* __restrict__ scales, int S,
                                                        uint16_t* __restrict__ y, int64_t ldy,
                                                        int M, int N, int K, int mtiles) {
    __shared__ Smem sm;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int wm = wave >> 2, wn = wave & 3;
    const int mtile = blockIdx.x % mtiles;
    const int ntile = blockIdx.x / mtiles;
    const int m0 = mtile * BM;

    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int KT = (K + BK - 1) / BK;
    Loader<FP8, GUARD, SWIGLU> ld;
    ld.load(x, w, scales, S, M, N, K, m0, ntile, 0);
    ld.store(sm.a[0], sm.b[0]);
    __syncthreads();

    const int frag_row = lane & 15;
    const int frag_k = (lane >> 4) * 8;
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) ld.load(x, w, scales, S, M, N, K, m0, ntile, (kt + 1) * BK);
        const uint16_t* sa = sm.a[buf] + (wm * WAVE_M + frag_row) * LDS_STRIDE + frag_k;
        const uint16_t* sb = sm.b[buf] + (wn * WAVE_N + frag_row) * LDS_STRIDE + frag_k;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            bf16x8 bfrag[NT];
#pragma unroll
            for (int j = 0; j < NT; ++j)
                bfrag[j] = *reinterpret_cast<const bf16x8*>(sb + j * 16 * LDS_STRIDE + kk);
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const bf16x8 afrag = *reinterpret_cast<const bf16x8*>(sa + i * 16 * LDS_STRIDE + kk);
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag, bfrag[j], acc[i][j], 0, 0, 0);
            }
        }
        if (kt + 1 < KT) ld.store(sm.a[buf ^ 1], sm.b[buf ^ 1]);
        __syncthreads();
    }

    // acc[i][j][r] = C[wm*128 + 16i + 4*(lane/16) + r][wn*64 + 16j + lane%16]
    const int rbase = m0 + wm * WAVE_M + 4 * (lane >> 4);
    if constexpr (SWIGLU) {
        const int D = N >> 1;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = ntile * (BN / 2) + wn * 32 + 16 * j + (lane & 15);
            if (col >= D) continue;
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = rbase + 16 * i + r;
                    if (row < M)
                        y[(int64_t)row * ldy + col] = swiglu_bf16_bits(
                            f32_to_bf16_bits(acc[i][j][r]), f32_to_bf16_bits(acc[i][j + 2][r]));
                }
        }
    } else {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int col = ntile * BN + wn * WAVE_N + 16 * j + (lane & 15);
            if (col >= N) continue;
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = rbase + 16 * i + r;
                    if (row < M) y[(int64_t)row * ldy + col] = f32_to_bf16_bits(acc[i][j][r]);
                }
        }
    }
}

template <bool FP8, bool SWIGLU>
hipError_t launch_t(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
                    int64_t ldy, int M, int N, int K, hipStream_t stream) {
    const int mtiles = (M + BM - 1) / BM;
    const int ntiles = SWIGLU ? ((N >> 1) + BN / 2 - 1) / (BN / 2) : (N + BN - 1) / BN;
    const bool aligned = (K % BK == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(w) % 16 == 0);
    dim3 grid(mtiles * ntiles);
    if (aligned)
        hipLaunchKernelGGL((gemm_kernel<FP8, false, SWIGLU>), grid, dim3(kThreads), 0, stream, x, w,
                           scales, S, y, ldy, M, N, K, mtiles);
    else
        hipLaunchKernelGGL((gemm_kernel<FP8, true, SWIGLU>), grid, dim3(kThreads), 0, stream, x, w,
                           scales, S, y, ldy, M, N, K, mtiles);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
                       int64_t ldy, int M, int N, int K, bool swiglu, hipStream_t stream) {
    const bool fp8 = scales != nullptr;
    if (fp8)
        return swiglu ? launch_t<true, true>(x, w, scales, S, y, ldy, M, N, K, stream)
                      : launch_t<true, false>(x, w, scales, S, y, ldy, M, N, K, stream);
    return swiglu ? launch_t<false, true>(x, w, nullptr, 1, y, ldy, M, N, K, stream)
                  : launch_t<false, false>(x, w, nullptr, 1, y, ldy, M, N, K, stream);
}

}  // namespace fp8lin
