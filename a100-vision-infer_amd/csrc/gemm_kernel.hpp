// Prefill GEMM kernel template: y[M,N] = x[M,K] * W^T on the BF16 matrix cores.
//
// W is E4M3FN codes with FP32 block scales -- each K slice of a weight tile is
// loaded as FP8 bytes, converted in registers with the reference rounding point
// bf16(decode(c) * s) (src/optimized.cu:32) and stored to LDS as BF16 -- or
// plain BF16 (decoded-weight cache, dequant-then-GEMM slabs, unquantized
// weights: src/engine.cpp:221,232,236).
//
// Tiling: a workgroup of WAVES_M x WAVES_N waves computes a BM x BN tile; each
// wave owns a (BM/WAVES_M) x (BN/WAVES_N) sub-tile held as 32x32 accumulators of
// v_mfma_f32_32x32x16_bf16 (FP32).  K advances BK per step through a double-
// buffered LDS ring whose rows are padded by 8 BF16 so the 32 rows read by one
// MFMA fragment fall in distinct banks; the next step's global loads are
// issued before the current step's MFMAs and written to the other LDS buffer
// after them, with one barrier per step.
//
// Fused gate/up + SwiGLU (src/engine.cpp:415): the B tile holds BN/2 gate rows
// and the BN/2 matching up rows, arranged so that in every wave's column range
// the first half are gate columns and the second half the up columns of the
// same outputs.  Accumulator (i, j) and (i, j + NT/2) then hold gate and up for
// the same output element in the same lane, and the epilogue applies SwiGLU in
// registers and writes only the [M, N/2] result.
#pragma once
#include "device.hpp"

namespace fp8lin {
namespace gemm {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <int BM_, int BN_, int BK_, int WAVES_M_, int WAVES_N_>
struct Cfg {
    static constexpr int BM = BM_, BN = BN_, BK = BK_;
    static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_;
    static constexpr int THREADS = 64 * WAVES_M * WAVES_N;
    static constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;  // wave tile
    static constexpr int MT = WTM / 32, NT = WTN / 32;            // 32x32 tiles per wave
    static constexpr int LDS_STRIDE = BK + 8;                     // BF16 per LDS row
    static constexpr int A_CHUNKS = BM * BK / 8 / THREADS;        // 16-byte BF16 chunks
    static constexpr int B8_CHUNKS = BN * BK / 16 / THREADS;      // 16-byte FP8 chunks
    static constexpr int B16_CHUNKS = BN * BK / 8 / THREADS;      // 16-byte BF16 chunks
    static constexpr int LDS_BYTES = 2 * (BM + BN) * LDS_STRIDE * 2;
    static_assert(BM * BK % (8 * THREADS) == 0 && BN * BK % (16 * THREADS) == 0, "tile/threads");
    static_assert(WTM % 32 == 0 && WTN % 32 == 0 && BK % 16 == 0, "wave tile");
};

// Weight row held by row `b` of the B tile (or -1 when out of range).
template <class C, bool SWIGLU>
__device__ __forceinline__ int64_t b_tile_row(int tile, int b, int N) {
    if constexpr (SWIGLU) {
        constexpr int HALF = C::WTN / 2;  // gate columns per wave
        const int D = N >> 1;
        const int q = b / C::WTN, w = b % C::WTN;
        const int j = tile * (C::BN / 2) + HALF * q + (w % HALF);
        if (j >= D) return -1;
        return w < HALF ? j : (int64_t)D + j;
    } else {
        const int64_t n = (int64_t)tile * C::BN + b;
        return n < N ? n : -1;
    }
}

template <class C, bool FP8, bool GUARD, bool SWIGLU>
struct Loader {
    u32x4 a[C::A_CHUNKS];
    u32x4 b[FP8 ? C::B8_CHUNKS : C::B16_CHUNKS];
    float s[FP8 ? C::B8_CHUNKS : 1];
    // Raw buffers (aligned path): 32-bit offsets, masked rows read zeros.
    rsrc_t rx, rw, rs;
    uint32_t aoff[C::A_CHUNKS], boff[FP8 ? C::B8_CHUNKS : C::B16_CHUNKS], soff[FP8 ? C::B8_CHUNKS : 1];

    // Per-thread base offsets of the tile (k0 = 0); load() adds the K step.
    __device__ __forceinline__ void init(const uint16_t* __restrict__ x, const void* __restrict__ w,
                                         const float* __restrict__ scales, int S, int M, int N, int K,
                                         int m0, int ntile) {
        if constexpr (!GUARD) {
            const int t = threadIdx.x;
            rx = make_rsrc(x, (uint32_t)((int64_t)M * K * 2));
            rw = make_rsrc(w, (uint32_t)((int64_t)N * K * (FP8 ? 1 : 2)));
            rs = make_rsrc(scales, FP8 ? (uint32_t)((int64_t)N * S * 4) : 0u);
            constexpr int ACH = C::BK / 8;
#pragma unroll
            for (int i = 0; i < C::A_CHUNKS; ++i) {
                const int q = t + C::THREADS * i;
                const int m = m0 + q / ACH, kc = (q % ACH) * 8;
                aoff[i] = m < M ? (uint32_t)(((int64_t)m * K + kc) * 2) : kBufferOob;
            }
            if constexpr (FP8) {
                constexpr int BCH = C::BK / 16;
#pragma unroll
                for (int i = 0; i < C::B8_CHUNKS; ++i) {
                    const int q = t + C::THREADS * i;
                    const int64_t n = b_tile_row<C, SWIGLU>(ntile, q / BCH, N);
                    boff[i] = n >= 0 ? (uint32_t)(n * K + (q % BCH) * 16) : kBufferOob;
                    soff[i] = n >= 0 ? (uint32_t)(n * S * 4) : kBufferOob;
                }
            } else {
#pragma unroll
                for (int i = 0; i < C::B16_CHUNKS; ++i) {
                    const int q = t + C::THREADS * i;
                    const int64_t n = b_tile_row<C, SWIGLU>(ntile, q / ACH, N);
                    boff[i] = n >= 0 ? (uint32_t)((n * K + (q % ACH) * 8) * 2) : kBufferOob;
                }
            }
        }
    }

    __device__ __forceinline__ void load(const uint16_t* __restrict__ x, const void* __restrict__ w,
                                         const float* __restrict__ scales, int S, int M, int N, int K,
                                         int m0, int ntile, int k0) {
        if constexpr (!GUARD) {
            // Masked offsets stay >= kBufferOob after adding k0 (< 2^31).
#pragma unroll
            for (int i = 0; i < C::A_CHUNKS; ++i)
                a[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                     rx, (int)aoff[i], k0 * 2, 0));
            if constexpr (FP8) {
                const int kb = S == 1 ? 0 : (k0 >> 7) * 4;
#pragma unroll
                for (int i = 0; i < C::B8_CHUNKS; ++i) {
                    b[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                         rw, (int)boff[i], k0, 0));
                    s[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                         rs, (int)soff[i], kb, 0));
                }
            } else {
#pragma unroll
                for (int i = 0; i < C::B16_CHUNKS; ++i)
                    b[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                         rw, (int)boff[i], k0 * 2, 0));
            }
            return;
        }
        const int t = threadIdx.x;
        constexpr int ACH = C::BK / 8;  // chunks per A row
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i) {
            const int q = t + C::THREADS * i;
            const int row = q / ACH, kc = (q % ACH) * 8;
            const int m = m0 + row;
            const uint16_t* src = x + (int64_t)(m < M ? m : 0) * K + k0 + kc;
            if constexpr (!GUARD) {
                a[i] = m < M ? load_u32x4(src) : u32x4{0, 0, 0, 0};
            } else {
                uint32_t v[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const int k = k0 + kc + 2 * d;
                    const uint32_t lo = (m < M && k < K) ? (uint32_t)src[2 * d] : 0u;
                    const uint32_t hi = (m < M && k + 1 < K) ? (uint32_t)src[2 * d + 1] : 0u;
                    v[d] = lo | (hi << 16);
                }
                a[i] = u32x4{v[0], v[1], v[2], v[3]};
            }
        }
        if constexpr (FP8) {
            constexpr int BCH = C::BK / 16;
            const uint8_t* codes = static_cast<const uint8_t*>(w);
#pragma unroll
            for (int i = 0; i < C::B8_CHUNKS; ++i) {
                const int q = t + C::THREADS * i;
                const int row = q / BCH, kc = (q % BCH) * 16;
                const int64_t n = b_tile_row<C, SWIGLU>(ntile, row, N);
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
                            const uint32_t byte = (n >= 0 && k < K) ? (uint32_t)src[4 * d + e] : 0u;
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
            for (int i = 0; i < C::B16_CHUNKS; ++i) {
                const int q = t + C::THREADS * i;
                const int row = q / ACH, kc = (q % ACH) * 8;
                const int64_t n = b_tile_row<C, SWIGLU>(ntile, row, N);
                const uint16_t* src = wb + (n >= 0 ? n : 0) * (int64_t)K + k0 + kc;
                if constexpr (!GUARD) {
                    b[i] = n >= 0 ? load_u32x4(src) : u32x4{0, 0, 0, 0};
                } else {
                    uint32_t v[4];
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const int k = k0 + kc + 2 * d;
                        const uint32_t lo = (n >= 0 && k < K) ? (uint32_t)src[2 * d] : 0u;
                        const uint32_t hi = (n >= 0 && k + 1 < K) ? (uint32_t)src[2 * d + 1] : 0u;
                        v[d] = lo | (hi << 16);
                    }
                    b[i] = u32x4{v[0], v[1], v[2], v[3]};
                }
            }
        }
    }

    __device__ __forceinline__ void store(uint16_t* __restrict__ sa, uint16_t* __restrict__ sb) const {
        const int t = threadIdx.x;
        constexpr int ACH = C::BK / 8;
#pragma unroll
        for (int i = 0; i < C::A_CHUNKS; ++i) {
            const int q = t + C::THREADS * i;
            const int row = q / ACH, kc = (q % ACH) * 8;
            *reinterpret_cast<u32x4*>(sa + row * C::LDS_STRIDE + kc) = a[i];
        }
        if constexpr (FP8) {
            constexpr int BCH = C::BK / 16;
#pragma unroll
            for (int i = 0; i < C::B8_CHUNKS; ++i) {
                const int q = t + C::THREADS * i;
                const int row = q / BCH, kc = (q % BCH) * 16;
                uint32_t wv[8];
                dequant4(b[i].x, s[i], wv[0], wv[1]);
                dequant4(b[i].y, s[i], wv[2], wv[3]);
                dequant4(b[i].z, s[i], wv[4], wv[5]);
                dequant4(b[i].w, s[i], wv[6], wv[7]);
                u32x4* dst = reinterpret_cast<u32x4*>(sb + row * C::LDS_STRIDE + kc);
                dst[0] = u32x4{wv[0], wv[1], wv[2], wv[3]};
                dst[1] = u32x4{wv[4], wv[5], wv[6], wv[7]};
            }
        } else {
#pragma unroll
            for (int i = 0; i < C::B16_CHUNKS; ++i) {
                const int q = t + C::THREADS * i;
                const int row = q / ACH, kc = (q % ACH) * 8;
                *reinterpret_cast<u32x4*>(sb + row * C::LDS_STRIDE + kc) = b[i];
            }
        }
    }
};

// Tile of workgroup `bid`, XCD-aware.  The dispatcher deals workgroups to the
// 8 XCDs round-robin (bid % 8), and each XCD has its own L2.  Workgroup bid is
// therefore given logical index L = (bid % 8) * per_xcd + bid / 8, so each XCD
// owns a contiguous range of logical tiles, and L walks groups of GROUP_M tile
// rows with the M index fastest: the ~32 workgroups an XCD runs at once cover
// a GROUP_M x (32 / GROUP_M) patch and share both the activation and the
// weight K-slices in that XCD's L2.  Returns false for padding workgroups.
constexpr int kXcds = 8;
template <int GROUP_M>
__device__ __forceinline__ bool tile_of(int bid, int mtiles, int ntiles, int& mt, int& nt) {
    const int tiles = mtiles * ntiles;
    const int per_xcd = (tiles + kXcds - 1) / kXcds;
    const int L = (bid % kXcds) * per_xcd + bid / kXcds;
    if (L >= tiles) return false;
    const int per_group = GROUP_M * ntiles;
    const int g = L / per_group;
    const int first_m = g * GROUP_M;
    const int gsize = min(GROUP_M, mtiles - first_m);
    const int r = L - g * per_group;
    mt = first_m + r % gsize;
    nt = r / gsize;
    return true;
}

// IGLP >= 0 asks the scheduler for its MFMA/LDS interleave strategy IGLP.
template <class C, bool FP8, bool GUARD, bool SWIGLU, int GROUP_N, int IGLP, int PF, int ST>
__global__ __launch_bounds__(C::THREADS) void gemm_kernel(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const float* __restrict__ scales,
    int S, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int mtiles, int ntiles) {
    extern __shared__ __align__(16) uint16_t smem[];
    // LDS: A[2][BM][LDS_STRIDE] then B[2][BN][LDS_STRIDE]
    auto sA = [&](int b) { return smem + b * (C::BM * C::LDS_STRIDE); };
    auto sB = [&](int b) { return smem + 2 * C::BM * C::LDS_STRIDE + b * (C::BN * C::LDS_STRIDE); };
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
    int mtile, ntile;
    if (!tile_of<GROUP_N>(blockIdx.x, mtiles, ntiles, mtile, ntile)) return;
    const int m0 = mtile * C::BM;

    f32x16_t acc[C::MT][C::NT];
#pragma unroll
    for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int j = 0; j < C::NT; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int KT = (K + C::BK - 1) / C::BK;
    // Global -> register staging, PF K steps ahead of the MFMAs: stage s is
    // loaded into register set s % PF and stored to LDS buffer s % 2 one step
    // before it is consumed.
    Loader<C, FP8, GUARD, SWIGLU> ld[PF];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        ld[p].init(x, w, scales, S, M, N, K, m0, ntile);
        if (p < KT) ld[p].load(x, w, scales, S, M, N, K, m0, ntile, p * C::BK);
    }
    ld[0].store(sA(0), sB(0));
    __syncthreads();

    const int frag_row = lane & 31;
    const int frag_k = (lane >> 5) * 8;
    auto step = [&](int kt, Loader<C, FP8, GUARD, SWIGLU>& refill, Loader<C, FP8, GUARD, SWIGLU>& next) {
        const int buf = kt & 1;
        if (kt + PF < KT) refill.load(x, w, scales, S, M, N, K, m0, ntile, (kt + PF) * C::BK);
        const uint16_t* sa = sA(buf) + (wm * C::WTM + frag_row) * C::LDS_STRIDE + frag_k;
        const uint16_t* sb = sB(buf) + (wn * C::WTN + frag_row) * C::LDS_STRIDE + frag_k;
        // Fragments of K sub-step kk+1 are read from LDS while the MFMAs of
        // sub-step kk run (two register sets).
        bf16x8 af[2][C::MT], bfr[2][C::NT];
#pragma unroll
        for (int i = 0; i < C::MT; ++i) af[0][i] = *reinterpret_cast<const bf16x8*>(sa + i * 32 * C::LDS_STRIDE);
#pragma unroll
        for (int j = 0; j < C::NT; ++j) bfr[0][j] = *reinterpret_cast<const bf16x8*>(sb + j * 32 * C::LDS_STRIDE);
#pragma unroll
        for (int s = 0; s < C::BK / 16; ++s) {
            const int cur = s & 1;
            if (s + 1 < C::BK / 16) {
#pragma unroll
                for (int i = 0; i < C::MT; ++i)
                    af[cur ^ 1][i] = *reinterpret_cast<const bf16x8*>(sa + i * 32 * C::LDS_STRIDE + (s + 1) * 16);
#pragma unroll
                for (int j = 0; j < C::NT; ++j)
                    bfr[cur ^ 1][j] = *reinterpret_cast<const bf16x8*>(sb + j * 32 * C::LDS_STRIDE + (s + 1) * 16);
            }
#pragma unroll
            for (int i = 0; i < C::MT; ++i)
#pragma unroll
                for (int j = 0; j < C::NT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[cur][i], bfr[cur][j], acc[i][j], 0, 0, 0);
            if constexpr (IGLP >= 0) __builtin_amdgcn_iglp_opt(IGLP);
            // Dequantize and store the next stage between the MFMA groups so
            // the VALU work co-executes with the matrix cores (its data was
            // loaded PF steps ago; the target buffer was released by the
            // previous barrier).
            if (s == ST && kt + 1 < KT) next.store(sA(buf ^ 1), sB(buf ^ 1));
        }
        if (ST < 0 && kt + 1 < KT) next.store(sA(buf ^ 1), sB(buf ^ 1));
        __syncthreads();
    };
    if constexpr (PF == 1) {
        for (int kt = 0; kt < KT; ++kt) step(kt, ld[0], ld[0]);
    } else {
        int kt = 0;
        for (; kt + 1 < KT; kt += 2) {
            step(kt, ld[0], ld[1]);
            step(kt + 1, ld[1], ld[0]);
        }
        if (kt < KT) step(kt, ld[0], ld[1]);
    }

    // acc[i][j][r] = C[wm*WTM + 32i + 8*(r/4) + 4*(lane/32) + r%4][wn*WTN + 32j + lane%32]
    const int rbase = m0 + wm * C::WTM + 4 * (lane >> 5);
    if constexpr (SWIGLU) {
        const int D = N >> 1;
#pragma unroll
        for (int j = 0; j < C::NT / 2; ++j) {
            const int col = ntile * (C::BN / 2) + wn * (C::WTN / 2) + 32 * j + (lane & 31);
            if (col >= D) continue;
#pragma unroll
            for (int i = 0; i < C::MT; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = rbase + 32 * i + 8 * (r >> 2) + (r & 3);
                    if (row < M)
                        y[(int64_t)row * ldy + col] = swiglu_bf16_bits(
                            f32_to_bf16_bits(acc[i][j][r]), f32_to_bf16_bits(acc[i][j + C::NT / 2][r]));
                }
        }
    } else {
#pragma unroll
        for (int j = 0; j < C::NT; ++j) {
            const int col = ntile * C::BN + wn * C::WTN + 32 * j + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int i = 0; i < C::MT; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = rbase + 32 * i + 8 * (r >> 2) + (r & 3);
                    if (row < M) y[(int64_t)row * ldy + col] = f32_to_bf16_bits(acc[i][j][r]);
                }
        }
    }
}

// Dynamic LDS above the default limit needs an explicit per-kernel opt-in
// (once per process; gfx950 has 160 KiB per workgroup).
inline hipError_t allow_lds(const void* kern, int bytes) {
    return hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

template <class C, bool FP8, bool SWIGLU, int GROUP_N, int IGLP = -1, int PF = 1, int ST = -1>
hipError_t launch(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
                  int64_t ldy, int M, int N, int K, hipStream_t stream) {
    const int mtiles = (M + C::BM - 1) / C::BM;
    const int ntiles = SWIGLU ? ((N >> 1) + C::BN / 2 - 1) / (C::BN / 2) : (N + C::BN - 1) / C::BN;
    // The aligned path uses raw-buffer loads with 32-bit byte offsets.
    const int64_t wbytes = (int64_t)N * K * (FP8 ? 1 : 2);
    const bool aligned = (K % C::BK == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(w) % 16 == 0) &&
                         (int64_t)M * K * 2 < ((int64_t)1 << 31) && wbytes < ((int64_t)1 << 31);
    const int per_xcd = (mtiles * ntiles + kXcds - 1) / kXcds;
    const dim3 grid(per_xcd * kXcds);
    if (aligned) {
        auto kern = gemm_kernel<C, FP8, false, SWIGLU, GROUP_N, IGLP, PF, ST>;
        static const hipError_t attr = allow_lds(reinterpret_cast<const void*>(kern), C::LDS_BYTES);
        if (attr != hipSuccess) return attr;
        hipLaunchKernelGGL(kern, grid, dim3(C::THREADS), C::LDS_BYTES, stream, x, w, scales, S, y, ldy,
                           M, N, K, mtiles, ntiles);
    } else {
        auto kern = gemm_kernel<C, FP8, true, SWIGLU, GROUP_N, IGLP, 1, -1>;
        static const hipError_t attr = allow_lds(reinterpret_cast<const void*>(kern), C::LDS_BYTES);
        if (attr != hipSuccess) return attr;
        hipLaunchKernelGGL(kern, grid, dim3(C::THREADS), C::LDS_BYTES, stream, x, w, scales, S, y, ldy,
                           M, N, K, mtiles, ntiles);
    }
    return hipGetLastError();
}

}  // namespace gemm
}  // namespace fp8lin
