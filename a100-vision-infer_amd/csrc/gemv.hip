// Decode GEMV for 1..8 activation rows sharing one pass over the weights.
//
// Reference numerics (src/optimized.cu:20-23, :42-60; src/deep_kernels.cu:23-63):
//   y[m,n] = bf16( sum_k x[m,k] * bf16(decode(code[n,k]) * scale[n, k/128]) )
// with FP32 accumulation.  The reference runs one 32-lane warp per weight row;
// here one 64-lane wave owns R weight rows and streams them with 128-bit loads:
// lane l handles 16-element chunks c = l, l+64, l+128, ... of each row, so one
// wave instruction reads 1 KiB of contiguous codes.  Per chunk the 16 codes
// are converted with v_cvt_pk_f32_fp8, multiplied by the row's block scale,
// rounded to BF16 with v_cvt_pk_bf16_f32 (the reference's rounding point) and
// accumulated with v_dot2_f32_bf16 against the matching BF16 activations.
// The K loop prefetches the next chunk's codes while the current one is
// converted.  The partial sums are combined with a butterfly over the wave.
//
// The accumulation order depends only on K: the byte-load fallback (unaligned
// pointers or K % 16 != 0) and the BF16-weight variant assemble the same
// registers and therefore produce bit-identical outputs, as the reference's
// tests require (tests/optimized_test.cpp:11-12, :57-62).
#include "device.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;

// One 16-element weight chunk, as 8 packed BF16 pairs.
template <bool FP8>
struct Chunk;

template <>
struct Chunk<true> {
    u32x4 codes;
    float scale;
};
template <>
struct Chunk<false> {
    u32x4 lo, hi;
};

template <bool FP8, bool WIDE>
__device__ __forceinline__ void load_chunk(Chunk<FP8>& ch, const void* __restrict__ w,
                                           const float* __restrict__ scales, int S, int64_t row,
                                           int K, int k0, bool valid) {
    if constexpr (FP8) {
        const uint8_t* wr = static_cast<const uint8_t*>(w) + row * (int64_t)K;
        if (!valid) {
            ch.codes = u32x4{0, 0, 0, 0};
            ch.scale = 0.0f;
            return;
        }
        ch.scale = scales[row * S + (S == 1 ? 0 : (k0 >> 7))];
        if constexpr (WIDE) {
            ch.codes = load_u32x4_stream(wr + k0);
        } else {
            uint32_t v[4];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                uint32_t word = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    int k = k0 + d * 4 + b;
                    uint32_t byte = k < K ? (uint32_t)wr[k] : 0u;
                    word |= byte << (8 * b);
                }
                v[d] = word;
            }
            ch.codes = u32x4{v[0], v[1], v[2], v[3]};
        }
    } else {
        const uint16_t* wr = static_cast<const uint16_t*>(w) + row * (int64_t)K;
        if (!valid) {
            ch.lo = u32x4{0, 0, 0, 0};
            ch.hi = u32x4{0, 0, 0, 0};
            return;
        }
        if constexpr (WIDE) {
            ch.lo = load_u32x4_stream(wr + k0);
            ch.hi = load_u32x4_stream(wr + k0 + 8);
        } else {
            uint32_t v[8];
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                int k = k0 + 2 * d;
                uint32_t a = k < K ? (uint32_t)wr[k] : 0u;
                uint32_t b = k + 1 < K ? (uint32_t)wr[k + 1] : 0u;
                v[d] = a | (b << 16);
            }
            ch.lo = u32x4{v[0], v[1], v[2], v[3]};
            ch.hi = u32x4{v[4], v[5], v[6], v[7]};
        }
    }
}

template <bool FP8>
__device__ __forceinline__ void chunk_to_bf16(const Chunk<FP8>& ch, uint32_t (&wv)[8]) {
    if constexpr (FP8) {
        dequant4(ch.codes.x, ch.scale, wv[0], wv[1]);
        dequant4(ch.codes.y, ch.scale, wv[2], wv[3]);
        dequant4(ch.codes.z, ch.scale, wv[4], wv[5]);
        dequant4(ch.codes.w, ch.scale, wv[6], wv[7]);
    } else {
        wv[0] = ch.lo.x; wv[1] = ch.lo.y; wv[2] = ch.lo.z; wv[3] = ch.lo.w;
        wv[4] = ch.hi.x; wv[5] = ch.hi.y; wv[6] = ch.hi.z; wv[7] = ch.hi.w;
    }
}

template <bool WIDE>
__device__ __forceinline__ void load_x(uint32_t (&xv)[8], const uint16_t* __restrict__ xr, int K,
                                       int k0, bool valid) {
    if (!valid) {
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] = 0;
        return;
    }
    if constexpr (WIDE) {
        u32x4 a = load_u32x4(xr + k0), b = load_u32x4(xr + k0 + 8);
        xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
        xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
    } else {
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            int k = k0 + 2 * d;
            uint32_t a = k < K ? (uint32_t)xr[k] : 0u;
            uint32_t b = k + 1 < K ? (uint32_t)xr[k + 1] : 0u;
            xv[d] = a | (b << 16);
        }
    }
}

// MR: compile-time bound on activation rows (runtime M <= MR); R: weight rows
// per wave.
template <int MR, int R, bool WIDE, bool FP8>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const float* __restrict__ scales,
    int S, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int64_t row0 = ((int64_t)blockIdx.x * kGemvWaves + wave) * R;
    if (row0 >= N) return;
    int64_t rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = row0 + r < N ? row0 + r : (int64_t)N - 1;

    const int chunks = (K + 15) >> 4;
    const int steps = (chunks + kWave - 1) / kWave;

    float acc[R][MR];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = 0.0f;

    Chunk<FP8> cur[R];
    {
        const int c = lane;
#pragma unroll
        for (int r = 0; r < R; ++r)
            load_chunk<FP8, WIDE>(cur[r], w, scales, S, rows[r], K, c << 4, c < chunks);
    }
    for (int j = 0; j < steps; ++j) {
        const int c = lane + j * kWave;
        const int k0 = c << 4;
        const bool valid = c < chunks;
        Chunk<FP8> nxt[R];
        const int cn = c + kWave;
#pragma unroll
        for (int r = 0; r < R; ++r)
            load_chunk<FP8, WIDE>(nxt[r], w, scales, S, rows[r], K, cn << 4, cn < chunks);

        uint32_t xv[MR][8];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const int mm = m < M ? m : M - 1;
            load_x<WIDE>(xv[m], x + (int64_t)mm * K, K, k0, valid);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t wv[8];
            chunk_to_bf16<FP8>(cur[r], wv);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float a = acc[r][m];
#pragma unroll
                for (int i = 0; i < 8; ++i) a = dot2_bf16(wv[i], xv[m][i], a);
                acc[r][m] = a;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) cur[r] = nxt[r];
    }

#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float total = wave_sum(acc[r][m]);
            if (lane == 0 && m < M && row0 + r < N) y[(int64_t)m * ldy + row0 + r] = f32_to_bf16_bits(total);
        }
    }
}

template <int MR, int R, bool FP8>
hipError_t launch_gemv_mr(const uint16_t* x, const void* w, const float* scales, int S,
                          uint16_t* y, int64_t ldy, int M, int N, int K, bool wide,
                          hipStream_t stream) {
    const int rows_per_block = kGemvWaves * R;
    dim3 grid((N + rows_per_block - 1) / rows_per_block);
    if (wide)
        hipLaunchKernelGGL((gemv_kernel<MR, R, true, FP8>), grid, dim3(kGemvThreads), 0, stream,
                           x, w, scales, S, y, ldy, M, N, K);
    else
        hipLaunchKernelGGL((gemv_kernel<MR, R, false, FP8>), grid, dim3(kGemvThreads), 0, stream,
                           x, w, scales, S, y, ldy, M, N, K);
    return hipGetLastError();
}

template <bool FP8>
hipError_t launch_gemv_t(const uint16_t* x, const void* w, const float* scales, int S,
                         uint16_t* y, int64_t ldy, int M, int N, int K, bool wide,
                         hipStream_t stream) {
    if (M <= 1) return launch_gemv_mr<1, 4, FP8>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
    if (M <= 2) return launch_gemv_mr<2, 4, FP8>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
    if (M <= 4) return launch_gemv_mr<4, 2, FP8>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
    return launch_gemv_mr<8, 2, FP8>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
}

}  // namespace

hipError_t launch_gemv(const uint16_t* x, const void* w, bool fp8, const float* scales, int S,
                       uint16_t* y, int64_t ldy, int M, int N, int K, bool wide,
                       hipStream_t stream) {
    if (fp8) return launch_gemv_t<true>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
    return launch_gemv_t<false>(x, w, nullptr, 1, y, ldy, M, N, K, wide, stream);
}

}  // namespace fp8lin
