// Few weight rows against many activation rows: the prefill form for
// N <= kSkinnyRows (the GDN in_proj_all group's 48 BF16 rows at a prefill
// chunk, src/engine.cpp:199), where 256x256 GEMM tiles would leave most CUs
// idle and the GEMV's prefill form re-reads 8 activation rows per 4 weight
// rows.
//
// One workgroup per 16 activation rows x 16 weight rows (for SwiGLU: 8 gate
// rows in slots 0..7 and the matching up rows in slots 8..15), so every
// output tile is one v_mfma_f32_16x16x32_bf16 accumulator: activation rows are
// the A operand (lane: row lane%16, K sub-range lane/16), weight rows the B
// operand (lane: row lane%16, the same K sub-range), so acc[i] =
// C[act row 4 (lane/16) + i][weight row lane%16].  The 4 waves take the 32-K
// steps w, w + 4, ... and load both operands straight from L2/HBM with raw
// buffer loads (rows past M or N read zeros); FP8 codes are converted at the
// reference rounding point bf16(decode(c) * s) (src/optimized.cu:32).  The
// four wave partials are added in LDS in wave order.  A row's sum depends on
// its K and data only, not on its slot or workgroup, so the fused SwiGLU form
// is fused_swiglu of the plain form's outputs bit for bit.
#include "device.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

constexpr int kSkWaves = 4;
constexpr int kSkUnroll = 8;  // steps per wave whose loads are in flight together

// Requirements (checked by the host): K % 32 == 0; x and w 16-byte aligned;
// FP8: S == K / 128 (K % 128 == 0) or S == 1 (one scale per row); M * K * 2,
// N * K * (FP8 ? 1 : 2) and N * S * 4 below 2^31.
template <bool FP8, bool SWIGLU>
__global__ __launch_bounds__(64 * kSkWaves) void skinny_mfma_kernel(const uint16_t* __restrict__ x,
                                                                   const void* __restrict__ w,
                                                                   const float* __restrict__ scales, int S,
                                                                   uint16_t* __restrict__ y, int64_t ldy, int M,
                                                                   int N, int K) {
    __shared__ float red[kSkWaves][16][16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.x * 16;
    const int half = N >> 1;
    // weight row of this lane's slot r, or -1
    int n;
    if constexpr (SWIGLU) {
        const int p = blockIdx.y * 8 + (r & 7);
        n = p < half ? (r < 8 ? p : half + p) : -1;
    } else {
        const int c = blockIdx.y * 16 + r;
        n = c < N ? c : -1;
    }
    const int m = m0 + r;
    const rsrc_t rx = make_rsrc(x, (uint32_t)((int64_t)M * K * 2));
    const rsrc_t rw = make_rsrc(w, (uint32_t)((int64_t)N * K * (FP8 ? 1 : 2)));
    const rsrc_t rs = make_rsrc(scales, FP8 ? (uint32_t)((int64_t)N * S * 4) : 0u);
    const uint32_t xrow = m < M ? (uint32_t)((int64_t)m * K * 2) : kBufferOob;
    const uint32_t wrow = n >= 0 ? (uint32_t)((int64_t)n * K * (FP8 ? 1 : 2)) : kBufferOob;
    const uint32_t srow = n >= 0 ? (uint32_t)((int64_t)n * S * 4) : kBufferOob;
    const int steps = K >> 5;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j0 = wave; j0 < steps; j0 += kSkWaves * kSkUnroll) {
        u32x4 xa[kSkUnroll], wb[kSkUnroll];
        float sc[kSkUnroll];
#pragma unroll
        for (int u = 0; u < kSkUnroll; ++u) {
            const int s = j0 + kSkWaves * u;
            const bool ok = s < steps;
            const int k = 32 * s + 8 * g;
            xa[u] = buf_load16<0>(rx, ok && xrow != kBufferOob ? xrow + (uint32_t)k * 2u : kBufferOob);
            if constexpr (FP8) {
                const uint32_t off = ok && wrow != kBufferOob ? wrow + (uint32_t)k : kBufferOob;
                const auto v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rw, (int)off, 0, 0));
                wb[u] = u32x4{v.x, v.y, 0u, 0u};
                // a step past K reads a zero scale too (not the next row's,
                // which could be NaN and turn the zero codes into NaN)
                const uint32_t soff =
                    ok && srow != kBufferOob ? srow + (S == 1 ? 0u : (uint32_t)(k >> 7) * 4u) : kBufferOob;
                sc[u] = buf_load_f32(rs, soff);
            } else {
                wb[u] = buf_load16<0>(rw, ok && wrow != kBufferOob ? wrow + (uint32_t)k * 2u : kBufferOob);
            }
        }
#pragma unroll
        for (int u = 0; u < kSkUnroll; ++u) {
            u32x4 b = wb[u];
            if constexpr (FP8) {
                uint32_t o[4];
                dequant4(wb[u].x, sc[u], o[0], o[1]);
                dequant4(wb[u].y, sc[u], o[2], o[3]);
                b = u32x4{o[0], o[1], o[2], o[3]};
            }
            // steps past the end load zeros, so they add exact zeros
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[u]),
                                                           __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][4 * g + i][r] = acc[i];
    __syncthreads();
    // thread t: activation row t / 16, slot t % 16; the partials in wave order
    const int t = threadIdx.x, om = t >> 4, os = t & 15;
    float v = red[0][om][os];
#pragma unroll
    for (int q = 1; q < kSkWaves; ++q) v = v + red[q][om][os];
    const int mm = m0 + om;
    if (mm >= M) return;
    if constexpr (SWIGLU) {
        // slot os + 8 holds the up row of slot os's gate row
        float u = red[0][om][os + 8 < 16 ? os + 8 : os];
#pragma unroll
        for (int q = 1; q < kSkWaves; ++q) u = u + red[q][om][os + 8 < 16 ? os + 8 : os];
        const int p = blockIdx.y * 8 + os;
        if (os < 8 && p < half)
            y[(int64_t)mm * ldy + p] = swiglu_bf16_bits(f32_to_bf16_bits(v), f32_to_bf16_bits(u));
    } else {
        const int c = blockIdx.y * 16 + os;
        if (c < N) y[(int64_t)mm * ldy + c] = f32_to_bf16_bits(v);
    }
}

template <bool FP8, bool SWIGLU>
hipError_t launch_sk(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y, int64_t ldy, int M,
                     int N, int K, hipStream_t stream) {
    const int cols = SWIGLU ? ((N >> 1) + 7) / 8 : (N + 15) / 16;
    hipLaunchKernelGGL((skinny_mfma_kernel<FP8, SWIGLU>), dim3((unsigned)((M + 15) / 16), (unsigned)cols),
                       dim3(64 * kSkWaves), 0, stream, x, w, scales, S, y, ldy, M, N, K);
    return hipGetLastError();
}

}  // namespace

bool skinny_mfma_supported(const uint16_t* x, const void* w, bool fp8, int S, int64_t M, int64_t N, int64_t K) {
    const int64_t lim = (int64_t)1 << 31;
    const bool scales_ok = !fp8 || S == 1 || (K % 128 == 0 && S == K / 128);
    return M > 0 && N > 0 && K > 0 && K % 32 == 0 && scales_ok && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(w) % 16 == 0 && M * K * 2 < lim && N * K * (fp8 ? 1 : 2) < lim &&
           N * (int64_t)S * 4 < lim;
}

hipError_t launch_skinny_mfma(const uint16_t* x, const void* w, bool fp8, const float* scales, int S, uint16_t* y,
                              int64_t ldy, int M, int N, int K, bool swiglu, hipStream_t stream) {
    if (fp8)
        return swiglu ? launch_sk<true, true>(x, w, scales, S, y, ldy, M, N, K, stream)
                      : launch_sk<true, false>(x, w, scales, S, y, ldy, M, N, K, stream);
    return swiglu ? launch_sk<false, true>(x, w, nullptr, 1, y, ldy, M, N, K, stream)
                  : launch_sk<false, false>(x, w, nullptr, 1, y, ldy, M, N, K, stream);
}

}  // namespace fp8lin
