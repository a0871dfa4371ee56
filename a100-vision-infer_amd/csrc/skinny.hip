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
// C[act row 4 (lane/16) + i][weight row lane%16].
//
// K advances in rounds of 512.  A round's 16 activation rows and 16 weight
// rows go HBM/L2 -> registers -> LDS as whole row segments (one 1 KiB row per
// load instruction, half a row of FP8 codes per 32 lanes): two register
// stages and two LDS buffers, a round's loads issued two rounds before its
// MFMAs, one barrier per round.  Wave w then reads its fragments for K [128 w, 128 w + 128) of
// the round from LDS (4 MFMAs); FP8 codes are converted at the reference
// rounding point bf16(decode(c) * s) (src/optimized.cu:32).  The four wave
// partials are added in LDS in wave order.  A row's sum depends on its K and
// data only, not on its slot or workgroup, so the fused SwiGLU form is
// fused_swiglu of the plain form's outputs bit for bit.
#include "device.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

constexpr int kSkWaves = 4;
constexpr int kSkKc = 512;              // K per round
constexpr int kSkRow = kSkKc * 2 + 16;  // LDS bytes per row (padded)

// Requirements (checked by the host): K % 32 == 0; x and w 16-byte aligned;
// FP8: S == K / 128 (K % 128 == 0) or S == 1 (one scale per row); M * K * 2,
// N * K * (FP8 ? 1 : 2) and N * S * 4 below 2^31.
template <bool FP8, bool SWIGLU>
__global__ __launch_bounds__(64 * kSkWaves) void skinny_mfma_kernel(const uint16_t* __restrict__ x,
                                                                   const void* __restrict__ w,
                                                                   const float* __restrict__ scales, int S,
                                                                   uint16_t* __restrict__ y, int64_t ldy, int M,
                                                                   int N, int K) {
    __shared__ __align__(16) uint8_t xs[2][16 * kSkRow];
    __shared__ __align__(16) uint8_t wsh[2][16 * kSkRow];
    __shared__ float ssc[2][16][4];  // FP8: scale of slot row, 128-K block of the round
    __shared__ float red[kSkWaves][16][16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.x * 16;
    const int half = N >> 1;
    // weight row of slot i, or -1
    auto slot_row = [&](int i) __attribute__((always_inline)) -> int {
        if constexpr (SWIGLU) {
            const int p = blockIdx.y * 8 + (i & 7);
            return p < half ? (i < 8 ? p : half + p) : -1;
        } else {
            const int c = blockIdx.y * 16 + i;
            return c < N ? c : -1;
        }
    };
    const rsrc_t rx = make_rsrc(x, (uint32_t)((int64_t)M * K * 2));
    const rsrc_t rw = make_rsrc(w, (uint32_t)((int64_t)N * K * (FP8 ? 1 : 2)));
    const rsrc_t rs = make_rsrc(scales, FP8 ? (uint32_t)((int64_t)N * S * 4) : 0u);
    // Loader rows of this wave: activation rows and weight slots w, w + 4,
    // w + 8, w + 12 (BF16 weights); FP8 codes: 2 slots per instruction,
    // w and w + 4 from lanes < 32 and >= 32, then w + 8 and w + 12.
    uint32_t xoff[4], woff[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int mm = m0 + wave + 4 * q;
        xoff[q] = mm < M ? (uint32_t)((int64_t)mm * K * 2) : kBufferOob;
        if constexpr (FP8) {
            const int slot = wave + 4 * (2 * q + (lane >> 5));
            const int n = slot_row(slot);
            woff[q] = q < 2 && n >= 0 ? (uint32_t)((int64_t)n * K) : kBufferOob;
        } else {
            const int n = slot_row(wave + 4 * q);
            woff[q] = n >= 0 ? (uint32_t)((int64_t)n * K * 2) : kBufferOob;
        }
    }
    // FP8 scales of a round: lane l < 64 of wave 0 -> slot l / 4, block l % 4
    const int sn = slot_row(lane >> 2);
    // two register stages: round rd's loads go to stage rd % 2, issued two
    // rounds before its MFMAs
    u32x4 xl[2][4], wl[2][4];
    float sl[2] = {0.0f, 0.0f};
    auto load_round = [&]<int ST>(int rd) __attribute__((always_inline)) {
        const int k0 = rd * kSkKc;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int kx = k0 + 8 * lane;
            xl[ST][q] = buf_load16<0>(rx, xoff[q] != kBufferOob && kx < K ? xoff[q] + (uint32_t)kx * 2u : kBufferOob);
            if constexpr (FP8) {
                if (q < 2) {
                    const int kw = k0 + 16 * (lane & 31);
                    wl[ST][q] = buf_load16<0>(rw, woff[q] != kBufferOob && kw < K ? woff[q] + (uint32_t)kw : kBufferOob);
                }
            } else {
                wl[ST][q] = buf_load16<0>(rw, woff[q] != kBufferOob && kx < K ? woff[q] + (uint32_t)kx * 2u : kBufferOob);
            }
        }
        if constexpr (FP8) {
            if (wave == 0) {
                const int blk = rd * (kSkKc / 128) + (lane & 3);
                const bool ok = sn >= 0 && blk * 128 < K;
                // blocks past K get a zero scale, so their zero codes stay zero
                sl[ST] = buf_load_f32(rs, ok ? (uint32_t)(((int64_t)sn * S + (S == 1 ? 0 : blk)) * 4) : kBufferOob);
            }
        }
    };
    // stage ST (round parity) into LDS buffer ST
    auto store_round = [&]<int ST>() __attribute__((always_inline)) {
        constexpr int b = ST;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            *reinterpret_cast<u32x4*>(&xs[b][(wave + 4 * q) * kSkRow + 16 * lane]) = xl[ST][q];
            if constexpr (FP8) {
                if (q < 2) {
                    const int slot = wave + 4 * (2 * q + (lane >> 5));
                    *reinterpret_cast<u32x4*>(&wsh[b][slot * kSkRow + 16 * (lane & 31)]) = wl[ST][q];
                }
            } else {
                *reinterpret_cast<u32x4*>(&wsh[b][(wave + 4 * q) * kSkRow + 16 * lane]) = wl[ST][q];
            }
        }
        if constexpr (FP8) {
            if (wave == 0) ssc[b][lane >> 2][lane & 3] = sl[ST];
        }
    };
    const int rounds = (K + kSkKc - 1) / kSkKc;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    // round rd: its stage into LDS buffer rd % 2, one barrier (that buffer's
    // previous round, rd - 2, is done in every wave), round rd + 2's loads
    // into the freed stage, then wave w's 4 MFMAs on K [128 w, 128 w + 128)
    auto do_round = [&]<int ST>(int rd) __attribute__((always_inline)) {
        constexpr int b = ST;
        store_round.template operator()<ST>();
        __syncthreads();
        if (rd + 2 < rounds) load_round.template operator()<ST>(rd + 2);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int kl = 128 * wave + 32 * s + 8 * g;  // K within the round
            const u32x4 a = *reinterpret_cast<const u32x4*>(&xs[b][r * kSkRow + 2 * kl]);
            u32x4 bw;
            if constexpr (FP8) {
                const u32x2 c = *reinterpret_cast<const u32x2*>(&wsh[b][r * kSkRow + kl]);
                const float sc = ssc[b][r][wave];
                uint32_t o[4];
                dequant4(c.x, sc, o[0], o[1]);
                dequant4(c.y, sc, o[2], o[3]);
                bw = u32x4{o[0], o[1], o[2], o[3]};
            } else {
                bw = *reinterpret_cast<const u32x4*>(&wsh[b][r * kSkRow + 2 * kl]);
            }
            // K past the end holds zeros (and zero scales), adding exact zeros
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                           __builtin_bit_cast(bf16x8, bw), acc, 0, 0, 0);
        }
    };
    load_round.template operator()<0>(0);
    if (rounds > 1) load_round.template operator()<1>(1);
    for (int rd = 0; rd < rounds; rd += 2) {
        do_round.template operator()<0>(rd);
        if (rd + 1 < rounds) do_round.template operator()<1>(rd + 1);
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
        const int ou = os + 8 < 16 ? os + 8 : os;
        float u = red[0][om][ou];
#pragma unroll
        for (int q = 1; q < kSkWaves; ++q) u = u + red[q][om][ou];
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
