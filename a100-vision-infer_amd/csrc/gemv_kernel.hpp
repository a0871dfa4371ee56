// Decode GEMV kernels for 1..8 activation rows sharing one pass over the
// weights (see gemv.hip for the dispatch and the numerics contract).
//
// A weight row is cut into 16-element chunks; lane l of a wave takes chunk
// c = l + 64*j of its rows at step j, so one wave step reads 1 KiB of
// contiguous codes per row with 128-bit loads.  Per chunk the 16 codes are
// converted with v_cvt_pk_f32_fp8, multiplied by the block scale, rounded to
// BF16 (v_cvt_pk_bf16_f32) and accumulated with v_dot2_f32_bf16.  A lane sums
// its chunks in step order; the 64 lane sums are then combined by a butterfly.
//
// Two kernels share that per-row order, so for one (K, W) they give the same
// bits whatever the load width, the weight type or the work distribution:
//  - gemv_kernel: W waves per workgroup split a row's steps (j = w, w+W, ...),
//    their sums are added in LDS in wave order; pointer loads, with a byte-load
//    variant for unaligned data or K % 16 != 0;
//  - gemv_ring_kernel: one wave owns R rows, the step loop is unrolled so every
//    load of the row group is issued up front (W = 1 order).  It uses raw
//    buffer loads: a masked lane gets an out-of-range offset and reads zeros,
//    so there is no branch around any load and the hardware wait counters let
//    the loads run ahead of the arithmetic.
#pragma once
#include "device.hpp"

namespace fp8lin {
namespace gemv {

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

// ------------------------------------------------------------ pointer loads
template <bool NT>
__device__ __forceinline__ u32x4 ld16(const void* p) {
    if constexpr (NT) return load_u32x4_stream(p);
    return load_u32x4(p);
}

template <bool FP8, bool WIDE, bool NT>
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
            ch.codes = ld16<NT>(wr + k0);
        } else {
            uint32_t v[4];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                uint32_t word = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int k = k0 + d * 4 + b;
                    const uint32_t byte = k < K ? (uint32_t)wr[k] : 0u;
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
            ch.lo = ld16<NT>(wr + k0);
            ch.hi = ld16<NT>(wr + k0 + 8);
        } else {
            uint32_t v[8];
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                const int k = k0 + 2 * d;
                const uint32_t a = k < K ? (uint32_t)wr[k] : 0u;
                const uint32_t b = k + 1 < K ? (uint32_t)wr[k + 1] : 0u;
                v[d] = a | (b << 16);
            }
            ch.lo = u32x4{v[0], v[1], v[2], v[3]};
            ch.hi = u32x4{v[4], v[5], v[6], v[7]};
        }
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
        const u32x4 a = load_u32x4(xr + k0), b = load_u32x4(xr + k0 + 8);
        xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
        xv[4] = b.x; xv[5] = b.y; xv[6] = b.z; xv[7] = b.w;
    } else {
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            const int k = k0 + 2 * d;
            const uint32_t a = k < K ? (uint32_t)xr[k] : 0u;
            const uint32_t b = k + 1 < K ? (uint32_t)xr[k + 1] : 0u;
            xv[d] = a | (b << 16);
        }
    }
}

// ------------------------------------------------------------- buffer loads
// Offsets are 32-bit: the host only uses these for matrices below 2 GiB.
struct Buffers {
    rsrc_t w, s, x;
};

__device__ __forceinline__ Buffers make_buffers(const uint16_t* x, const void* w,
                                                const float* scales, int S, int M, int N, int K,
                                                bool fp8) {
    Buffers b;
    b.w = make_rsrc(w, (uint32_t)((int64_t)N * K * (fp8 ? 1 : 2)));
    b.s = make_rsrc(scales, fp8 ? (uint32_t)((int64_t)N * S * 4) : 0u);
    b.x = make_rsrc(x, (uint32_t)((int64_t)M * K * 2));
    return b;
}

template <bool FP8, int AUX>
__device__ __forceinline__ void load_chunk_buf(Chunk<FP8>& ch, const Buffers& b, int S, int64_t row,
                                               int K, int k0, bool valid) {
    if constexpr (FP8) {
        const uint32_t off = valid ? (uint32_t)(row * K + k0) : kBufferOob;
        const uint32_t soff = valid ? (uint32_t)((row * S + (S == 1 ? 0 : (k0 >> 7))) * 4) : kBufferOob;
        ch.codes = buf_load16<AUX>(b.w, off);
        ch.scale = buf_load_f32(b.s, soff);
    } else {
        const uint32_t off = valid ? (uint32_t)((row * K + k0) * 2) : kBufferOob;
        ch.lo = buf_load16<AUX>(b.w, off);
        ch.hi = buf_load16<AUX>(b.w, valid ? off + 16 : kBufferOob);
    }
}

__device__ __forceinline__ void load_x_buf(uint32_t (&xv)[8], const Buffers& b, int m, int K,
                                           int k0, bool valid) {
    const uint32_t off = valid ? (uint32_t)((m * K + k0) * 2) : kBufferOob;
    const u32x4 a = buf_load16<0>(b.x, off);
    const u32x4 c = buf_load16<0>(b.x, valid ? off + 16 : kBufferOob);
    xv[0] = a.x; xv[1] = a.y; xv[2] = a.z; xv[3] = a.w;
    xv[4] = c.x; xv[5] = c.y; xv[6] = c.z; xv[7] = c.w;
}

// ------------------------------------------------------------------- shared
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

// acc[r][m] += dot(weights of chunk r, activations of row m)
template <int R, int MR, bool FP8>
__device__ __forceinline__ void accumulate(float (&acc)[R][MR], const Chunk<FP8> (&ch)[R],
                                           const uint32_t (&xv)[MR][8]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        uint32_t wv[8];
        chunk_to_bf16<FP8>(ch[r], wv);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float a = acc[r][m];
#pragma unroll
            for (int i = 0; i < 8; ++i) a = dot2_bf16(wv[i], xv[m][i], a);
            acc[r][m] = a;
        }
    }
}

// Weight row held by slot r of row group g (and whether it exists).
template <int R, bool SWIGLU>
__device__ __forceinline__ int64_t slot_row(int64_t g, int r, int N, bool& ok) {
    if constexpr (SWIGLU) {
        const int64_t D = N >> 1;
        const int64_t j = g * (R / 2) + (r % (R / 2));
        ok = j < D;
        const int64_t row = r < R / 2 ? j : D + j;
        return ok ? row : 0;
    } else {
        const int64_t row = g * R + r;
        ok = row < N;
        return ok ? row : 0;
    }
}

// Store the R x MR totals of a row group (lane 0 calls this).
template <int R, int MR, bool SWIGLU>
__device__ __forceinline__ void store_group(uint16_t* __restrict__ y, int64_t ldy, int M,
                                            const int64_t (&rows)[R], const bool (&ok)[R],
                                            const float (&tot)[R][MR]) {
    if constexpr (SWIGLU) {
#pragma unroll
        for (int r = 0; r < R / 2; ++r) {
            if (!ok[r]) continue;
#pragma unroll
            for (int m = 0; m < MR; ++m)
                if (m < M)
                    y[(int64_t)m * ldy + rows[r]] = swiglu_bf16_bits(
                        f32_to_bf16_bits(tot[r][m]), f32_to_bf16_bits(tot[r + R / 2][m]));
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (!ok[r]) continue;
#pragma unroll
            for (int m = 0; m < MR; ++m)
                if (m < M) y[(int64_t)m * ldy + rows[r]] = f32_to_bf16_bits(tot[r][m]);
        }
    }
}

__device__ __forceinline__ int group_count(int N, int R, bool swiglu) {
    return swiglu ? ((N >> 1) + R / 2 - 1) / (R / 2) : (N + R - 1) / R;
}

// ------------------------------------------------- W-split kernel (general)
// MR: compile-time bound on activation rows (runtime M <= MR).  R: weight rows
// per workgroup (even for SWIGLU).  W: waves per workgroup.  NT: non-temporal
// weight loads.  WIDE: 128-bit loads (K % 16 == 0, 16-byte aligned pointers),
// else byte loads.
// gridDim.y > 1: block y takes activation rows [y * MR, y * MR + MR) (the
// prefill form for a few weight rows).
template <int MR, int R, int W, bool WIDE, bool FP8, bool SWIGLU, bool NT>
__global__ __launch_bounds__(64 * W) void gemv_kernel(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const float* __restrict__ scales,
    int S, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K) {
    if (blockIdx.y) {
        x += (int64_t)blockIdx.y * MR * K;
        y += (int64_t)blockIdx.y * MR * ldy;
        M = min(MR, M - (int)blockIdx.y * MR);
    }
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int64_t g = blockIdx.x;

    int64_t rows[R];
    bool row_ok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = slot_row<R, SWIGLU>(g, r, N, row_ok[r]);

    const int chunks = (K + 15) >> 4;
    const int steps = (chunks + kWave - 1) / kWave;

    float acc[R][MR];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = 0.0f;

    Chunk<FP8> cur[R];
    {
        const int c = lane + wave * kWave;
#pragma unroll
        for (int r = 0; r < R; ++r)
            load_chunk<FP8, WIDE, NT>(cur[r], w, scales, S, rows[r], K, c << 4,
                                      row_ok[r] && wave < steps && c < chunks);
    }
    for (int j = wave; j < steps; j += W) {
        const int c = lane + j * kWave;
        const int k0 = c << 4;
        const bool valid = c < chunks;
        Chunk<FP8> nxt[R];
        const int cn = c + W * kWave;
#pragma unroll
        for (int r = 0; r < R; ++r)
            load_chunk<FP8, WIDE, NT>(nxt[r], w, scales, S, rows[r], K, cn << 4,
                                      row_ok[r] && cn < chunks);
        uint32_t xv[MR][8];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const int mm = m < M ? m : M - 1;
            load_x<WIDE>(xv[m], x + (int64_t)mm * K, K, k0, valid);
        }
        accumulate<R, MR, FP8>(acc, cur, xv);
#pragma unroll
        for (int r = 0; r < R; ++r) cur[r] = nxt[r];
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = wave_sum(acc[r][m]);

    float total[R][MR];
    if constexpr (W == 1) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MR; ++m) total[r][m] = acc[r][m];
    } else {
        __shared__ float red[W][R * MR];
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < MR; ++m) red[wave][r * MR + m] = acc[r][m];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float t = red[0][r * MR + m];
#pragma unroll
                for (int v = 1; v < W; ++v) t += red[v][r * MR + m];
                total[r][m] = t;
            }
    }
    if (lane == 0) store_group<R, MR, SWIGLU>(y, ldy, M, rows, row_ok, total);
}

template <int MR, int R, int W, bool FP8, bool SWIGLU, bool NT>
hipError_t launch(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
                  int64_t ldy, int M, int N, int K, bool wide, hipStream_t stream) {
    const int64_t groups = SWIGLU ? ((N >> 1) + R / 2 - 1) / (R / 2) : ((int64_t)N + R - 1) / R;
    dim3 grid((unsigned)groups, (unsigned)((M + MR - 1) / MR));
    if (wide)
        hipLaunchKernelGGL((gemv_kernel<MR, R, W, true, FP8, SWIGLU, NT>), grid, dim3(64 * W), 0,
                           stream, x, w, scales, S, y, ldy, M, N, K);
    else
        hipLaunchKernelGGL((gemv_kernel<MR, R, W, false, FP8, SWIGLU, NT>), grid, dim3(64 * W), 0,
                           stream, x, w, scales, S, y, ldy, M, N, K);
    return hipGetLastError();
}

// ------------------------------------------------------ unrolled ring kernel
// K <= 1024 * MAXSTEPS, K % 16 == 0.  Each wave owns one row group of R rows;
// all loads of the row group are issued before the arithmetic.  WPG waves
// share a workgroup to cut the number of workgroups the dispatcher launches
// (measured 3-9% faster at the decode shapes with WPG = 4).  For wide weights
// (kSharedXRows) they also load the activations once per workgroup: x [M, K]
// goes to LDS by direct-to-LDS DMA (1 KiB per instruction, spread over the
// waves, issued before the weight loads), and each wave reads a step's
// fragments from there when it needs them; otherwise every wave loads its own
// x fragments, as many bytes as its weights, from L2.  Each wave still owns
// its rows alone.  ring_lds_bytes() is the dynamic LDS the shared form needs.
template <int MR, int WPG>
constexpr int ring_x_dmas(int K) {  // DMAs per wave (the same count in every wave)
    return (MR * K * 2 / 1024 + 1 + WPG - 1) / WPG;
}
template <int MR, int WPG, bool XS>
size_t ring_lds_bytes(int K) { return XS ? (size_t)ring_x_dmas<MR, WPG>(K) * WPG * 1024 : 0; }

__device__ __forceinline__ void ring_dma16(uint32_t m0v, uint32_t voff, rsrc_t r) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0v), "v"(voff), "s"(r)
                 : "memory", "m0");
}

// The R x MR wave-summed totals of row group g (every lane gets them).
// XS: the workgroup's activations through LDS (WPG > 1).
template <int MR, int R, int MAXSTEPS, bool FP8, bool SWIGLU, int AUX, int WPG, bool XS>
__device__ __forceinline__ void ring_group(const Buffers& b, int S, int M, int N, int K, int64_t g, int lane,
                                           int64_t (&rows)[R], bool (&row_ok)[R], float (&acc)[R][MR]) {
#pragma unroll
    for (int r = 0; r < R; ++r) rows[r] = slot_row<R, SWIGLU>(g, r, N, row_ok[r]);
    const int chunks = K >> 4;
    const int steps = (chunks + kWave - 1) / kWave;

    Chunk<FP8> ring[MAXSTEPS][R];
    uint32_t xv[MAXSTEPS][MR][8];
    extern __shared__ __align__(16) uint8_t xs[];  // [M][K] BF16, rows packed
    static_assert(!XS || WPG > 1, "shared activations need several waves");
    if constexpr (XS) {
        // x by DMA: instruction d of wave w moves bytes [1024 (w + WPG d), +1024)
        // of x (past M*K*2 the buffer returns zeros).
        const int wave = threadIdx.x / kWave;
        const int nd = ring_x_dmas<MR, WPG>(K);
        for (int d = 0; d < nd; ++d) {
            const uint32_t blk = (uint32_t)(wave + WPG * d);
            ring_dma16(__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)xs + blk * 1024u),
                       blk * 1024u + (uint32_t)lane * 16u, b.x);
        }
#pragma unroll
        for (int j = 0; j < MAXSTEPS; ++j) {
            const int c = lane + j * kWave;
#pragma unroll
            for (int r = 0; r < R; ++r)
                load_chunk_buf<FP8, AUX>(ring[j][r], b, S, rows[r], K, c << 4, row_ok[r] && c < chunks);
        }
        // this wave's DMAs are older than its 2 R MAXSTEPS weight loads
        asm volatile("s_waitcnt vmcnt(%0)" ::"i"(2 * R * MAXSTEPS) : "memory");
        __syncthreads();
    } else {
#pragma unroll
        for (int j = 0; j < MAXSTEPS; ++j) {
            const int c = lane + j * kWave;
#pragma unroll
            for (int r = 0; r < R; ++r)
                load_chunk_buf<FP8, AUX>(ring[j][r], b, S, rows[r], K, c << 4, row_ok[r] && c < chunks);
#pragma unroll
            for (int m = 0; m < MR; ++m) load_x_buf(xv[j][m], b, m < M ? m : M - 1, K, c << 4, c < chunks);
        }
    }
    // a step's activation fragments from LDS (XS)
    auto x_step = [&](int j) __attribute__((always_inline)) {
        if constexpr (XS) {
            const int c = lane + j * kWave;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const int mm = m < M ? m : M - 1;
                u32x4 lo{0u, 0u, 0u, 0u}, hi{0u, 0u, 0u, 0u};
                if (c < chunks) {
                    const u32x4* p = reinterpret_cast<const u32x4*>(xs + ((int64_t)mm * K + (c << 4)) * 2);
                    lo = p[0];
                    hi = p[1];
                }
                xv[j][m][0] = lo.x; xv[j][m][1] = lo.y; xv[j][m][2] = lo.z; xv[j][m][3] = lo.w;
                xv[j][m][4] = hi.x; xv[j][m][5] = hi.y; xv[j][m][6] = hi.z; xv[j][m][7] = hi.w;
            }
        }
    };
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXSTEPS; ++j) {
        // keep each step's LDS reads in its step (hoisted, all steps'
        // fragments would be live at once): the previous step's sums are
        // finished before this step's reads issue
        if constexpr (XS) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < MR; ++m) asm volatile("" : "+v"(acc[r][m])::"memory");
        }
        x_step(j);
        // Steps past the end leave acc untouched (a select, not a branch).
        float nxt[R][MR];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MR; ++m) nxt[r][m] = acc[r][m];
        accumulate<R, MR, FP8>(nxt, ring[j], xv[j]);
        const bool live = j < steps;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[r][m] = live ? nxt[r][m] : acc[r][m];
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[r][m] = wave_sum(acc[r][m]);
}

template <int MR, int R, int MAXSTEPS, bool FP8, bool SWIGLU, int AUX, int WPG, bool XS>
__global__ __launch_bounds__(64 * WPG) void gemv_ring_kernel(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const float* __restrict__ scales,
    int S, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t g = (int64_t)blockIdx.x * WPG + threadIdx.x / kWave;
    const Buffers b = make_buffers(x, w, scales, S, M, N, K, FP8);
    int64_t rows[R];
    bool row_ok[R];
    float acc[R][MR];
    ring_group<MR, R, MAXSTEPS, FP8, SWIGLU, AUX, WPG, XS>(b, S, M, N, K, g, lane, rows, row_ok, acc);
    if (lane == 0) store_group<R, MR, SWIGLU>(y, ldy, M, rows, row_ok, acc);
}

// Two weights at one activation row in one launch: workgroups [0, blocks_a)
// run the FP8 weight's ring groups (two rows per wave, two waves), the rest
// the BF16 weight's rows (one per wave) -- the GDN in_proj_all group's 8192
// FP8 and 48 BF16 rows, whose second launch would pay its own ramp.  Each
// part's rows are summed exactly as in its own launch (a wave owns its rows,
// activations are not shared through LDS in either), so the outputs are
// those of the two launches bit for bit.
template <int MAXSTEPS, int AUX>
__global__ __launch_bounds__(128) void gemv_ring_pair_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ wa, const float* __restrict__ sa, int sa_cols,
    uint16_t* __restrict__ ya, int na, const uint16_t* __restrict__ wb, uint16_t* __restrict__ yb, int nb,
    int64_t ldy, int K, int blocks_a) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    if ((int)blockIdx.x < blocks_a) {
        const int64_t g = (int64_t)blockIdx.x * 2 + wave;
        const Buffers b = make_buffers(x, wa, sa, sa_cols, 1, na, K, true);
        int64_t rows[2];
        bool row_ok[2];
        float acc[2][1];
        ring_group<1, 2, MAXSTEPS, true, false, AUX, 2, false>(b, sa_cols, 1, na, K, g, lane, rows, row_ok, acc);
        if (lane == 0) store_group<2, 1, false>(ya, ldy, 1, rows, row_ok, acc);
    } else {
        const int64_t g = (int64_t)(blockIdx.x - blocks_a) * 2 + wave;
        const Buffers b = make_buffers(x, wb, nullptr, 1, 1, nb, K, false);
        int64_t rows[1];
        bool row_ok[1];
        float acc[1][1];
        ring_group<1, 1, MAXSTEPS, false, false, AUX, 2, false>(b, 1, 1, nb, K, g, lane, rows, row_ok, acc);
        if (lane == 0) store_group<1, 1, false>(yb, ldy, 1, rows, row_ok, acc);
    }
}

// The ring kernel with the output head's candidate epilogue: no logits are
// written.  Each workgroup rounds its rows' totals to BF16 (the logits
// fp8lin_linear would store) and writes, per activation row m, the best
// {value bits, column} of its WPG * R columns to one of the row's
// 8 * ceil(gridDim.x / 8) pair slots under the candidate order (larger value,
// then smaller column; NaN as +inf).  Workgroup b writes slot
// (b % 8) * ceil(gridDim.x / 8) + b / 8; the finishing launch skips the slots
// no workgroup writes.  A finishing launch reduces the pairs of a row; its
// per-row arrival counters are cleared here (workgroup 0), so they start at
// zero whatever the workspace held.
template <int MR, int R, int MAXSTEPS, int AUX, int WPG, bool XS>
__global__ __launch_bounds__(64 * WPG) void gemv_ring_cand_kernel(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const float* __restrict__ scales,
    int S, int M, int N, int K, uint32_t* __restrict__ part, uint32_t* __restrict__ counters) {
    if (blockIdx.x == 0 && (int)threadIdx.x < M) counters[threadIdx.x] = 0;
    __shared__ float sv[WPG][MR];
    __shared__ uint32_t sid[WPG][MR];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int64_t g = (int64_t)blockIdx.x * WPG + wave;
    const Buffers b = make_buffers(x, w, scales, S, M, N, K, true);
    int64_t rows[R];
    bool row_ok[R];
    float acc[R][MR];
    ring_group<MR, R, MAXSTEPS, true, false, AUX, WPG, XS>(b, S, M, N, K, g, lane, rows, row_ok, acc);
    if (lane == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float best = -__builtin_inff();
            uint32_t id = 0xffffffffu;
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row_ok[r]) pick_bf16(best, id, f32_to_bf16_bits(acc[r][m]), (uint32_t)rows[r]);
            sv[wave][m] = best;
            sid[wave][m] = id;
        }
    }
    __syncthreads();
    if (threadIdx.x < MR && (int)threadIdx.x < M) {
        const int m = threadIdx.x;
        float best = sv[0][m];
        uint32_t id = sid[0][m];
#pragma unroll
        for (int v = 1; v < WPG; ++v) pick(best, id, sv[v][m], sid[v][m]);
        // Workgroup b runs on XCD b % 8: slot b / 8 of that XCD's contiguous
        // run of pairs, so a cache line of pairs is written from one L2.
        const int64_t nb = gridDim.x, per_xcd = (nb + 7) / 8, xcd = blockIdx.x % 8;
        const int64_t slot = xcd * per_xcd + blockIdx.x / 8;
        uint32_t* p = part + ((int64_t)m * 8 * per_xcd + slot) * 2;
        p[0] = __builtin_bit_cast(uint32_t, best);
        p[1] = id;
    }
}

// Activations through LDS from this many weight rows on (measured at the
// decode shapes: 75968- and 17408-row weights gain, 5120 and 4096 rows at
// K = 8704 and 4096 lose to the workgroup barrier).
constexpr int kSharedXRows = 16384;

template <int MR, int R, int MAXSTEPS, bool FP8, bool SWIGLU, int AUX, int WPG, bool XS>
hipError_t launch_ring_xs(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y, int64_t ldy,
                          int M, int N, int K, hipStream_t stream) {
    const int64_t groups = SWIGLU ? ((N >> 1) + R / 2 - 1) / (R / 2) : ((int64_t)N + R - 1) / R;
    const int64_t blocks = (groups + WPG - 1) / WPG;
    const size_t lds = ring_lds_bytes<MR, WPG, XS>(K);
    hipLaunchKernelGGL((gemv_ring_kernel<MR, R, MAXSTEPS, FP8, SWIGLU, AUX, WPG, XS>), dim3((unsigned)blocks),
                       dim3(64 * WPG), lds, stream, x, w, scales, S, y, ldy, M, N, K);
    return hipGetLastError();
}

template <int MR, int R, int MAXSTEPS, bool FP8, bool SWIGLU, int AUX, int WPG = 4>
hipError_t launch_ring(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
                       int64_t ldy, int M, int N, int K, hipStream_t stream) {
    if constexpr (WPG > 1) {
        if (N >= kSharedXRows)
            return launch_ring_xs<MR, R, MAXSTEPS, FP8, SWIGLU, AUX, WPG, true>(x, w, scales, S, y, ldy, M, N, K,
                                                                              stream);
    }
    return launch_ring_xs<MR, R, MAXSTEPS, FP8, SWIGLU, AUX, WPG, false>(x, w, scales, S, y, ldy, M, N, K, stream);
}

template <int MR, int R, int MAXSTEPS, int AUX, int WPG = 4>
int64_t ring_cand_blocks(int N) {
    return ((int64_t)N + (int64_t)R * WPG - 1) / ((int64_t)R * WPG);
}

template <int MR, int R, int MAXSTEPS, int AUX, int WPG, bool XS>
hipError_t launch_ring_cand_xs(const uint16_t* x, const void* w, const float* scales, int S, int M, int N, int K,
                               uint32_t* part, uint32_t* counters, hipStream_t stream) {
    const int64_t blocks = ring_cand_blocks<MR, R, MAXSTEPS, AUX, WPG>(N);
    const size_t lds = ring_lds_bytes<MR, WPG, XS>(K);
    hipLaunchKernelGGL((gemv_ring_cand_kernel<MR, R, MAXSTEPS, AUX, WPG, XS>), dim3((unsigned)blocks),
                       dim3(64 * WPG), lds, stream, x, w, scales, S, M, N, K, part, counters);
    return hipGetLastError();
}

template <int MR, int R, int MAXSTEPS, int AUX, int WPG = 4>
hipError_t launch_ring_cand(const uint16_t* x, const void* w, const float* scales, int S, int M, int N, int K,
                            uint32_t* part, uint32_t* counters, hipStream_t stream) {
    if (N >= kSharedXRows)
        return launch_ring_cand_xs<MR, R, MAXSTEPS, AUX, WPG, true>(x, w, scales, S, M, N, K, part, counters, stream);
    return launch_ring_cand_xs<MR, R, MAXSTEPS, AUX, WPG, false>(x, w, scales, S, M, N, K, part, counters, stream);
}

}  // namespace gemv
}  // namespace fp8lin
