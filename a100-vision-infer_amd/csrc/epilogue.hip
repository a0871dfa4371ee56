// Decode epilogue and output-head kernels around the linear layers:
//   - RMSNorm and the fused residual add + RMSNorm that follows each
//     row-parallel projection (src/optimized.cu:71, src/dual_path.cu:12-28);
//   - the per-rank vocabulary candidates of the output head and their merge
//     across ranks (src/dual_path.cu:29-67,79-92);
//   - the multi-axis rotary embedding of the attention heads
//     (src/optimized.cu:77-78) and its fusion with the per-head q/k RMSNorm
//     on the QKV-gate projection output (src/engine.cpp:279-287).
#include <cmath>

#include "device.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

// Threads per row: one 8-element vector per thread up to D = 8192, so a
// decode row is read in one round of loads.  Depends on D only, so a row's
// result does not depend on how many rows share the launch.
constexpr int kNormMaxThreads = 1024;
int norm_threads(int D) {
    const int t = ((D + 7) / 8 + 63) / 64 * 64;
    return t < 64 ? 64 : (t > kNormMaxThreads ? kNormMaxThreads : t);
}

// Block sum of one float per thread: wave butterfly, then the wave sums in
// wave order.  Every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = scratch[0];
    for (int q = 1; q < waves; ++q) t += scratch[q];
    return t;
}

__device__ __forceinline__ uint32_t bf16_add(uint32_t a, uint32_t b) {
    return f32_to_bf16_bits(bf16_bits_to_f32(a) + bf16_bits_to_f32(b));
}

// One workgroup of norm_threads(D) threads per row.  Thread t owns elements
// 8t + 8Tj + [0, 8), j = 0, 1, ..., in that order whatever the load width, so
// the sum of squares -- and with it the output -- is the same for the
// residual form and for RMSNorm of the stored sum, as the reference requires
// (tests/dual_path_test.cpp:17).  VEC (D % 8 == 0, 16-byte aligned buffers):
// the first two vectors of each thread stay in registers between the passes
// and their weights are loaded before the block sum; further vectors are read
// back from the residual (or x) in the second pass.
//
// RED: `update` holds `ranks` partial outputs [ranks][rows][D] (the
// row-parallel projection's per-rank results, gathered); the update is
// bf16(sum over ranks in order, in FP32) -- the reference's reduce
// (src/engine.cpp:183-195) folded into the residual add.
template <bool RES, bool VEC, bool RED = false>
__global__ __launch_bounds__(kNormMaxThreads) void rms_kernel(const uint16_t* __restrict__ x,
                                                              const uint16_t* __restrict__ update,
                                                              const uint16_t* __restrict__ w,
                                                              uint16_t* __restrict__ residual,
                                                              uint16_t* __restrict__ y, int D, float eps,
                                                              int centered, int ranks = 0,
                                                              int64_t rank_stride = 0) {
    __shared__ float scratch[kNormMaxThreads / 64];
    const int64_t base = (int64_t)blockIdx.x * D;
    const int t = threadIdx.x, T = blockDim.x;
    const float c = centered ? 1.0f : 0.0f;
    float ss = 0.0f;
    if constexpr (VEC) {
        // first pass over one vector: residual (stored) or x bits, and its squares
        auto first = [&](int i0) __attribute__((always_inline)) -> u32x4 {
            u32x4 v = load_u32x4(x + base + i0);
            if constexpr (RES) {
                u32x4 u = load_u32x4(update + base + i0);
                if constexpr (RED) {
                    float sum[8];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        sum[2 * q] = bf16_bits_to_f32(u[q] & 0xffffu);
                        sum[2 * q + 1] = bf16_bits_to_f32(u[q] >> 16);
                    }
                    for (int r = 1; r < ranks; ++r) {
                        const u32x4 p = load_u32x4(update + r * rank_stride + base + i0);
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            sum[2 * q] += bf16_bits_to_f32(p[q] & 0xffffu);
                            sum[2 * q + 1] += bf16_bits_to_f32(p[q] >> 16);
                        }
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        u[q] = (uint32_t)f32_to_bf16_bits(sum[2 * q]) | ((uint32_t)f32_to_bf16_bits(sum[2 * q + 1]) << 16);
                }
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    v[q] = bf16_add(v[q] & 0xffffu, u[q] & 0xffffu) | (bf16_add(v[q] >> 16, u[q] >> 16) << 16);
                *reinterpret_cast<u32x4*>(residual + base + i0) = v;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float a = bf16_bits_to_f32(v[q] & 0xffffu), b = bf16_bits_to_f32(v[q] >> 16);
                ss = __builtin_fmaf(a, a, ss);
                ss = __builtin_fmaf(b, b, ss);
            }
            return v;
        };
        const int i0a = 8 * t, i0b = 8 * t + 8 * T;
        u32x4 ka = {0, 0, 0, 0}, kb = {0, 0, 0, 0}, wa = {0, 0, 0, 0}, wb = {0, 0, 0, 0};
        if (i0a < D) ka = first(i0a);
        if (i0b < D) kb = first(i0b);
        for (int i0 = i0b + 8 * T; i0 < D; i0 += 8 * T) first(i0);
        if (i0a < D) wa = load_u32x4(w + i0a);
        if (i0b < D) wb = load_u32x4(w + i0b);
        const float inv = rsqrtf(block_sum(ss, scratch) / (float)D + eps);
        auto norm = [&](uint32_t v, uint32_t wt) __attribute__((always_inline)) -> uint32_t {
            float n = bf16_bits_to_f32(v) * inv;
            if (!centered) n = bf16_bits_to_f32(f32_to_bf16_bits(n));
            return f32_to_bf16_bits(n * (bf16_bits_to_f32(wt) + c));
        };
        auto second = [&](int i0, const u32x4& v, const u32x4& wv) __attribute__((always_inline)) {
            u32x4 o;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                o[q] = norm(v[q] & 0xffffu, wv[q] & 0xffffu) | (norm(v[q] >> 16, wv[q] >> 16) << 16);
            *reinterpret_cast<u32x4*>(y + base + i0) = o;
        };
        if (i0a < D) second(i0a, ka, wa);
        if (i0b < D) second(i0b, kb, wb);
        const uint16_t* src = RES ? residual : x;
        for (int i0 = i0b + 8 * T; i0 < D; i0 += 8 * T)
            second(i0, load_u32x4(src + base + i0), load_u32x4(w + i0));
    } else {
        for (int i0 = 8 * t; i0 < D; i0 += 8 * T) {
            for (int j = 0; j < 8 && i0 + j < D; ++j) {
                float v = bf16_bits_to_f32(x[base + i0 + j]);
                if constexpr (RES) {
                    uint32_t u = update[base + i0 + j];
                    if constexpr (RED) {
                        float sum = bf16_bits_to_f32(u);
                        for (int q = 1; q < ranks; ++q) sum += bf16_bits_to_f32(update[q * rank_stride + base + i0 + j]);
                        u = f32_to_bf16_bits(sum);
                    }
                    const uint16_t r = (uint16_t)bf16_add(x[base + i0 + j], u);
                    residual[base + i0 + j] = r;
                    v = bf16_bits_to_f32(r);
                }
                ss = __builtin_fmaf(v, v, ss);
            }
        }
        const float inv = rsqrtf(block_sum(ss, scratch) / (float)D + eps);
        const uint16_t* src = RES ? residual : x;
        for (int i0 = 8 * t; i0 < D; i0 += 8 * T) {
            for (int j = 0; j < 8 && i0 + j < D; ++j) {
                float n = bf16_bits_to_f32(src[base + i0 + j]) * inv;
                if (!centered) n = bf16_bits_to_f32(f32_to_bf16_bits(n));
                y[base + i0 + j] = f32_to_bf16_bits(n * (bf16_bits_to_f32(w[i0 + j]) + c));
            }
        }
    }
}

// ---- vocabulary candidates ----
// Stage 1, grid (chunks, M) x 256 threads: the best of one 2048-column chunk
// of a row as {float bits, column} into part[(m * chunks + chunk) * 2].  One
// 16-byte load per thread (VEC: N % 8 == 0 and 16-byte aligned rows), so
// every chunk is one round of loads and a 75968-wide decode row spreads over
// 38 CUs.  Stage 2, grid M x 64 threads: the best of a row's chunks as
// out[2m] = value, out[2m+1] = column + offset (doubles).
constexpr int kVocabChunk = 2048;
constexpr int kVocabThreads = kVocabChunk / 8;

template <bool VEC>
__global__ __launch_bounds__(kVocabThreads) void vocab_partial_kernel(const uint16_t* __restrict__ logits, int N,
                                                                      int chunks, uint32_t* __restrict__ part) {
    __shared__ float sv[kVocabThreads / 64];
    __shared__ uint32_t sid[kVocabThreads / 64];
    const int t = threadIdx.x, chunk = blockIdx.x, m = blockIdx.y;
    const uint16_t* row = logits + (int64_t)m * N;
    float best = -__builtin_inff();
    uint32_t id = 0xffffffffu;
    if constexpr (VEC) {
        const int64_t i0 = (int64_t)chunk * kVocabChunk + 8 * t;
        if (i0 < N) {
            const u32x4 v = load_u32x4(row + i0);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                pick_bf16(best, id, v[q] & 0xffffu, (uint32_t)(i0 + 2 * q));
                pick_bf16(best, id, v[q] >> 16, (uint32_t)(i0 + 2 * q + 1));
            }
        }
    } else {
        uint32_t b[8];
        const int64_t i0 = (int64_t)chunk * kVocabChunk + t;
#pragma unroll
        for (int j = 0; j < 8; ++j) b[j] = i0 + j * kVocabThreads < N ? row[i0 + j * kVocabThreads] : 0u;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (i0 + j * kVocabThreads < N) pick_bf16(best, id, b[j], (uint32_t)(i0 + j * kVocabThreads));
    }
    wave_pick(best, id);
    const int lane = t & 63, wave = t >> 6;
    if (lane == 0) {
        sv[wave] = best;
        sid[wave] = id;
    }
    __syncthreads();
    if (t == 0) {
#pragma unroll
        for (int q = 1; q < kVocabThreads / 64; ++q) pick(best, id, sv[q], sid[q]);
        uint32_t* p = part + ((int64_t)m * chunks + chunk) * 2;
        p[0] = __builtin_bit_cast(uint32_t, best);
        p[1] = id;
    }
}

// THREADS threads per row; pairs are read as 8-byte words, UNROLL per thread
// in flight (branch-free raw buffer loads).
template <int THREADS, int UNROLL>
__global__ __launch_bounds__(THREADS) void vocab_finish_kernel(const uint32_t* __restrict__ part, int chunks,
                                                               int64_t offset, double* __restrict__ out) {
    __shared__ float sv[THREADS / 64];
    __shared__ uint32_t sid[THREADS / 64];
    const int m = blockIdx.x;
    // raw buffer loads: a pair past the row's end reads zeros instead of
    // branching, so all UNROLL loads of a thread issue back to back
    const rsrc_t r = make_rsrc(part + (int64_t)m * chunks * 2, (uint32_t)chunks * 8u);
    float best = -__builtin_inff();
    uint32_t id = 0xffffffffu;
    for (int c0 = threadIdx.x; c0 < chunks; c0 += UNROLL * THREADS) {
        u32x2 p[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
            p[u] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                                 r, (int)((uint32_t)(c0 + u * THREADS) * 8u), 0, 0));
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
            if (c0 + u * THREADS < chunks) pick(best, id, __builtin_bit_cast(float, p[u].x), p[u].y);
    }
    wave_pick(best, id);
    if constexpr (THREADS > 64) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        if (lane == 0) {
            sv[wave] = best;
            sid[wave] = id;
        }
        __syncthreads();
        if (threadIdx.x != 0) return;
#pragma unroll
        for (int q = 1; q < THREADS / 64; ++q) pick(best, id, sv[q], sid[q]);
    }
    if (threadIdx.x == 0) {
        out[2 * m] = (double)best;
        out[2 * m + 1] = (double)((int64_t)id + offset);
    }
}

// grid (kCandSlices, M) x 256 threads, over the pairs of nb workgroups in
// 8 XCD runs of ceil(nb / 8) slots (gemv_ring_cand_kernel's layout; slot
// (x, j) holds workgroup x + 8j, unwritten when that is nb or more).  Slice s
// of row m reduces slots [s * per, (s + 1) * per) in one round of loads and
// publishes its best pair;
// the slice workgroup that arrives last (device-scope counter, cleared by the
// producing kernel) reduces the kCandSlices slice pairs in slice order (any
// order gives the same pair: the candidate order is total) and writes out[m].
constexpr int kSliceThreads = 256;
__global__ __launch_bounds__(kSliceThreads) void cand_finish_sliced_kernel(const uint32_t* __restrict__ part,
                                                                           int nb, int per,
                                                                           uint32_t* __restrict__ slices,
                                                                           uint32_t* __restrict__ counters,
                                                                           int64_t offset, double* __restrict__ out) {
    __shared__ float sv[kSliceThreads / 64];
    __shared__ uint32_t sid[kSliceThreads / 64];
    __shared__ int last;
    const int s = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
    const int run = (nb + 7) / 8, chunks = 8 * run;
    const int lo = s * per, hi = min(chunks, lo + per);
    const rsrc_t r = make_rsrc(part + (int64_t)m * chunks * 2, (uint32_t)chunks * 8u);
    float best = -__builtin_inff();
    uint32_t id = 0xffffffffu;
    for (int c0 = lo + t; c0 < hi; c0 += 8 * kSliceThreads) {
        u32x2 p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            p[u] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                                 r, (int)((uint32_t)(c0 + u * kSliceThreads) * 8u), 0, 0));
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + u * kSliceThreads;
            if (c < hi && c / run + 8 * (c % run) < nb) pick(best, id, __builtin_bit_cast(float, p[u].x), p[u].y);
        }
    }
    wave_pick(best, id);
    const int lane = t & 63, wave = t >> 6;
    if (lane == 0) {
        sv[wave] = best;
        sid[wave] = id;
    }
    __syncthreads();
    if (t == 0) {
#pragma unroll
        for (int q = 1; q < kSliceThreads / 64; ++q) pick(best, id, sv[q], sid[q]);
        uint32_t* sp = slices + ((int64_t)m * kCandSlices + s) * 2;
        __hip_atomic_store(sp, __builtin_bit_cast(uint32_t, best), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(sp + 1, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // release the slice pair, then count this slice in
        const uint32_t before = __hip_atomic_fetch_add(counters + m, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last = before == (uint32_t)(kCandSlices - 1);
    }
    __syncthreads();
    if (!last) return;
    if (t < 64) {
        float b = -__builtin_inff();
        uint32_t i = 0xffffffffu;
        if (t < kCandSlices) {
            const uint32_t* sp = slices + ((int64_t)m * kCandSlices + t) * 2;
            b = __builtin_bit_cast(float, __hip_atomic_load(sp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            i = __hip_atomic_load(sp + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        wave_pick(b, i);
        if (t == 0) {
            out[2 * m] = (double)b;
            out[2 * m + 1] = (double)((int64_t)i + offset);
        }
    }
}

// One thread per row: the best candidate over ranks, -1 when any rank's entry
// is non-finite or its id is not an integer in [0, INT_MAX].
__global__ __launch_bounds__(128) void merge_candidates_kernel(const double* __restrict__ gathered, int ranks,
                                                               int64_t rows, int64_t* __restrict__ out) {
    const int64_t r = (int64_t)blockIdx.x * 128 + threadIdx.x;
    if (r >= rows) return;
    double best = -__builtin_inf();
    int64_t id = INT64_MAX;
    bool invalid = false;
    for (int k = 0; k < ranks; ++k) {
        const double v = gathered[(k * rows + r) * 2], raw = gathered[(k * rows + r) * 2 + 1];
        if (!__builtin_isfinite(v) || !__builtin_isfinite(raw) || raw < 0 || raw > 2147483647.0 ||
            raw != __builtin_floor(raw)) {
            invalid = true;
            continue;
        }
        const int64_t next = (int64_t)raw;
        if (v > best || (v == best && next < id)) {
            best = v;
            id = next;
        }
    }
    out[r] = invalid ? -1 : id;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// ---- rotary embedding ----
// Grid (T, ceil(heads / (4 * iters))): a workgroup of 4 waves takes `iters`
// groups of 4 heads of one token, one head per wave per iteration.  The
// token's cos/sin pairs are computed into LDS once per workgroup and shared by
// its heads; each wave stages one head row of D values in LDS.  Every wave
// runs `iters` iterations and reaches every barrier (`live` is false past the
// last head).  The launcher picks iters = 1 for short inputs (parallel heads:
// decode latency) and all heads per workgroup for long ones (one table per
// token); the arithmetic per element is the same either way.
constexpr int kRopeWaves = 4;

// cos and sin of pair f at token t, rounded to BF16 (src/optimized.cu:77):
// the axis is 1 for f mod 3 == 1 below 3*hs, 2 for f mod 3 == 2 below 3*ws,
// else 0; angle = float(pos) * powf(theta, -2f*f/R) in FP32.  The power is
// evaluated in FP64 as exp2(e * log2(theta)) (log2t = log2(theta), computed
// once per launch on the host; relative error about 2^-48) and rounded once
// to FP32, i.e. the correctly rounded powf except at near-halfway values
// (CUDA's powf is within 2 ulp of it); f = 0 gives 1 exactly, as
// powf(theta, -0) does.  At position p an ulp of the frequency moves the
// angle by about p * 2^-24 rad, so a library-dependent last bit would show
// at long contexts.
__device__ __forceinline__ float2 rope_cos_sin(const int64_t* __restrict__ pos, int T, int t, int f, int R,
                                               double log2t, int hs, int ws) {
    const int axis = (f % 3 == 1 && f < hs * 3) ? 1 : ((f % 3 == 2 && f < ws * 3) ? 2 : 0);
    const float e = -2.0f * (float)f / (float)R;
    const float freq = f == 0 ? 1.0f : (float)exp2((double)e * log2t);
    const float angle = (float)pos[(int64_t)axis * T + t] * freq;
    float s, c;
    sincosf(angle, &s, &c);
    return make_float2(bf16_bits_to_f32(f32_to_bf16_bits(c)), bf16_bits_to_f32(f32_to_bf16_bits(s)));
}

// bf16(bf16(x * co) + bf16(rotated * si)), the reference's rounding points.
__device__ __forceinline__ uint16_t rope_one(float x, float rotated, float co, float si) {
    const float a = bf16_bits_to_f32(f32_to_bf16_bits(x * co));
    const float b = bf16_bits_to_f32(f32_to_bf16_bits(rotated * si));
    return f32_to_bf16_bits(a + b);
}

// Dynamic LDS: cs[R/2] float2 (rounded up to 16 bytes, so the rows below are
// 16-byte aligned for the vector accesses), then kRopeWaves rows of D BF16
// values (row stride rounded up to 8 values).
__host__ __device__ constexpr size_t rope_rows_offset(int R) { return ((size_t)(R / 2) * 8 + 15) / 16 * 16; }
__host__ __device__ constexpr size_t rope_lds(int D, int R) {
    return rope_rows_offset(R) + (size_t)kRopeWaves * ((D + 7) / 8 * 8) * 2;
}

// Fills cs for token t (all threads).  Called after the row loads are
// issued, so the table's arithmetic overlaps their latency; the barrier that
// follows the row staging publishes it.
__device__ __forceinline__ void rope_table(float2* cs, const int64_t* __restrict__ pos, int T, int t, int R,
                                           double log2t, int hs, int ws) {
    for (int f = threadIdx.x; f < R / 2; f += 64 * kRopeWaves) cs[f] = rope_cos_sin(pos, T, t, f, R, log2t, hs, ws);
}

// The wave's row is in LDS; rotates pairs (f, f + R/2) in place (lane l takes
// f = l, l + 64, ...), barrier, then writes the row to y (16-byte stores when
// VEC).  `live` is wave-uniform; every wave reaches the barrier.  Row
// staging and the final copy use one ownership, lane l <-> 8-value chunks
// l, l + 64, ..., so the next iteration's staging writes only what the same
// lane has already read.
template <bool VEC>
__device__ __forceinline__ void rope_finish(uint16_t* row, const float2* cs, uint16_t* __restrict__ y, int D, int R,
                                            bool live, int lane) {
    const int half = R >> 1;
    if (live)
        for (int f = lane; f < half; f += 64) {
            const float2 c = cs[f];
            const float x1 = bf16_bits_to_f32(row[f]), x2 = bf16_bits_to_f32(row[f + half]);
            row[f] = rope_one(x1, -x2, c.x, c.y);
            row[f + half] = rope_one(x2, x1, c.x, c.y);
        }
    __syncthreads();
    if (!live) return;
    if constexpr (VEC) {
        for (int c = lane; c < D / 8; c += 64)
            *reinterpret_cast<u32x4*>(y + 8 * c) = *reinterpret_cast<const u32x4*>(row + 8 * c);
    } else {
        for (int c = lane; c < (D + 7) / 8; c += 64)
            for (int d = 8 * c; d < 8 * c + 8 && d < D; ++d) y[d] = row[d];
    }
}

// x, y [T, H, D].  VEC: D % 8 == 0 and x, y 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(64 * kRopeWaves) void rope_kernel(const uint16_t* __restrict__ x,
                                                               const int64_t* __restrict__ pos,
                                                               uint16_t* __restrict__ y, int T, int H, int D, int R,
                                                               double log2t, int hs, int ws, int iters) {
    extern __shared__ __align__(16) unsigned char lds[];
    float2* cs = reinterpret_cast<float2*>(lds);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint16_t* row = reinterpret_cast<uint16_t*>(lds + rope_rows_offset(R)) + wave * ((D + 7) / 8 * 8);
    const int t = blockIdx.x;
    for (int it = 0; it < iters; ++it) {
        const int h = (blockIdx.y * iters + it) * kRopeWaves + wave;
        const bool live = h < H;
        const int64_t base = ((int64_t)t * H + (live ? h : 0)) * D;
        if constexpr (VEC) {
            // the first chunk of 8 values per lane (all of a row up to D = 512)
            // is loaded before the table; further chunks after it
            u32x4 v0 = {0, 0, 0, 0};
            if (live && lane < D / 8) v0 = load_u32x4(x + base + 8 * lane);
            if (it == 0) rope_table(cs, pos, T, t, R, log2t, hs, ws);
            if (live) {
                if (lane < D / 8) *reinterpret_cast<u32x4*>(row + 8 * lane) = v0;
                for (int c = lane + 64; c < D / 8; c += 64)
                    *reinterpret_cast<u32x4*>(row + 8 * c) = load_u32x4(x + base + 8 * c);
            }
        } else {
            if (it == 0) rope_table(cs, pos, T, t, R, log2t, hs, ws);
            if (live)
                for (int c = lane; c < (D + 7) / 8; c += 64)
                    for (int d = 8 * c; d < 8 * c + 8 && d < D; ++d) row[d] = x[base + d];
        }
        __syncthreads();
        rope_finish<VEC>(row, cs, y + base, D, R, live, lane);
    }
}

// The QKV-gate output p [T, ld] holds per token H query heads of 2D (query,
// then gate) followed by HK key heads and HK value heads of D
// (src/engine.cpp:279-282).  Grid (T, ceil((H + HK) / 4)); head hh < H reads
// query head hh, else key head hh - H.  Its D values are RMS-normalised with weight w (q_norm or
// k_norm) exactly as rms_kernel does for D <= 512 -- lane l owns elements
// [8l, 8l + 8) and adds their squares in order, one wave sum, the same
// normalisation arithmetic -- so the result equals fp8lin_rms of the
// contiguous rows bit for bit; the BF16 result is then rotated as
// rope_kernel does.  q [T, H, D], k [T, HK, D].  VEC: D % 8 == 0, ld % 8 == 0
// and p, q, k, the weights 16-byte aligned.
template <bool VEC>
__global__ __launch_bounds__(64 * kRopeWaves) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ p, int64_t ld, const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw,
    const int64_t* __restrict__ pos, uint16_t* __restrict__ q, uint16_t* __restrict__ k, int T, int H, int HK,
    int D, int R, double log2t, int hs, int ws, float eps, int centered, int iters) {
    extern __shared__ __align__(16) unsigned char lds[];
    float2* cs = reinterpret_cast<float2*>(lds);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint16_t* row = reinterpret_cast<uint16_t*>(lds + rope_rows_offset(R)) + wave * ((D + 7) / 8 * 8);
    const int t = blockIdx.x;
    const float c = centered ? 1.0f : 0.0f;
    const int i0 = 8 * lane;
    auto head_src = [&](int hh) -> const uint16_t* {
        return p + t * ld + (hh < H ? (int64_t)hh * 2 * D : (int64_t)H * 2 * D + (int64_t)(hh - H) * D);
    };
    // VEC: the norm weights and up to kPrefetch iterations' head chunks are
    // loaded before the table and the first barrier, so a workgroup's HBM
    // reads are in flight together rather than one head per round trip.
    constexpr int kPrefetch = 4;
    u32x4 wqv = {0, 0, 0, 0}, wkv = {0, 0, 0, 0};
    if constexpr (VEC) {
        if (i0 < D) {
            wqv = load_u32x4(qw + i0);
            wkv = load_u32x4(kw + i0);
        }
    }
    for (int it0 = 0; it0 < iters; it0 += kPrefetch) {
        u32x4 pre[kPrefetch];
#pragma unroll
        for (int j = 0; j < kPrefetch; ++j) {
            const int hh = (blockIdx.y * iters + it0 + j) * kRopeWaves + wave;
            pre[j] = u32x4{0, 0, 0, 0};
            if constexpr (VEC)
                if (it0 + j < iters && hh < H + HK && i0 < D) pre[j] = load_u32x4(head_src(hh) + i0);
        }
        // every thread fills its share of the table, live or not
        if (it0 == 0) rope_table(cs, pos, T, t, R, log2t, hs, ws);
#pragma unroll
        for (int j = 0; j < kPrefetch; ++j) {
            if (it0 + j >= iters) break;  // uniform over the workgroup
            const int hh = (blockIdx.y * iters + it0 + j) * kRopeWaves + wave;
            const bool live = hh < H + HK;
            const bool is_q = hh < H;
            const uint16_t* src = head_src(hh);
            const uint16_t* w = is_q ? qw : kw;
            uint16_t* dst = is_q ? q + ((int64_t)t * H + hh) * D : k + ((int64_t)t * HK + (hh - H)) * D;
            uint32_t xb[8], wb[8];
            if constexpr (VEC) {
                const u32x4 wv = is_q ? wqv : wkv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xb[2 * e] = pre[j][e] & 0xffffu;
                    xb[2 * e + 1] = pre[j][e] >> 16;
                    wb[2 * e] = wv[e] & 0xffffu;
                    wb[2 * e + 1] = wv[e] >> 16;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    xb[e] = live && i0 + e < D ? src[i0 + e] : 0u;
                    wb[e] = live && i0 + e < D ? w[i0 + e] : 0u;
                }
            }
            if (live) {
                float ss = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float v = bf16_bits_to_f32(xb[e]);
                    ss = __builtin_fmaf(v, v, ss);
                }
                const float inv = rsqrtf(wave_sum(ss) / (float)D + eps);
                uint32_t o[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float n = bf16_bits_to_f32(xb[e]) * inv;
                    if (!centered) n = bf16_bits_to_f32(f32_to_bf16_bits(n));
                    o[e] = f32_to_bf16_bits(n * (bf16_bits_to_f32(wb[e]) + c));
                }
                if constexpr (VEC) {
                    if (i0 < D)
                        *reinterpret_cast<u32x4*>(row + i0) =
                            u32x4{o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16)};
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (i0 + e < D) row[i0 + e] = (uint16_t)o[e];
                }
            }
            __syncthreads();
            rope_finish<VEC>(row, cs, dst, D, R, live, lane);
        }
    }
}

// Token-major form of qk_norm_rope_kernel for long inputs: one wave per
// token takes all of its query and key heads, so the token's cos/sin pairs
// are computed once per wave and no workgroup barrier is needed.
//  - Normalisation: a head of D = 8 * LPH values spans LPH lanes (8 values
//    each), so one 16-byte load per lane covers 64 / LPH heads; up to 8 such
//    loads (a chunk) are issued before any arithmetic.  The arithmetic is that
//    of qk_norm_rope_kernel, value for value: lane li of a head adds the
//    squares of its 8 values in order, the LPH-lane butterfly (xor LPH/2 .. 1)
//    is that kernel's wave butterfly without the steps that add zeros, then
//    the same normalisation and weight.  Lanes past the rotary part (li >= R/8)
//    store their BF16 results; the others leave them in the wave's LDS.
//  - Rotation: 8 pairs (f, f + R/2) per lane, for all heads of the chunk, from
//    LDS; rope_finish's arithmetic, with bf16(-x2 * s) = -bf16(x2 * s) (round
//    to nearest even is symmetric), so bf16(bf16(x1 c) + bf16(-x2 s)) is
//    computed as bf16(bf16(x1 c) - bf16(x2 s)).
// Requires the VEC conditions of qk_norm_rope_kernel, D in {64, ..., 512}
// and R / 16 a power of two (a lane's pairs then have the same f for every
// head: f = 8 (lane mod R/16) + [0, 8)).
template <int LPH>
__global__ __launch_bounds__(256) void qk_norm_rope_token_kernel(
    const uint16_t* __restrict__ p, int64_t ld, const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw,
    const int64_t* __restrict__ pos, uint16_t* __restrict__ q, uint16_t* __restrict__ k, int T, int H, int HK,
    int R, double log2t, int hs, int ws, float eps, int centered) {
    constexpr int D = 8 * LPH, HPI = 64 / LPH, G = 8, CH = G * HPI;  // heads per chunk
    // per wave: the token's cos/sin pairs, then the chunk's rotary values
    // (CH heads x R BF16, at most 8 KiB since R <= D)
    __shared__ float2 tab[4][D / 2];
    __shared__ __align__(16) uint16_t rot_lds[4][CH * D];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= T) return;  // the whole wave: no workgroup barrier follows
    const int li = lane % LPH, sub = lane / LPH;
    const int heads = H + HK, groups = (heads + HPI - 1) / HPI;
    const uint16_t* src = p + (int64_t)t * ld + 8 * li;
    auto head_dst = [&](int hh) __attribute__((always_inline)) -> uint16_t* {
        return hh < H ? q + ((int64_t)t * H + hh) * D : k + ((int64_t)t * HK + (hh - H)) * D;
    };
    auto load_group = [&](int g) __attribute__((always_inline)) -> u32x4 {
        const int hh = g * HPI + sub;
        if (g >= groups || hh >= heads) return u32x4{0, 0, 0, 0};
        return load_u32x4(src + (hh < H ? (int64_t)hh * 2 * D : (int64_t)H * 2 * D + (int64_t)(hh - H) * D));
    };
    u32x4 pre[G];
#pragma unroll
    for (int j = 0; j < G; ++j) pre[j] = load_group(j);
    const u32x4 wqv = load_u32x4(qw + 8 * li), wkv = load_u32x4(kw + 8 * li);
    // the token's table, under the loads' latency (the wave's own LDS writes,
    // read back by the same wave: a wave-level fence orders them)
    for (int f = lane; f < R / 2; f += 64) tab[wave][f] = rope_cos_sin(pos, T, t, f, R, log2t, hs, ws);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int r16 = R / 16;  // lanes (8 pairs each) per head in the rotation
    float co[8], si[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float2 cs = tab[wave][8 * (lane & (r16 - 1)) + e];
        co[e] = cs.x;
        si[e] = cs.y;
    }
    const float c = centered ? 1.0f : 0.0f;
    float wq[8], wk[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        wq[2 * e] = bf16_bits_to_f32(wqv[e] & 0xffffu) + c;
        wq[2 * e + 1] = bf16_bits_to_f32(wqv[e] >> 16) + c;
        wk[2 * e] = bf16_bits_to_f32(wkv[e] & 0xffffu) + c;
        wk[2 * e + 1] = bf16_bits_to_f32(wkv[e] >> 16) + c;
    }
    const bool rot = li < 2 * r16;
    uint16_t* rl = rot_lds[wave];
    for (int g0 = 0; g0 < groups; g0 += G) {
        // ---- normalisation of the chunk's heads
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int g = g0 + j;
            if (g >= groups) break;  // uniform over the wave
            const int hh = g * HPI + sub;
            float v[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[2 * e] = bf16_bits_to_f32(pre[j][e] & 0xffffu);
                v[2 * e + 1] = bf16_bits_to_f32(pre[j][e] >> 16);
            }
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[e], v[e], ss);
#pragma unroll
            for (int d = LPH / 2; d >= 1; d >>= 1) ss += __shfl_xor(ss, d, kWave);
            const float inv = rsqrtf(ss / (float)D + eps);
            const bool is_q = hh < H;
            uint32_t pk[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                f32x2 n{v[2 * e] * inv, v[2 * e + 1] * inv};
                if (!centered) {
                    const uint32_t r = pack_bf16x2(n);
                    n = f32x2{bf16_bits_to_f32(r & 0xffffu), bf16_bits_to_f32(r >> 16)};
                }
                pk[e] = pack_bf16x2(f32x2{n[0] * (is_q ? wq[2 * e] : wk[2 * e]),
                                          n[1] * (is_q ? wq[2 * e + 1] : wk[2 * e + 1])});
            }
            const u32x4 out{pk[0], pk[1], pk[2], pk[3]};
            if (hh < heads) {
                if (rot)
                    *reinterpret_cast<u32x4*>(rl + (j * HPI + sub) * R + 8 * li) = out;
                else
                    *reinterpret_cast<u32x4*>(head_dst(hh) + 8 * li) = out;
            }
        }
        // the next chunk's loads before this chunk's rotation
        const int nheads = min(heads - g0 * HPI, CH);
        if (g0 + G < groups) {
#pragma unroll
            for (int j = 0; j < G; ++j) pre[j] = load_group(g0 + G + j);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // ---- rotation: unit u = (head u / r16, pairs 8 (u mod r16) + [0, 8))
        for (int u = lane; u < nheads * r16; u += 64) {
            const int hl = u / r16, fb = 8 * (u & (r16 - 1));
            uint16_t* base = rl + hl * R + fb;
            const u32x4 a = *reinterpret_cast<const u32x4*>(base);
            const u32x4 b = *reinterpret_cast<const u32x4*>(base + R / 2);
            uint32_t o1[4], o2[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float n1[2], n2[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float x1 = bf16_bits_to_f32(h ? a[e] >> 16 : a[e] & 0xffffu);
                    const float x2 = bf16_bits_to_f32(h ? b[e] >> 16 : b[e] & 0xffffu);
                    const float cc = co[2 * e + h], sn = si[2 * e + h];
                    const uint32_t p1 = pack_bf16x2(f32x2{x1 * cc, x2 * sn});  // bf16(x1 c), bf16(x2 s)
                    const uint32_t p2 = pack_bf16x2(f32x2{x2 * cc, x1 * sn});  // bf16(x2 c), bf16(x1 s)
                    n1[h] = bf16_bits_to_f32(p1 & 0xffffu) - bf16_bits_to_f32(p1 >> 16);
                    n2[h] = bf16_bits_to_f32(p2 & 0xffffu) + bf16_bits_to_f32(p2 >> 16);
                }
                o1[e] = pack_bf16x2(f32x2{n1[0], n1[1]});
                o2[e] = pack_bf16x2(f32x2{n2[0], n2[1]});
            }
            uint16_t* dst = head_dst(g0 * HPI + hl) + fb;
            *reinterpret_cast<u32x4*>(dst) = u32x4{o1[0], o1[1], o1[2], o1[3]};
            *reinterpret_cast<u32x4*>(dst + R / 2) = u32x4{o2[0], o2[1], o2[2], o2[3]};
        }
        // this chunk's LDS reads before the next chunk's writes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

}  // namespace

hipError_t launch_rms(const uint16_t* x, const uint16_t* update, const uint16_t* w, uint16_t* residual,
                      uint16_t* y, int64_t M, int D, float eps, bool centered, hipStream_t stream) {
    const bool vec = D % 8 == 0 && aligned16(x) && aligned16(w) && aligned16(y) &&
                     (!update || (aligned16(update) && aligned16(residual)));
    const dim3 grid((unsigned)M), block(norm_threads(D));
    const int c = centered ? 1 : 0;
    if (update) {
        if (vec)
            hipLaunchKernelGGL((rms_kernel<true, true>), grid, block, 0, stream, x, update, w, residual, y, D, eps, c);
        else
            hipLaunchKernelGGL((rms_kernel<true, false>), grid, block, 0, stream, x, update, w, residual, y, D, eps, c);
    } else {
        if (vec)
            hipLaunchKernelGGL((rms_kernel<false, true>), grid, block, 0, stream, x, update, w, residual, y, D, eps, c);
        else
            hipLaunchKernelGGL((rms_kernel<false, false>), grid, block, 0, stream, x, update, w, residual, y, D, eps,
                               c);
    }
    return hipGetLastError();
}

hipError_t launch_reduce_rms(const uint16_t* x, const uint16_t* partials, int ranks, const uint16_t* w,
                             uint16_t* residual, uint16_t* y, int64_t M, int D, float eps, bool centered,
                             hipStream_t stream) {
    const bool vec = D % 8 == 0 && aligned16(x) && aligned16(w) && aligned16(y) && aligned16(partials) &&
                     aligned16(residual);
    const dim3 grid((unsigned)M), block(norm_threads(D));
    const int c = centered ? 1 : 0;
    const int64_t stride = M * D;
    if (vec)
        hipLaunchKernelGGL((rms_kernel<true, true, true>), grid, block, 0, stream, x, partials, w, residual, y, D, eps,
                           c, ranks, stride);
    else
        hipLaunchKernelGGL((rms_kernel<true, false, true>), grid, block, 0, stream, x, partials, w, residual, y, D,
                           eps, c, ranks, stride);
    return hipGetLastError();
}

int64_t vocab_chunks(int64_t N) { return (N + kVocabChunk - 1) / kVocabChunk; }


hipError_t launch_vocab_candidates(const uint16_t* logits, int M, int N, int64_t offset, uint32_t* part,
                                   double* out, hipStream_t stream) {
    const int chunks = (int)vocab_chunks(N);
    const dim3 grid(chunks, M), block(kVocabThreads);
    if (N % 8 == 0 && aligned16(logits))
        hipLaunchKernelGGL(vocab_partial_kernel<true>, grid, block, 0, stream, logits, N, chunks, part);
    else
        hipLaunchKernelGGL(vocab_partial_kernel<false>, grid, block, 0, stream, logits, N, chunks, part);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_candidates_finish(part, M, chunks, offset, out, stream);
}

hipError_t launch_candidates_finish_sliced(const uint32_t* part, int M, int64_t chunks, uint32_t* slices,
                                           uint32_t* counters, int64_t offset, double* out, hipStream_t stream) {
    const int64_t slots = (chunks + 7) / 8 * 8;
    const int per = (int)((slots + kCandSlices - 1) / kCandSlices);
    hipLaunchKernelGGL(cand_finish_sliced_kernel, dim3(kCandSlices, M), dim3(kSliceThreads), 0, stream, part,
                       (int)chunks, per, slices, counters, offset, out);
    return hipGetLastError();
}

hipError_t launch_candidates_finish(const uint32_t* part, int M, int64_t chunks, int64_t offset, double* out,
                                    hipStream_t stream) {
    hipLaunchKernelGGL((vocab_finish_kernel<64, 4>), dim3(M), dim3(64), 0, stream, part, (int)chunks, offset, out);
    return hipGetLastError();
}

hipError_t launch_merge_candidates(const double* gathered, int ranks, int64_t rows, int64_t* out,
                                   hipStream_t stream) {
    hipLaunchKernelGGL(merge_candidates_kernel, dim3((unsigned)((rows + 127) / 128)), dim3(128), 0, stream,
                       gathered, ranks, rows, out);
    return hipGetLastError();
}

// Head groups of 4 per workgroup: all of a token's heads from T = 1024 on
// (enough workgroups to fill the chip, one table per token), else one.
// From this many tokens on, the Q/K epilogue runs token-major (one wave per
// token) where its shape allows (measured at H = 12, HK = 2, D = 256: equal
// at T = 512, 1.3x faster at 1024, 1.8x at 4096; slower below 512, where
// T / 4 workgroups leave CUs idle).
constexpr int kRopeTokenMajor = 512;

int rope_iters(int T, int heads) { return T >= 1024 ? (heads + kRopeWaves - 1) / kRopeWaves : 1; }
dim3 rope_grid(int T, int heads, int iters) {
    const int per = kRopeWaves * iters;
    return dim3((unsigned)T, (unsigned)((heads + per - 1) / per));
}

hipError_t launch_rope(const uint16_t* x, const int64_t* pos, uint16_t* y, int T, int H, int D, int R, float theta,
                       int hs, int ws, hipStream_t stream) {
    const bool vec = D % 8 == 0 && aligned16(x) && aligned16(y);
    const size_t lds = rope_lds(D, R);
    const int iters = rope_iters(T, H);
    const double log2t = std::log2((double)theta);
    if (vec)
        hipLaunchKernelGGL(rope_kernel<true>, rope_grid(T, H, iters), dim3(64 * kRopeWaves), lds, stream, x, pos, y,
                           T, H, D, R, log2t, hs, ws, iters);
    else
        hipLaunchKernelGGL(rope_kernel<false>, rope_grid(T, H, iters), dim3(64 * kRopeWaves), lds, stream, x, pos, y,
                           T, H, D, R, log2t, hs, ws, iters);
    return hipGetLastError();
}

hipError_t launch_qk_norm_rope(const uint16_t* p, int64_t ld, const uint16_t* qw, const uint16_t* kw,
                               const int64_t* pos, uint16_t* q, uint16_t* k, int T, int H, int HK, int D, int R,
                               float theta, int hs, int ws, float eps, bool centered, hipStream_t stream) {
    const bool vec = D % 8 == 0 && ld % 8 == 0 && aligned16(p) && aligned16(qw) && aligned16(kw) && aligned16(q) &&
                     aligned16(k);
    const size_t lds = rope_lds(D, R);
    const int c = centered ? 1 : 0;
    const int iters = rope_iters(T, H + HK);
    const double log2t = std::log2((double)theta);
    if (vec && T >= kRopeTokenMajor && R % 16 == 0 && ((R / 16) & (R / 16 - 1)) == 0 &&
        (D == 64 || D == 128 || D == 256 || D == 512)) {
        const dim3 grid((unsigned)((T + 3) / 4)), block(256);
        switch (D) {
            case 64:
                hipLaunchKernelGGL(qk_norm_rope_token_kernel<8>, grid, block, 0, stream, p, ld, qw, kw, pos, q, k, T,
                                   H, HK, R, log2t, hs, ws, eps, c);
                break;
            case 128:
                hipLaunchKernelGGL(qk_norm_rope_token_kernel<16>, grid, block, 0, stream, p, ld, qw, kw, pos, q, k,
                                   T, H, HK, R, log2t, hs, ws, eps, c);
                break;
            case 256:
                hipLaunchKernelGGL(qk_norm_rope_token_kernel<32>, grid, block, 0, stream, p, ld, qw, kw, pos, q, k,
                                   T, H, HK, R, log2t, hs, ws, eps, c);
                break;
            default:
                hipLaunchKernelGGL(qk_norm_rope_token_kernel<64>, grid, block, 0, stream, p, ld, qw, kw, pos, q, k,
                                   T, H, HK, R, log2t, hs, ws, eps, c);
        }
        return hipGetLastError();
    }
    if (vec)
        hipLaunchKernelGGL(qk_norm_rope_kernel<true>, rope_grid(T, H + HK, iters), dim3(64 * kRopeWaves), lds,
                           stream, p, ld, qw, kw, pos, q, k, T, H, HK, D, R, log2t, hs, ws, eps, c, iters);
    else
        hipLaunchKernelGGL(qk_norm_rope_kernel<false>, rope_grid(T, H + HK, iters), dim3(64 * kRopeWaves), lds,
                           stream, p, ld, qw, kw, pos, q, k, T, H, HK, D, R, log2t, hs, ws, eps, c, iters);
    return hipGetLastError();
}

}  // namespace fp8lin
