// Small-M (2..64 activation rows) block-FP8 linear on the matrix cores.
//
// Contract of fp8_tensor_small (src/fp8_tensor.cu:18-71): K % 128 == 0, block
// scales [N, K/128], each weight is decoded to BF16 with the reference
// rounding point bf16(decode(c) * s) before the BF16 matrix multiply, FP32
// accumulation.  The reference's split (1 or 4) only partitions its work
// (src/fp8_tensor.cu:41-51); here the K partition is the kernel's own and the
// same for both values, so both give the same bits.
//
// MI355X design: the path is an HBM stream of FP8 codes (M <= 16 rows reuse
// each code at most 16 times), so the kernel is built around keeping enough
// bytes in flight with coalesced loads, and holds no load data in registers
// across steps:
//   - a workgroup owns 16 weight rows; its 4 waves split K: wave w takes block
//     w (128 K) of every 4-block chunk and accumulates one 16x16 block of
//     v_mfma_f32_16x16x32_bf16 (weight rows = B operand, activation rows = A
//     operand; lanes for activation rows >= M read a zero row).  The four
//     partial sums are added in LDS in wave order;
//   - codes go HBM -> LDS by direct-to-LDS DMA (buffer_load_dwordx4 ... lds),
//     8 rows x 128 B per instruction, into a per-wave ring of D blocks of
//     16 rows x 128 K (2 KiB each).  Row r of a slot holds its 16-byte chunks
//     XOR-swizzled by (r >> 1) & 7, which keeps the MFMA-layout reads free of
//     bank conflicts;
//   - activations x[m][512-K chunk] and the block scales of a chunk are DMA'd
//     the same way XA chunks ahead into buffers the waves share (one barrier
//     per chunk);
//   - per block a lane reads 2 x 16 codes, one scale and 4 activation
//     fragments from LDS, converts the codes (v_cvt_pk_f32_fp8, v_mul_f32,
//     v_cvt_pk_bf16_f32) and issues 4 MFMAs.
// Every DMA of a step is issued unconditionally (blocks past K, rows past N or
// M get out-of-range offsets and land zeros), so the issue order is the same
// for every shape and the s_waitcnt counts below are fixed numbers.  The same
// template also builds 64-row workgroups (NBW == 4: each wave its own 16 rows
// over all blocks), which measured slower at every decode shape.
//
// Wide weights (N >= 32 rows per compute unit, K in a 1024-wide band ending
// at 4096, 5120 or 9216) run small_m_stream_kernel instead: one workgroup per
// compute unit, each owning an equal contiguous range of rows (ceil(N / CUs)),
// so the work is balanced to a few rows instead of the 16-row workgroup
// granularity that leaves a partial last round (1088 workgroups over 512
// slots at the 17408-row gate/up).  See the kernel for its pipeline.
//
// Most decode shapes run small_m_row_wide_kernel, the row-staged form: one
// workgroup per compute unit streams its rows (up to 80 at M <= 8, 64 at
// 9..16 rows, 32 at 17..64; 32 when K > 5120) 512 bytes of each row per
// stage, with the activations staged beside the codes (8, 16 or 32 rows per
// stage; 256 bytes per stage where 512 would not fit the LDS: 80 rows at
// 9..32 rows and K = 4224..5120, and 64 staged rows at 33..64; see that
// kernel).
//
// Every kernel here DMAs the weight codes, which one launch reads once, with
// the non-temporal cache policy (dma16_nt): 10-15% more bytes per second
// from HBM than the default policy in these patterns.
#include <algorithm>
#include <utility>

#include "gemm_fp8.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

using gemm_fp8::barrier;
using gemm_fp8::dma16;
using gemm_fp8::dma16_nt;
using gemm_fp8::i32x4;
using gemm_fp8::make_desc;
using gemm_fp8::wait_vm;

constexpr int kRowX = 1040;  // LDS stride of an activation row (1 KiB + 16 B)
constexpr int kMaxM = 16;    // rows of the 16x16x32 MFMA tile's activation side
constexpr int kStreamMaxM = 32;  // two tiles in the row-range kernel
constexpr int kMaxLds = 160 * 1024;

__device__ __forceinline__ int sw(int r) { return (r >> 1) & 7; }

// 64 lanes x 4 B from global (voff, bounds-checked) into LDS [m0v, m0v + 256).
__device__ __forceinline__ void dma4(uint32_t m0v, uint32_t voff, i32x4 desc) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(m0v), "v"(voff), "s"(desc)
                 : "memory", "m0");
}

// Issue order of a wave, per 4-block chunk: at its first own block, after the
// wait, CS DMAs prefetch chunk c + XA (XQ activation rows, 1 scale block);
// at the end of each own block, 2 DMAs refill its ring slot D own blocks
// ahead.  A wave owns NBW blocks of each chunk.  The vmcnt at the first own
// block of a chunk (W0) and at the others (W1) is the number of DMAs issued
// after the oldest one the block needs: its codes, the chunk's scales and
// (first block) the chunk's activation rows.
constexpr int cmin(int a, int b) { return a < b ? a : b; }
constexpr int wait0(int D, int CS, int NBW, int XA) {
    return cmin(2 * (D - 1) + CS * (D / NBW - 1), 2 * XA * NBW + CS * (XA - 1));
}
constexpr int wait1(int D, int CS, int NBW, int XA) {
    return cmin(2 * (D - 1) + CS * (D / NBW), 2 * XA * NBW + 2 + CS * XA);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4 v{a, b, c, d};
    return __builtin_bit_cast(bf16x8, v);
}

// Workgroup shapes (W waves):
//   NBW == 4: each wave owns 16 rows and all blocks of a chunk;
//   NBW == 4 / W: the waves share 16 rows and split every chunk's 4 blocks
//     (wave w takes blocks w, w + W, ...); their partial sums are added in
//     LDS in wave order.
// MX (8, 16 or 32: one or two 16-row MFMA tiles) bounds the activation rows
// a launch may have.  TL row tiles per workgroup (K-split form): the waves
// w / (W / TL) = t hold tile t's rows and split its blocks as W / TL waves
// would alone, sharing one set of activation buffers.
template <int W, int D, int NBW, int XA, int MX, int TL = 1>
struct SmallCfg {
    static_assert(MX == 8 || MX == 16 || MX == 32, "8, 16 or 32 activation rows");
    static constexpr int T = MX > 16 ? 2 : 1;  // 16-row activation tiles
    static constexpr bool KSPLIT = NBW < 4;
    static constexpr int ROWS = KSPLIT ? 16 : 16 * W;
    static constexpr int TW = W / TL;  // waves per row tile
    static constexpr int XBUFS = XA + 1;
    static constexpr int XQ = MX / W;  // activation rows DMA'd per wave per chunk
    static constexpr int CS = XQ + 1;
    static constexpr int W0 = wait0(D, CS, NBW, XA), W1 = wait1(D, CS, NBW, XA);
    static_assert(TL == 1 || (KSPLIT && W % TL == 0), "row tiles split the waves evenly");
    static_assert(XQ >= 1, "every wave stages activation rows");
    static_assert(TW * NBW == 4 || NBW == 4, "a chunk's blocks are split evenly");
    static_assert(D % NBW == 0 && W0 <= 63 && W1 <= 63, "ring depth");
    static constexpr size_t lds(int M) {
        return (size_t)W * D * 2048 + (size_t)XBUFS * (M + 1) * kRowX + (size_t)W * XBUFS * 256;
    }
};

// Requirements (checked by the host): 2 <= M <= MX, K % 128 == 0,
// 32 * K < 2^31.
// per (KSPLIT form): rows of each workgroup, 1..16 (pairs for SW, 1..8); a
// row's sum does not depend on which workgroup or slot holds it.
// SW: gate/up + SwiGLU (N weight rows, gate [0, N/2), up [N/2, N); y is
// [M, N/2]).  Workgroup b then holds gate rows 8b..8b+7 in its slots 0..7
// and the matching up rows in slots 8..15; a row's sum does not depend on
// its slot, so the outputs are fused_swiglu of the plain kernel's, bit for
// bit.  Also requires N * K / 32 < 2^31 (scale offsets over the whole
// matrix).
template <int W, int D, int NBW, int XA, int MX, bool SW, int TL = 1>
__global__ __launch_bounds__(64 * W) void small_m_kernel(const uint16_t* __restrict__ x,
                                                         const uint8_t* __restrict__ codes,
                                                         const float* __restrict__ scales,
                                                         uint16_t* __restrict__ y, int64_t ldy, int M, int N,
                                                         int K, int per) {
    using C = SmallCfg<W, D, NBW, XA, MX, TL>;
    static_assert(!SW || C::KSPLIT, "the SwiGLU form pairs the 16 rows of one workgroup");
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    const int KB = K >> 7;
    const int nchunks = (KB + 3) >> 2;
    // the wave's row tile and its place among the tile's waves
    const int tile = wave / C::TW, wt = wave % C::TW;
    // this wave's first row and its row count
    const int64_t nw = C::KSPLIT ? ((int64_t)blockIdx.x * TL + tile) * per
                                 : (int64_t)blockIdx.x * C::ROWS + 16 * wave;
    const int rows_here = (int)max((int64_t)0, min((int64_t)(C::KSPLIT ? per : 16), (int64_t)N - nw));
    // SW: output pairs pb..pb+pairs-1 (gate row pb + r in slot r, up row
    // half + pb + r in slot 8 + r)
    const int half = N >> 1;
    const int64_t pb = ((int64_t)blockIdx.x * TL + tile) * per;
    const int pairs = (int)max((int64_t)0, min((int64_t)per, (int64_t)half - pb));
    const int xbuf = (M + 1) * kRowX;
    const uint32_t o_codes = (uint32_t)(wave * D * 2048);
    const uint32_t o_x = (uint32_t)(W * D * 2048);
    const uint32_t o_sc = o_x + C::XBUFS * xbuf + wave * (C::XBUFS * 256);
    // the partial-sum exchange reuses the code rings once every wave is done
    static_assert(W * 1024 * C::T <= W * D * 2048, "reduction buffer fits in the code rings");
    const uint32_t o_red = 0;

    // row M of every activation buffer stays zero: lanes for rows >= M read it
    for (int e = threadIdx.x; e < C::XBUFS * 64; e += 64 * W)
        *reinterpret_cast<u32x4*>(lds + o_x + (e >> 6) * xbuf + M * kRowX + (e & 63) * 16) = u32x4{0, 0, 0, 0};
    __syncthreads();

    // Code DMA instruction q fills slots 8q..8q+7 from descriptor dwq[q]:
    // the workgroup's rows (plain), or its 8 gate rows (q = 0) and 8 up rows
    // (q = 1).
    i32x4 dwq[2];
    if constexpr (SW) {
        dwq[0] = make_desc(codes + (pairs ? pb * K : 0), (uint32_t)(pairs * K));
        dwq[1] = make_desc(codes + (pairs ? (half + pb) * K : 0), (uint32_t)(pairs * K));
    } else {
        dwq[0] = dwq[1] = make_desc(codes + (rows_here ? nw * K : 0), (uint32_t)(rows_here * K));
    }
    const i32x4 ds = SW ? make_desc(scales, (uint32_t)((int64_t)N * KB * 4))
                        : make_desc(scales + (rows_here ? nw * KB : 0), (uint32_t)(rows_here * KB * 4));
    const i32x4 dx = make_desc(x, (uint32_t)(M * K * 2));

    // Own block j of this wave -> global block index.
    auto gblk = [&](int j) __attribute__((always_inline)) -> int {
        const int c = j / NBW, p = j % NBW;
        return 4 * c + (C::KSPLIT ? wt + C::TW * p : p);
    };
    // DMA lane offsets.  Codes, instruction q: lane -> row 8q + lane/8, LDS
    // position lane%8 <- chunk (lane%8) ^ sw(row) of the block's 128 codes.
    uint32_t cvoff[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int r = 8 * q + (lane >> 3);
        const int lr = SW ? (lane >> 3) : r;  // row within the descriptor
        cvoff[q] = (uint32_t)(lr * K + 16 * ((lane & 7) ^ sw(r)));
    }
    // Scales of chunk c: lane -> slot lane/4, block 4c + lane%4 (LDS [slot][4]).
    uint32_t svoff = (uint32_t)((lane >> 2) * KB * 4 + 4 * (lane & 3));
    bool sok = true;
    if constexpr (SW) {
        const int r = lane >> 2, pr_ = r & 7;
        sok = pr_ < pairs;
        const int64_t n = (r < 8 ? 0 : half) + pb + pr_;
        svoff = sok ? (uint32_t)(n * KB * 4 + 4 * (lane & 3)) : 0u;
    }
    auto dma_codes = [&](int j) __attribute__((always_inline)) {
        const int blk = gblk(j);
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds0 + o_codes + (uint32_t)(j % D) * 2048u);
        const bool ok = blk < KB;
#pragma unroll
        for (int q = 0; q < 2; ++q)
            dma16_nt(m0 + q * 1024, ok ? cvoff[q] + (uint32_t)blk * 128u : kBufferOob, dwq[q], 0);
    };
    auto dma_chunk = [&](int c) __attribute__((always_inline)) {
        const uint32_t xb = lds0 + o_x + (uint32_t)((c % C::XBUFS) * xbuf);
#pragma unroll
        for (int q = 0; q < C::XQ; ++q) {
            const int m = wave + W * q;
            const int k = c * 512 + 8 * lane;
            const uint32_t off = m < M && k < K ? (uint32_t)((m * K + k) * 2) : kBufferOob;
            // rows >= M land (zeros) in the zero row, which no DMA else writes
            dma16(__builtin_amdgcn_readfirstlane(xb + (uint32_t)(m < M ? m : M) * kRowX), off, dx, 0);
        }
        const uint32_t sb = lds0 + o_sc + (uint32_t)((c % C::XBUFS) * 256);
        const bool ok = sok && 4 * c + (lane & 3) < KB;
        dma4(__builtin_amdgcn_readfirstlane(sb), ok ? svoff + (uint32_t)(16 * c) : kBufferOob, ds);
    };

    // Read side, lane (row = lane%16, g = lane/16).
    const int row = lane & 15, g = lane >> 4;
    const uint32_t c0off = (uint32_t)(row * 128 + 16 * (g ^ sw(row)));
    const uint32_t c1off = (uint32_t)(row * 128 + 16 * ((4 + g) ^ sw(row)));
    uint32_t xrow[C::T];
#pragma unroll
    for (int tt = 0; tt < C::T; ++tt)
        xrow[tt] = (uint32_t)((16 * tt + row < M ? 16 * tt + row : M) * kRowX + 32 * g);

    // ---- prologue: XA chunks of activations and scales, own blocks 0..D-1
#pragma unroll
    for (int c = 0; c < XA; ++c) dma_chunk(c);
#pragma unroll
    for (int j = 0; j < D; ++j) dma_codes(j);
    wait_vm<0>();
    barrier();

    f32x4 acc[C::T];
#pragma unroll
    for (int tt = 0; tt < C::T; ++tt) acc[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int c = 0; c < nchunks; ++c) {
        const uint32_t xb = o_x + (uint32_t)((c % C::XBUFS) * xbuf);
        const uint32_t sb = o_sc + (uint32_t)((c % C::XBUFS) * 256);
        [&]<int... P>(std::integer_sequence<int, P...>) __attribute__((always_inline)) {
            ([&]() __attribute__((always_inline)) {
                constexpr int p = P;
                const int j = NBW * c + p;
                const int b = C::KSPLIT ? wt + C::TW * p : p;  // block within the chunk
                if constexpr (p == 0) {
                    // this chunk's activations, scales and first block landed in
                    // every wave, and every wave is done with the buffers of
                    // chunk c - 1, which chunk c + XA reuses
                    wait_vm<C::W0>();
                    barrier();
                    dma_chunk(c + XA);
                } else {
                    wait_vm<C::W1>();
                }
                const uint32_t slot = o_codes + (uint32_t)(j % D) * 2048u;
                const u32x4 c0 = *reinterpret_cast<const u32x4*>(lds + slot + c0off);
                const u32x4 c1 = *reinterpret_cast<const u32x4*>(lds + slot + c1off);
                const float s = *reinterpret_cast<const float*>(lds + sb + row * 16 + b * 4);
                u32x4 xf[C::T][4];
#pragma unroll
                for (int tt = 0; tt < C::T; ++tt)
#pragma unroll
                    for (int f = 0; f < 4; ++f)
                        xf[tt][f] = *reinterpret_cast<const u32x4*>(lds + xb + xrow[tt] + b * 256 +
                                                                    (f >> 1) * 128 + (f & 1) * 16);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const u32x4 cw = h ? c1 : c0;
                    uint32_t wv[8];
                    dequant4(cw.x, s, wv[0], wv[1]);
                    dequant4(cw.y, s, wv[2], wv[3]);
                    dequant4(cw.z, s, wv[4], wv[5]);
                    dequant4(cw.w, s, wv[6], wv[7]);
#pragma unroll
                    for (int tt = 0; tt < C::T; ++tt) {
                        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, xf[tt][2 * h]), as_bf16x8(wv[0], wv[1], wv[2], wv[3]),
                            acc[tt], 0, 0, 0);
                        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, xf[tt][2 * h + 1]), as_bf16x8(wv[4], wv[5], wv[6], wv[7]),
                            acc[tt], 0, 0, 0);
                    }
                }
                // the slot's codes are in registers; refill it D own blocks ahead
                gemm_fp8::wait_lgkm<0>();
                dma_codes(j + D);
            }(), ...);
        }(std::make_integer_sequence<int, NBW>{});
    }
    // DMAs past the end still target this workgroup's LDS
    wait_vm<0>();

    // acc[tt][i] = C[m = 16 tt + 4g + i][n = row]
    constexpr int T = C::T;
    float total[T][4];
    if constexpr (C::KSPLIT) {
        float* red = reinterpret_cast<float*>(lds + o_red);
        __syncthreads();  // every wave has read its last ring slot
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave * 256 * T + (16 * tt + 4 * g + i) * 16 + row] = acc[tt][i];
        __syncthreads();
        if (wt != 0) return;
        // the tile's waves in order
        const float* tr = red + tile * C::TW * 256 * T;
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = (16 * tt + 4 * g + i) * 16 + row;
                float t = tr[e];
#pragma unroll
                for (int w = 1; w < C::TW; ++w) t = t + tr[w * 256 * T + e];
                total[tt][i] = t;
            }
    } else {
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) total[tt][i] = acc[tt][i];
    }
    if constexpr (SW) {
        // slot row + 8 holds the up row of slot row's gate row
        float up[T][4];
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) up[tt][i] = __shfl_down(total[tt][i], 8, kWave);
        if (row < 8 && row < pairs) {
#pragma unroll
            for (int tt = 0; tt < T; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = 16 * tt + 4 * g + i;
                    if (m < M)
                        y[(int64_t)m * ldy + pb + row] =
                            swiglu_bf16_bits(f32_to_bf16_bits(total[tt][i]), f32_to_bf16_bits(up[tt][i]));
                }
        }
    } else if (row < rows_here) {
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 16 * tt + 4 * g + i;
                if (m < M) y[(int64_t)m * ldy + nw + row] = f32_to_bf16_bits(total[tt][i]);
            }
    }
}

// per: rows (pairs for SW) of each row tile, TL tiles per workgroup.
template <int W, int D, int NBW, int XA, int MX, bool SW, int TL = 1>
hipError_t launch(const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y, int64_t ldy, int M,
                  int N, int K, int per, hipStream_t stream) {
    using C = SmallCfg<W, D, NBW, XA, MX, TL>;
    auto kern = small_m_kernel<W, D, NBW, XA, MX, SW, TL>;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    if (attr != hipSuccess) return attr;
    static_assert(C::KSPLIT, "rows per workgroup are set at run time only in the K-split form");
    const int tiles = SW ? (N / 2 + per - 1) / per : (N + per - 1) / per;
    const int groups = (tiles + TL - 1) / TL;
    const size_t lds = C::lds(M);
    if (lds > (size_t)kMaxLds) return hipErrorInvalidValue;
    hipLaunchKernelGGL(kern, dim3(groups), dim3(64 * W), lds, stream, x, codes, scales, y, ldy, M, N, K, per);
    return hipGetLastError();
}

// ---- persistent row-range form -------------------------------------------
//
// Workgroup b owns rows [b * per, min(N, (b + 1) * per)) and walks them in
// pieces of pr <= 16 rows, as equal as the range allows (33 rows: 3 x 11).  Its 8 waves split K block-wise: wave w owns the 128-K
// blocks w + 8j, j < NB, of every piece, so its activation fragments (the
// MFMA A operand of those blocks, 16 VGPRs per block) are loaded once and stay
// in registers for the whole kernel.  Per step (piece p, own block j) a wave
// consumes one 16-row x 128-code slot of its LDS ring of D slots (step
// t = p * NB + j lives in slot t % D, D <= NB) and immediately refills it with
// the codes of step t + D; the scales of a whole piece ([j][row] per wave)
// come by DMA two pieces ahead into three piece buffers.  At the end of a
// piece the eight partial 16x16 sums go through LDS and one wave adds them in
// wave order into a BF16 staging row block; the staged outputs are written
// once at the end.
//
// Issue order x fragments, scales of pieces 0 and 1, codes of steps 0..D-1,
// then per step (scales of piece p + 2 at j == 0) and 2 code DMAs: the
// number of loads issued after a step's codes is then the same fixed number
// at every step from the first on, which is what wait_vm counts.  The
// activations are raw buffer loads in inline asm, outside the compiler's wait
// counting; their registers are tied to the first explicit wait.
//
// Summation order: per wave, its blocks in K order through MFMA; then the 8
// wave partials in wave order.  It depends on K only (not on the row range),
// so split 1 and 4 and every workgroup count give the same bits.
constexpr int kStreamWaves = 8;
// Partial-sum exchange of T 16-row activation tiles: two buffers of 8 waves x
// 16 T x 16 floats.
constexpr int stream_red(int T) { return 2 * kStreamWaves * 1024 * T; }

template <int NB>
constexpr int stream_scale_dmas() { return (16 * NB + 63) / 64; }
template <int NB, int D, int T = 1>
constexpr int stream_lds_fixed() {
    return kStreamWaves * D * 2048 + kStreamWaves * 3 * stream_scale_dmas<NB>() * 256 + stream_red(T);
}
constexpr int floordiv(int a, int b) { return a >= 0 ? a / b : -((-a + b - 1) / b); }

// Requirements (checked by the host): 1 <= M <= 16 T (T = 2, two activation
// tiles, only with NB <= 5), K % 128 == 0, 8 * (NB - 1) < K / 128 <= 8 * NB,
// N * K < 2^31, per * M * 2 bytes of LDS beyond stream_lds_fixed.
// SW: gate/up + SwiGLU (N weight rows, gate [0, N/2), up [N/2, N); y is
// [M, N/2]).  The units of the ranges and pieces are then output pairs: a
// piece of pr <= 8 pairs holds its gate rows in slots 0..pr-1 and their up
// rows in slots 8..8+pr-1.  A row's sum does not depend on its slot or
// piece, so the outputs are fused_swiglu of the plain kernel's, bit for bit.
// CAND: the output head's vocabulary candidates instead of y.  Per activation
// row m the workgroup writes the best {BF16 logit as float bits, column} of
// its row range (the logits fp8lin_linear would store; larger value, then
// smaller column, NaN as +inf) to pair m * gridDim + blockIdx of part, the
// layout of the two-stage candidates' chunk pairs.
template <int NB, int D, bool SW, bool CAND, int T>
__global__ __launch_bounds__(64 * kStreamWaves) void small_m_stream_kernel(const uint16_t* __restrict__ x,
                                                                          const uint8_t* __restrict__ codes,
                                                                          const float* __restrict__ scales,
                                                                          uint16_t* __restrict__ y, int64_t ldy,
                                                                          int M, int N, int K, int per, int pr,
                                                                          uint32_t* __restrict__ part) {
    constexpr int W = kStreamWaves;
    static_assert(!(SW && CAND), "candidates of a plain projection only");
    constexpr int SC = stream_scale_dmas<NB>();
    static_assert(D <= NB, "the prologue matches the steady-state issue order only for D <= NB");
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    const int KB = K >> 7;
    const int half = N >> 1;
    const int units = SW ? half : N;  // rows, or output pairs
    const int r0 = (int)blockIdx.x * per;
    const int r1 = min(units, r0 + per);
    const int np = r1 > r0 ? (r1 - r0 + pr - 1) / pr : 0;
    // piece order starts at blockIdx % np, so the short last piece of each
    // range does not come at the same time on every compute unit
    const int rot = np ? (int)blockIdx.x % np : 0;
    const uint32_t o_codes = (uint32_t)(wave * D * 2048);
    const uint32_t o_sc = (uint32_t)(W * D * 2048 + wave * 3 * SC * 256);
    const uint32_t o_red = (uint32_t)(W * D * 2048 + W * 3 * SC * 256);
    const uint32_t o_out = o_red + stream_red(T);

    const i32x4 dw = make_desc(codes, (uint32_t)((int64_t)N * K));
    const i32x4 ds = make_desc(scales, (uint32_t)((int64_t)N * KB * 4));
    const i32x4 dx = make_desc(x, (uint32_t)(M * K * 2));

    auto piece = [&](int p) __attribute__((always_inline)) -> int {  // first unit of piece p
        int q = p + rot;
        if (q >= np) q -= np;
        return r0 + pr * q;
    };
    // Code DMA lanes: instruction q, lane -> row 8q + lane/8, LDS position
    // lane%8 <- 16-byte chunk (lane%8) ^ sw(row) of the block's 128 codes.
    uint32_t cvoff[2];
    int crow[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int r = 8 * q + (lane >> 3);
        crow[q] = r;
        cvoff[q] = (uint32_t)(16 * ((lane & 7) ^ sw(r)));
    }
    const int row = lane & 15, g = lane >> 4;
    // Weight row in slot sr (0..15) of the piece starting at unit base, and
    // whether it exists.
    auto slot_row = [&](int base, int sr, bool& ok) __attribute__((always_inline)) -> int {
        if constexpr (SW) {
            const int u = base + (sr & 7);
            ok = (sr & 7) < pr && u < r1;
            return sr < 8 ? u : half + u;
        } else {
            const int n = base + sr;
            ok = sr < pr && n < r1;
            return n;
        }
    };
    auto issue_codes = [&](int p, int j, int slot) __attribute__((always_inline)) {
        const int blk = wave + W * j;
        const bool ok = p < np && blk < KB;
        const int base = ok ? piece(p) : 0;
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds0 + o_codes + (uint32_t)slot * 2048u);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            bool rok;
            const int n = slot_row(base, crow[q], rok);
            dma16_nt(m0 + q * 1024, ok && rok ? (uint32_t)(n * K + blk * 128) + cvoff[q] : kBufferOob, dw, 0);
        }
    };
    // scales of piece p into buffer p % 3 as [j][row]
    auto issue_scales = [&](int p) __attribute__((always_inline)) {
        const int base = p < np ? piece(p) : 0;
        const uint32_t m0 = lds0 + o_sc + (uint32_t)((p % 3) * SC * 256);
#pragma unroll
        for (int i = 0; i < SC; ++i) {
            const int e = 64 * i + lane;
            const int j = e >> 4, blk = wave + W * j;
            bool rok;
            const int n = slot_row(base, e & 15, rok);
            const bool ok = p < np && j < NB && blk < KB && rok;
            dma4(__builtin_amdgcn_readfirstlane(m0 + i * 256), ok ? (uint32_t)((n * KB + blk) * 4) : kBufferOob,
                 ds);
        }
    };

    // Activation fragments of the own blocks, A operand layout of tile tt:
    // lane (m = 16 tt + row, K sub-range g); K offset within a block 16g +
    // 64(f/2) + 8(f%2), the same permutation as the code words the lane
    // converts.  Rows >= M read zeros.
    u32x4 xr[NB][4 * T];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int blk = wave + W * j;
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            const int mr = 16 * tt + row;
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                const int k = blk * 128 + 16 * g + 64 * (f >> 1) + 8 * (f & 1);
                const uint32_t off = mr < M && blk < KB ? (uint32_t)((mr * K + k) * 2) : kBufferOob;
                asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(xr[j][4 * tt + f]) : "v"(off), "s"(dx));
            }
        }
    }
    issue_scales(0);
    issue_scales(1);
#pragma unroll
    for (int t = 0; t < D; ++t) issue_codes(t / NB, t % NB, t);
    wait_vm<2 * (D - 1)>();  // the activations, the first two scale pieces, step 0's codes
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int tt = 0; tt < T; ++tt)
            asm volatile("" : "+v"(xr[j][4 * tt]), "+v"(xr[j][4 * tt + 1]), "+v"(xr[j][4 * tt + 2]),
                         "+v"(xr[j][4 * tt + 3]));
    float* red = reinterpret_cast<float*>(lds + o_red);
    uint16_t* out = reinterpret_cast<uint16_t*>(lds + o_out);

    int sbase = 0;  // (p * NB) % D
    for (int p = 0; p < np; ++p) {
        f32x4 acc[T];
#pragma unroll
        for (int tt = 0; tt < T; ++tt) acc[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        const uint32_t sbuf = o_sc + (uint32_t)((p % 3) * SC * 256);
        [&]<int... J>(std::integer_sequence<int, J...>) __attribute__((always_inline)) {
            ([&]() __attribute__((always_inline)) {
                constexpr int j = J;
                // loads issued after this step's codes: 2 per step over the
                // D - 1 steps since, plus SC at each piece start among them
                constexpr int starts = floordiv(j - 1, NB) - floordiv(j - D, NB);
                wait_vm<2 * (D - 1) + SC * starts>();
                int slot = sbase + j;
                slot = slot >= D ? slot - D : slot;
                if constexpr (NB > D) slot = slot >= D ? slot - D : slot;
                const uint32_t sa = o_codes + (uint32_t)slot * 2048u;
                const u32x4 c0 = *reinterpret_cast<const u32x4*>(lds + sa + row * 128 + 16 * (g ^ sw(row)));
                const u32x4 c1 = *reinterpret_cast<const u32x4*>(lds + sa + row * 128 + 16 * ((4 + g) ^ sw(row)));
                const float s = *reinterpret_cast<const float*>(lds + sbuf + (j * 16 + row) * 4);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const u32x4 cw = h ? c1 : c0;
                    uint32_t wv[8];
                    dequant4(cw.x, s, wv[0], wv[1]);
                    dequant4(cw.y, s, wv[2], wv[3]);
                    dequant4(cw.z, s, wv[4], wv[5]);
                    dequant4(cw.w, s, wv[6], wv[7]);
#pragma unroll
                    for (int tt = 0; tt < T; ++tt) {
                        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, xr[j][4 * tt + 2 * h]), as_bf16x8(wv[0], wv[1], wv[2], wv[3]),
                            acc[tt], 0, 0, 0);
                        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, xr[j][4 * tt + 2 * h + 1]),
                            as_bf16x8(wv[4], wv[5], wv[6], wv[7]), acc[tt], 0, 0, 0);
                    }
                }
                // the slot's codes and the scale are in registers: refill
                gemm_fp8::wait_lgkm<0>();
                if constexpr (j == 0) issue_scales(p + 2);
                issue_codes(p + (j + D) / NB, (j + D) % NB, slot);
            }(), ...);
        }(std::make_integer_sequence<int, NB>{});
        sbase += NB % D;
        sbase = sbase >= D ? sbase - D : sbase;
        // acc[tt][i] = C[m = 16 tt + 4g + i][n = row]; only rows m < M are kept
        constexpr int RW = 256 * T;  // floats per wave in a buffer
        float* rb = red + (p & 1) * (W * RW);
#pragma unroll
        for (int tt = 0; tt < T; ++tt) {
            if (16 * tt + 4 * g < M) {
#pragma unroll
                for (int i = 0; i < 4; ++i) rb[wave * RW + (16 * tt + 4 * g + i) * 16 + row] = acc[tt][i];
            }
        }
        // Two buffers: wave (p % 8) reads buffer p & 1 before it reaches the
        // barrier that ends piece p + 1, after which buffer p & 1 is rewritten.
        gemm_fp8::wait_lgkm<0>();
        barrier();
        if (wave == (p & (W - 1)) && (!SW || row < 8)) {
            const int n0 = piece(p);
#pragma unroll
            for (int tt = 0; tt < T; ++tt) {
                if (16 * tt + 4 * g >= M) continue;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int m = 16 * tt + 4 * g + i;
                    float t = rb[m * 16 + row];
#pragma unroll
                    for (int w = 1; w < W; ++w) t = t + rb[w * RW + m * 16 + row];
                    uint16_t v = f32_to_bf16_bits(t);
                    if constexpr (SW) {
                        // the up row of this pair sits in slot row + 8
                        float u = rb[m * 16 + row + 8];
#pragma unroll
                        for (int w = 1; w < W; ++w) u = u + rb[w * RW + m * 16 + row + 8];
                        v = swiglu_bf16_bits(v, f32_to_bf16_bits(u));
                    }
                    if (m < M && row < pr && n0 + row < r1) out[m * per + (n0 - r0) + row] = v;
                }
            }
        }
    }
    // DMAs past the last piece still target this workgroup's LDS
    wait_vm<0>();
    gemm_fp8::wait_lgkm<0>();
    __syncthreads();
    const int rows = r1 - r0;
    if constexpr (CAND) {
        for (int m = wave; m < M; m += W) {
            float best = -__builtin_inff();
            uint32_t id = 0xffffffffu;
            for (int r = lane; r < rows; r += 64) pick_bf16(best, id, out[m * per + r], (uint32_t)(r0 + r));
            wave_pick(best, id);
            if (lane == 0) {
                uint32_t* pp = part + ((int64_t)m * gridDim.x + blockIdx.x) * 2;
                pp[0] = __builtin_bit_cast(uint32_t, best);
                pp[1] = id;
            }
        }
    } else {
        for (int e = threadIdx.x; e < M * rows; e += 64 * W) {
            const int m = e / rows, r = e - m * rows;
            y[(int64_t)m * ldy + r0 + r] = out[m * per + r];
        }
    }
}

// per: rows (pairs for SW) of each workgroup's range.  CAND: part as
// small_m_stream_kernel describes (y unused).
template <int NB, int D, bool SW, bool CAND, int T>
hipError_t launch_stream(const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y, int64_t ldy,
                         int M, int N, int K, int per, hipStream_t stream, uint32_t* part) {
    auto kern = small_m_stream_kernel<NB, D, SW, CAND, T>;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    if (attr != hipSuccess) return attr;
    const int units = SW ? N / 2 : N;
    const int groups = (units + per - 1) / per;
    const size_t lds = (size_t)stream_lds_fixed<NB, D, T>() + (size_t)per * M * 2;
    // pieces of at most 16 rows (8 pairs), as equal as the range allows
    const int cap = SW ? 8 : 16;
    const int pieces = (per + cap - 1) / cap;
    const int pr = (per + pieces - 1) / pieces;
    hipLaunchKernelGGL(kern, dim3(groups), dim3(64 * kStreamWaves), lds, stream, x, codes, scales, y, ldy, M, N, K,
                       per, pr, part);
    return hipGetLastError();
}

// Blocks per wave of the stream kernel for this K (0: not served).
int stream_nb(int K) {
    const int KB = K / 128;
    for (int nb : {4, 5, 9})
        if (KB > 8 * (nb - 1) && KB <= 8 * nb) return nb;
    return 0;
}

// ---- row-staged form -----------------------------------------------------------
//
// Workgroup b (8 waves, one workgroup per CU) owns units [b U / G, (b + 1) U
// / G) of the U = N rows (N / 2 output pairs for SW): up to NT 16-row MFMA
// tiles (SW: tile t holds the gate rows of pairs 8t..8t+7 in lanes 0..7 and
// their up rows in lanes 8..15).  The codes stream through an LDS ring of 3
// stages; stage s is the 512 bytes of K [512 s, 512 s + 512) of every row
// (256 bytes in the half-stage form, where 512 would not fit), one
// direct-to-LDS DMA moving two rows' 512 bytes (non-temporal: the codes are
// read once).  The activations of a stage (M <= MX rows x 1 KiB) come by
// DMA with the stage's codes, MX / 8 per wave (MX = 8, 16 or 32); rows past
// M land zeros in the zero row M that the padding lanes read.  The
// block scales of the workgroup's rows come once, into a table after the
// ring (dword DMAs, so that no load straddles the end of the range's
// scales).
//
// LDS rows are 16-byte chunks XOR-swizzled so that the reads of one K offset
// from 16 rows fall on distinct banks (codes: slot s = (tile s / 16, lane row
// s % 16) at 512 s, chunk c at c ^ (s & 15); x: row m chunk c at c ^ 2m);
// each DMA lane fetches the global chunk that belongs at its LDS position.
// K % 128 == 0 keeps every XOR inside a group of chunks that is wholly in or
// out of range.
//
// Wave w owns K [512 s + 64 w, +64) of every stage s and every tile.  Lane
// (n, g) reads the 16 codes of row n at 64 w + 16 g, converts them with the
// row's scale and issues the two MFMAs of the K-step pair (codes 0..7, then
// 8..15, against x at the same K).  The 8 waves' 16x16 sums are then added in
// LDS in wave order.  Summation order: per wave its K-steps in K order
// through MFMA, then the wave partials in wave order; it depends on K only
// (not on the row range, the tile, M or MX), so the SwiGLU form's sums are
// the plain form's bit for bit.
//
// Issue order per wave: the scale table, codes(0), x(0), codes(1), x(1);
// then at stage j (after the wait and the barrier) codes(j + 2), x(j + 2).
// The wait at stage j needs x(j) and everything older; codes(j + 1) and
// x(j + 1) are younger: vmcnt(NT + MX / 8).  Stages past K still issue their
// DMAs, with out-of-range offsets that land zeros in the ring, so the counts
// are the same at every stage (a dummy register load in their place, in an
// early form, overwrote a register the compiler had given to another value).
constexpr int kRowMaxM = 8;                                   // activation rows staged at M <= 8
constexpr int kRowD = 3;                                      // stages in the ring
constexpr int kWideWaves = 8;
constexpr int kWideKS = 512;                                  // K bytes of a row per stage
constexpr int kWideMaxK = 5120;
template <int MX, int KS = kWideKS>
constexpr int wide_xslot() { return (MX + 1) * 2 * KS; }      // x rows 0..M-1 and the zero row
constexpr int kWideTable = 80 * (kWideMaxK / 128) * 4;        // 80 rows x 40 blocks
constexpr int kWideTableHalf = kWideTable / 2;                // SW: the up rows' scales
template <int NT, int KS = kWideKS>
constexpr int wide_stage() { return 16 * NT * KS; }
template <int NT, int KS = kWideKS>
constexpr int wide_code_dmas() { return (16 * NT * KS / 1024 + kWideWaves - 1) / kWideWaves; }  // per wave
template <int NT, int D = kRowD, int KS = kWideKS>
constexpr int wide_ox() { return D * wide_stage<NT, KS>(); }
template <int NT, int MX, int D = kRowD, int KS = kWideKS>
constexpr int wide_otab() { return wide_ox<NT, D, KS>() + D * wide_xslot<MX, KS>(); }
// The table, then (where the last code DMA of a stage would run past the
// stage) 1 KiB that such DMAs fill with zeros.
template <int NT, int MX, int D = kRowD, int KS = kWideKS>
constexpr int wide_odump() { return wide_otab<NT, MX, D, KS>() + kWideTable; }
template <int NT, int MX, int D = kRowD, int KS = kWideKS>
constexpr int wide_lds() {
    return wide_odump<NT, MX, D, KS>() + (wide_code_dmas<NT, KS>() * kWideWaves * 1024 > wide_stage<NT, KS>() ? 1024 : 0);
}
static_assert(wide_lds<5, 8>() <= kMaxLds && wide_lds<4, 16>() <= kMaxLds && wide_lds<2, 32>() <= kMaxLds &&
                  wide_lds<5, 32, kRowD, 256>() <= kMaxLds && wide_lds<2, 64, kRowD, 256>() <= kMaxLds,
              "wide row-staged LDS");

// Requirements (checked by the host): 1 <= M <= MX (8; 16 with NT <= 4; 32
// with NT <= 2; with KS = 256, 16 or 32 with NT <= 5, 64 with NT <= 2), K % 128 == 0,
// K <= KS NS <= 5120 (9216 with NT <= 2), at most 16 NT rows (8 NT pairs) per
// workgroup, N * K < 2^31.  MX = 16 stages 16 activation rows (two DMAs per
// wave and stage at KS = 512: rows w and w + 8); the MFMA tile is the same.
// MX = 32 stages 32 and runs two activation tiles, rows 0..15 and 16..31
// (MX = 64, at KS = 256 only: four): each converted code word feeds the
// MFMAs of every activation tile, each with its own accumulator, so a row's
// sums do not depend on the other tiles.
//
// KS is the stage's K bytes per row.  KS = 512: wave w owns K [512 s + 64 w,
// +64) of stage s, a lane 16 codes, two MFMAs per tile.  KS = 256 (half the
// ring and activation slots, for the tiles that do not fit at 512): wave w
// owns K [256 s + 32 w, +32), a lane (n, g) the 8 codes of row n at
// 32 w + 8 g, one MFMA per tile; a code DMA moves four rows' 256 bytes, an
// activation DMA two rows' 512 bytes (a pair past M lands zeros in the zero
// row and the unused row after it).  The summation order (per wave its
// K-steps in K order, then the wave partials in wave order) depends on K and
// KS only.
template <int NS, bool SW, int NT, int MX, int D, int KS = kWideKS>
__global__ __launch_bounds__(64 * kWideWaves) void small_m_row_wide_kernel(const uint16_t* __restrict__ x,
                                                                           const uint8_t* __restrict__ codes,
                                                                           const float* __restrict__ scales,
                                                                           uint16_t* __restrict__ y, int64_t ldy,
                                                                           int M, int N, int K) {
    constexpr int W = kWideWaves, STAGE = wide_stage<NT, KS>(), OX = wide_ox<NT, D, KS>();
    constexpr int OTAB = wide_otab<NT, MX, D, KS>(), XSLOT = wide_xslot<MX, KS>();
    constexpr int XROW = 2 * KS;                 // activation bytes of a row per stage
    constexpr int XRPD = 1024 / XROW;            // activation rows per DMA
    constexpr int XD = MX / (8 * XRPD);          // activation DMAs per wave
    constexpr int RPD = 1024 / KS;               // code rows per DMA
    constexpr int CD = wide_code_dmas<NT, KS>(); // code DMAs per wave
    constexpr int CPR = KS / 16;                 // 16-byte chunks of a row's stage
    constexpr int KW = KS / 8;                   // K of a wave per stage
    constexpr int MI = MX >= 16 ? MX / 16 : 1;   // activation tiles
    constexpr bool DUMP = CD * W * 1024 > STAGE;  // the last code DMAs run past the stage
    static_assert(KS == 512 || KS == 256, "512- or 256-byte stages");
    static_assert(D >= 3, "at least two stages in flight");
    static_assert(MX == 8 || MX == 16 || MX == 32 || MX == 64, "8, 16, 32 or 64 activation rows");
    static_assert(KS == 512 ? MX <= 32 : MX >= 16, "512-byte stages stage 8..32 rows, 256-byte 16..64");
    static_assert(W * NT * MI * 256 * 4 <= OTAB, "partial sums fit below the scale table");
    static_assert(16 * NT * (NS * KS / 128) * 4 <= kWideTable, "the scale table holds the tiles' rows");
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    const int S = K >> 7;
    const int nst = (K + KS - 1) / KS;
    const int half = N >> 1;
    const int units = SW ? half : N;
    const int u0 = (int)((int64_t)blockIdx.x * units / gridDim.x);
    const int R = (int)((int64_t)(blockIdx.x + 1) * units / gridDim.x) - u0;  // rows, or pairs

    for (int e = threadIdx.x; e < D * (XROW / 16); e += 64 * W)
        *reinterpret_cast<u32x4*>(lds + OX + (e >> (KS == 512 ? 6 : 5)) * XSLOT + M * XROW +
                                  (e & (XROW / 16 - 1)) * 16) = u32x4{0, 0, 0, 0};
    __syncthreads();

    i32x4 dq[2], sq[2];
    if constexpr (SW) {
        dq[0] = make_desc(codes + (R ? (int64_t)u0 * K : 0), (uint32_t)(R * K));
        dq[1] = make_desc(codes + (R ? (int64_t)(half + u0) * K : 0), (uint32_t)(R * K));
        sq[0] = make_desc(scales + (R ? (int64_t)u0 * S : 0), (uint32_t)(R * S * 4));
        sq[1] = make_desc(scales + (R ? (int64_t)(half + u0) * S : 0), (uint32_t)(R * S * 4));
    } else {
        dq[0] = dq[1] = make_desc(codes + (R ? (int64_t)u0 * K : 0), (uint32_t)(R * K));
        sq[0] = sq[1] = make_desc(scales + (R ? (int64_t)u0 * S : 0), (uint32_t)(R * S * 4));
    }
    const i32x4 dx = make_desc(x, (uint32_t)(M * K * 2));

    // Code DMA q of a stage: instruction i = wave + 8 q fills slots RPD i ..
    // RPD i + RPD - 1 (CPR lanes each); lane l fetches chunk (l % CPR) ^
    // (slot & 15) of its slot's row, local row lr of descriptor part (SW:
    // slot lane rows 0..7 gate, 8..15 up).  An instruction past the stage
    // (its slots past 16 NT) fills the dump area with zeros.
    uint32_t cvoff[CD];
    int cch[CD];
#pragma unroll
    for (int q = 0; q < CD; ++q) {
        const int slot = RPD * (wave + W * q) + (lane >> (KS == 512 ? 5 : 4));
        const int t = slot >> 4, n = slot & 15;
        const int lr = SW ? 8 * t + (n & 7) : slot;
        cch[q] = (lane & (CPR - 1)) ^ n;
        cvoff[q] = (!DUMP || slot < 16 * NT) && lr < R ? (uint32_t)(lr * K + 16 * cch[q]) : kBufferOob;
    }
    auto issue_codes = [&](int s) __attribute__((always_inline)) {
        const uint32_t base = lds0 + (uint32_t)((s % D) * STAGE);
#pragma unroll
        for (int q = 0; q < CD; ++q) {
            const int ins = wave + W * q;
            const int part = SW ? ((RPD * ins) & 15) >> 3 : 0;  // an instruction's slots are all gate or all up
            const bool ok = s < nst && KS * s + 16 * cch[q] < K && cvoff[q] != kBufferOob;
            uint32_t dst = base + (uint32_t)(ins * 1024);
            if constexpr (DUMP)
                if ((ins + 1) * 1024 > STAGE) dst = lds0 + (uint32_t)wide_odump<NT, MX, D, KS>();
            dma16_nt(__builtin_amdgcn_readfirstlane(dst), ok ? cvoff[q] + (uint32_t)(KS * s) : kBufferOob,
                     dq[part], 0);
        }
    };
    // Activation DMA h of a stage: rows r0 = XRPD (wave + 8 h) .. r0 + XRPD -
    // 1, 64 / XRPD lanes each; chunk p of row m holds the row's chunk p ^ (2 m
    // mod XROW / 16).  Rows past M land zeros (a DMA wholly past M at the
    // zero row M).
    auto issue_x = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < XD; ++h) {
            const int r0 = XRPD * (wave + 8 * h);
            const int xm = XRPD == 1 ? r0 : r0 + (lane >> 5);
            const int xch = KS == 512 ? lane ^ (2 * xm) : (lane & 31) ^ ((2 * xm) & 31);
            const int k = KS * s + 8 * xch;
            const bool ok = xm < M && k < K;
            const uint32_t dst = lds0 + (uint32_t)(OX + (s % D) * XSLOT + (r0 < M ? r0 : M) * XROW);
            dma16(__builtin_amdgcn_readfirstlane(dst), ok ? (uint32_t)((xm * K + k) * 2) : kBufferOob, dx, 0);
        }
    };

    // Scale table (dword DMAs, 256 bytes each): plain, the rows' R x S floats
    // over the 8 waves; SW, the gate rows' (waves 0..3) and, from
    // kWideTableHalf, the up rows' (waves 4..7).
    {
        const int part = SW ? wave >> 2 : 0;
        const int c = SW ? wave & 3 : wave, cs = SW ? 4 : 8;
        const int nt = (SW ? kWideTableHalf : kWideTable) / 256;
        const uint32_t bytes = (uint32_t)(R * S * 4);
        for (int idx = c; idx < nt; idx += cs) {
            const uint32_t at = (uint32_t)(256 * idx);
            if (at >= bytes) break;
            const uint32_t off = at + 4u * (uint32_t)lane;
            dma4(__builtin_amdgcn_readfirstlane(lds0 + OTAB + (uint32_t)(part * kWideTableHalf) + at),
                 off < bytes ? off : kBufferOob, sq[part]);
        }
    }
    auto sidx = [&](int slot) __attribute__((always_inline)) -> int {
        if constexpr (SW) {
            const int t = slot >> 4, n = slot & 15;
            return (n < 8 ? 0 : kWideTableHalf / 4) + (8 * t + (n & 7)) * S;
        }
        return slot * S;
    };

#pragma unroll
    for (int p = 0; p < D - 1; ++p) {
        issue_codes(p);
        issue_x(p);
    }

    const int row = lane & 15, g = lane >> 4;
    // a lane's activation fragment: chunk 8 w + 2 g (and the next) of a
    // 1 KiB row at KS = 512, chunk 4 w + g of a 512-byte row at KS = 256
    uint32_t xoff[MI];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
        const int xr = 16 * mi + row < M ? 16 * mi + row : M;
        const int ch = KS == 512 ? 8 * wave + 2 * g : 4 * wave + g;
        xoff[mi] = (uint32_t)(OX + xr * XROW + 16 * (ch ^ (KS == 512 ? 2 * (xr & (MX - 1)) : (2 * xr) & 31)));
    }
    const uint32_t coff = KS == 512 ? (uint32_t)(row * KS + 16 * ((4 * wave + g) ^ row))
                                    : (uint32_t)(row * KS + 16 * ((2 * wave + (g >> 1)) ^ row) + 8 * (g & 1));
    f32x4 acc[NT][MI];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) acc[t][mi] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const float* tab = reinterpret_cast<const float*>(lds + OTAB);
#pragma unroll
    for (int j = 0; j < NS; ++j) {
        wait_vm<(D - 2) * (CD + XD)>();
        gemm_fp8::wait_lgkm<0>();  // stage j - 1's LDS reads are in registers
        barrier();
        issue_codes(j + D - 1);
        issue_x(j + D - 1);
        if (j < nst && KS * j + KW * wave < K) {
            const int blk = KS == 512 ? 4 * j + (wave >> 1) : 2 * j + (wave >> 2);
            if constexpr (KS == 512) {
                u32x4 x0[MI], x1[MI];
#pragma unroll
                for (int mi = 0; mi < MI; ++mi) {
                    x0[mi] = *reinterpret_cast<const u32x4*>(lds + xoff[mi] + (j % D) * XSLOT);
                    x1[mi] = *reinterpret_cast<const u32x4*>(lds + xoff[mi] + (j % D) * XSLOT + 16);
                }
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const u32x4 cw = *reinterpret_cast<const u32x4*>(lds + (j % D) * STAGE + t * 16 * KS + coff);
                    const float sc = tab[sidx(16 * t + row) + blk];
                    uint32_t wv[8];
                    dequant4(cw.x, sc, wv[0], wv[1]);
                    dequant4(cw.y, sc, wv[2], wv[3]);
                    dequant4(cw.z, sc, wv[4], wv[5]);
                    dequant4(cw.w, sc, wv[6], wv[7]);
#pragma unroll
                    for (int mi = 0; mi < MI; ++mi) {
                        acc[t][mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, x0[mi]),
                                                                             as_bf16x8(wv[0], wv[1], wv[2], wv[3]),
                                                                             acc[t][mi], 0, 0, 0);
                        acc[t][mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, x1[mi]),
                                                                             as_bf16x8(wv[4], wv[5], wv[6], wv[7]),
                                                                             acc[t][mi], 0, 0, 0);
                    }
                }
            } else {
                u32x4 x0[MI];
#pragma unroll
                for (int mi = 0; mi < MI; ++mi)
                    x0[mi] = *reinterpret_cast<const u32x4*>(lds + xoff[mi] + (j % D) * XSLOT);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const uint2 cw = *reinterpret_cast<const uint2*>(lds + (j % D) * STAGE + t * 16 * KS + coff);
                    const float sc = tab[sidx(16 * t + row) + blk];
                    uint32_t wv[4];
                    dequant4(cw.x, sc, wv[0], wv[1]);
                    dequant4(cw.y, sc, wv[2], wv[3]);
#pragma unroll
                    for (int mi = 0; mi < MI; ++mi)
                        acc[t][mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, x0[mi]),
                                                                             as_bf16x8(wv[0], wv[1], wv[2], wv[3]),
                                                                             acc[t][mi], 0, 0, 0);
                }
            }
        }
    }
    wait_vm<0>();
    __syncthreads();

    // acc[t][mi][i] = C[m = 16 mi + 4 g + i][slot 16 t + row]; partials in
    // wave order (block tm = MI t + mi)
    float* red = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                red[((wave * NT + t) * MI + mi) * 256 + (4 * g + i) * 16 + row] = acc[t][mi][i];
    __syncthreads();
    auto total = [&](int tm, int e) __attribute__((always_inline)) -> float {
        float v = red[tm * 256 + e];
#pragma unroll
        for (int w = 1; w < W; ++w) v = v + red[(w * NT * MI + tm) * 256 + e];
        return v;
    };
    for (int q = threadIdx.x; q < NT * MI * 256; q += 64 * W) {
        const int tm = q >> 8, t = tm / MI, e = q & 255, m = 16 * (tm % MI) + (e >> 4), n = e & 15;
        if (m >= M) continue;
        if constexpr (SW) {
            if (n < 8 && 8 * t + n < R)
                y[(int64_t)m * ldy + u0 + 8 * t + n] =
                    swiglu_bf16_bits(f32_to_bf16_bits(total(tm, e)), f32_to_bf16_bits(total(tm, e + 8)));
        } else {
            if (16 * t + n < R) y[(int64_t)m * ldy + u0 + 16 * t + n] = f32_to_bf16_bits(total(tm, e));
        }
    }
}

template <int NS, bool SW, int NT, int MX, int D = kRowD, int KS = kWideKS>
hipError_t launch_row_wide(const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y,
                           int64_t ldy, int M, int N, int K, int groups, hipStream_t stream) {
    auto kern = small_m_row_wide_kernel<NS, SW, NT, MX, D, KS>;
    constexpr int lds = wide_lds<NT, MX, D, KS>();
    static_assert(lds <= kMaxLds, "row-staged LDS");
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kern, dim3(groups), dim3(64 * kWideWaves), lds, stream, x, codes, scales, y, ldy, M, N, K);
    return hipGetLastError();
}

// Tiles of the wide row-staged form where it runs for this geometry (0: it
// does not); groups in `groups`.  Measured on MI355X against the row-range
// kernel (graph replay over 1 GiB of rotated codes, M = 4 / 8): faster at
// K = 5120 for every row count (17408 rows 19.6 / 19.7 us against 20.2 /
// 20.7, 12288 rows 14.1 / 14.2 against 15.8 / 16.3, 8240 rows 10.9 / 11.2
// against 13.1 / 13.8) and at K = 4096 up to 40 rows per CU (8240 rows 10.5
// / 10.7 against 11.1 / 11.6), slower at K = 4096 from 48 rows per CU
// (17408 rows 19.1 / 19.2 against 17.0 / 17.6, 12288 rows 13.8 / 13.9
// against 13.2 / 13.6), so those stay on the row-range kernel.
// At 9..16 rows (16 staged activation rows, at most 4 tiles in LDS, 2 when
// K > 5120 for the scale table) it replaces the K-split tiles and the
// row-range kernel at every shape measured (graph replay, random weights,
// M = 9 / 16, non-temporal code DMAs in both): 8240 x 5120 11.0 / 11.5 us
// against 13.4 / 15.0 (row-range), 12288 x 5120 13.8 / 14.1 against 15.8 /
// 17.0, 7168 x 5120 9.5 / 10.1 against 10.6 / 11.2 (K-split), 5120 x 5120
// 8.8 / 9.2 against 9.6 / 10.1, 5120 x 8704 12.3 / 13.3 against 13.5 / 14.2,
// 8240 x 4096 10.9 / 11.0 against 11.0 / 12.4.  At 17..32 rows (32 staged
// activation rows, two activation tiles, at most 2 tiles in LDS: 163 328
// bytes at K > 5120) it replaces the K-split tiles with two activation tiles
// at every shape measured (graph replay, random weights, M = 17 / 32):
// 5120 x 8704 17.0 / 17.2 us against 18.1 / 18.9, 7168 x 5120 12.0 / 12.9
// against 13.2 / 14.1, 5120 x 5120 11.0 / 11.9 against 12.0 / 13.1, 2048 x
// 5120 8.1 / 9.4 against 10.9 / 11.9, 3072 x 8704 12.1 / 14.3 against 16.2 /
// 17.2, 6144 x 9216 16.5 / 18.2 against 18.5 / 20.2, 6144 x 4096 10.3 / 10.9
// against 10.8 / 11.7.  With 256-byte stages (half the ring and activation
// slots) it also takes 5 tiles at 9..16 rows and 3..5 at 17..32, at K =
// 4224..5120 (M = 9 / 16 / 17 / 32, against the row-range kernel): gate/up
// 19.5 / 19.4 / 21.5 / 21.9 us against 20.2 / 21.4 / 22.8 / 26.6, 8240 x 5120
// 13.9 / 15.2 us at M = 17 / 32 against 16.6 / 20.1, 12288 x 5120 15.4 /
// 17.2 against 18.6 / 22.6.  At K = 4096 the row-range kernel stays (17408 x
// 4096 16.2 against 21.1 us at M = 9 in that form).  The choice depends on
// the weight geometry and on the row count's range (1..8, 9..16, 17..32)
// only, the same for the plain and the SwiGLU form.
int row_wide_tiles(int M, int N, int K, bool swiglu, int& groups) {
    const int cus = compute_units();
    const int units = swiglu ? N / 2 : N;
    if (M < 1 || M > 64 || K % 128 != 0 || K > 9216 || units < 1 || (int64_t)N * K >= ((int64_t)1 << 31))
        return 0;
    const int rows_per_cu = (N + cus - 1) / cus;
    groups = std::min(cus, units);
    const int per = (units + groups - 1) / groups;
    const int t = swiglu ? (per + 7) / 8 : (per + 15) / 16;
    if (M > 32) return t >= 1 && t <= 2 ? t : 0;  // 64 staged rows in 256-byte stages
    if (M > kRowMaxM) {
        // 512-byte stages hold 4 tiles at 9..16 rows, 2 at 17..32; more (the
        // 256-byte stages) only at K = 4224..5120
        if (K > kWideMaxK) return t >= 1 && t <= 2 ? t : 0;
        if (t <= (M > 16 ? 2 : 4)) return t >= 1 ? t : 0;
        return K > 4096 && t <= 5 ? t : 0;
    }
    if (K > kWideMaxK) return t >= 1 && t <= 2 ? t : 0;
    if (K <= 4096 && stream_nb(K) != 0 && rows_per_cu > 40) return 0;
    return t >= 1 && t <= 5 ? t : 0;
}

}  // namespace

// The row-staged form (row_wide_tiles) runs first.  Its first version
// streamed up to 32 rows per CU in 1 KiB row pieces with 16 waves per
// workgroup (two tiles, 3 stages of 32 KiB); with the non-temporal code DMAs
// the 512-byte form took every such shape from it (graph replay, random
// weights, M = 4 / 8, on one box): 7168 x 5120 8.98 / 9.15 us against 10.21 /
// 10.33, 5120 x 5120 8.02 / 8.19 against 8.75 / 8.89, 6144 x 4096 7.87 /
// 8.11 against 9.45 / 9.62, 5120 x 8704 11.74 / 11.83 against 12.15 /
// 12.25, 2048 x 5120 6.59 / 6.62 against 8.09 / 8.12.  Variants of the
// first version measured slower: 8 waves, activations held in registers
// (loaded up front or per stage: an extra 2 us on the code stream), an
// activation ring one stage ahead, and no activation DMA for the waves of
// padding rows.
//
// Otherwise (K > 9216, or more rows per CU than the row-staged form holds
// where the row-range kernel does not serve) a workgroup holds two row tiles
// (about one workgroup per CU): four waves per tile split every chunk's 4 blocks,
// each with a 3-block ring, and the eight waves share the activation
// buffers, staged 2 chunks ahead.  Each tile sums exactly as a four-wave
// workgroup alone would.  At M = 8 (before the row-staged form): 13.6 / 10.8
// us at down / QKV-gate against 14.4 / 11.5 with one tile per workgroup (two
// workgroups per CU), and deeper prefetch was slower in both forms (one
// tile: 3 chunks ahead at M = 8; two tiles: a 5-block ring 4 chunks ahead
// 14.6 / 11.8 us, 6 blocks 5 ahead slower still at M <= 4).  9..16 rows keep
// one tile per workgroup (16 activation rows staged per chunk).  Measured on
// MI355X at the decode shapes (M = 2..8) the K-split tiles beat 64-row
// workgroups (the NBW == 4 form) for every shape.
//
// The stream kernel serves N >= 32 rows per compute unit (measured on MI355X
// at M = 2, 4, 8: 17408 x 5120 gate/up 16-18% faster, the 75968-row head
// 7-21%, the 8240-row in_proj_all 5-13%).  At 7168 and 5120 rows (28 and 20
// per CU) the 16-row workgroups stay faster, also against equal pieces of 14
// and 10 rows (6-12% slower: fewer code bytes in flight per CU).
constexpr int kStreamRowsPerCu = 32;
// With two activation tiles (17..32 rows) the row-range kernel serves 32 rows
// per CU and more, as with one: the 7168-row QKV-gate (28 per CU) at M = 17 /
// 24 / 32 runs 13.7 / 14.5 / 14.6 us in the K-split tiles (two per
// workgroup), against 15.3 / 17.1 / 18.9 in the row-range kernel (measured
// on MI355X).
constexpr int kStreamRowsPerCuT2 = 32;

namespace {

// Whether launch_small_m runs the row-range kernel for this geometry (its
// blocks per wave in nb, rows per workgroup for the plain form in per_rows).
// 17..32 activation rows take two 16-row tiles, whose activation registers
// (8 NB dwordx4 per lane) fit beside the rest for NB <= 5 (K <= 5120).
bool stream_form(int M, int N, int K, int& nb, int& per_rows) {
    const int cus = compute_units();
    nb = stream_nb(K);
    const int rows_per_cu = M > kMaxM ? kStreamRowsPerCuT2 : kStreamRowsPerCu;
    if (!nb || M < 1 || M > kStreamMaxM || N < rows_per_cu * cus || (int64_t)N * K >= ((int64_t)1 << 31))
        return false;
    if (M > kMaxM && nb > 5) return false;
    per_rows = (N + cus - 1) / cus;
    const int fixed = M > kMaxM ? (nb == 4 ? stream_lds_fixed<4, 4, 2>() : stream_lds_fixed<5, 5, 2>())
                      : nb == 4 ? stream_lds_fixed<4, 4>()
                      : nb == 5 ? stream_lds_fixed<5, 5>()
                                : stream_lds_fixed<9, 7>();
    return (int64_t)fixed + (int64_t)per_rows * M * 2 <= kMaxLds;
}

// The row-range kernel for stream_form's geometry: per rows (pairs for SW)
// per workgroup, one or two activation tiles.
template <bool SW, bool CAND>
hipError_t dispatch_stream(int nb, const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y,
                           int64_t ldy, int M, int N, int K, int per, hipStream_t stream, uint32_t* part) {
    if (M > kMaxM) {
        if (nb == 4) return launch_stream<4, 4, SW, CAND, 2>(x, codes, scales, y, ldy, M, N, K, per, stream, part);
        return launch_stream<5, 5, SW, CAND, 2>(x, codes, scales, y, ldy, M, N, K, per, stream, part);
    }
    if (nb == 4) return launch_stream<4, 4, SW, CAND, 1>(x, codes, scales, y, ldy, M, N, K, per, stream, part);
    if (nb == 5) return launch_stream<5, 5, SW, CAND, 1>(x, codes, scales, y, ldy, M, N, K, per, stream, part);
    return launch_stream<9, 7, SW, CAND, 1>(x, codes, scales, y, ldy, M, N, K, per, stream, part);
}

}  // namespace


// fp8lin_linear at two rows and K <= 5120 takes the matrix-core path where it
// measured faster than the two-row ring GEMV (graph replay, random weights):
// the weights of the row-range kernel (the output heads: 75968 x 5120 61.8
// against 66.6 us, 124160 x 5120 96.0 against 109.2) and those of the
// row-staged form with 25..40 rows per CU (7168 x 5120 9.0 against 9.8,
// 8192 x 5120 9.5 against 10.0, 8240 x 5120 10.4 against 10.6).  Fewer rows
// per CU (5120 x 5120 8.0 against 7.8, 2048 x 5120 6.5 against 5.1) and the
// 68 of gate/up (18.1 against 17.8) keep the GEMV.
bool small_m_wide_rows(int M, int N, int K) {
    int groups = 0;
    return row_wide_tiles(M, N, K, false, groups) != 0;
}

bool small_m_two_rows(int N, int K) {
    if (small_m_candidates_supported(2, N, K)) return true;
    const int cus = compute_units();
    const int rows_per_cu = (N + cus - 1) / cus;
    int groups = 0;
    return rows_per_cu > 24 && rows_per_cu <= 40 && row_wide_tiles(2, N, K, false, groups) != 0;
}

bool small_m_candidates_supported(int M, int N, int K) {
    int nb = 0, per = 0, groups = 0;
    // only where fp8lin_linear runs the row-range kernel (its candidates
    // are that kernel's sums)
    if (row_wide_tiles(M, N, K, false, groups)) return false;
    return stream_form(M, N, K, nb, per);
}

namespace {

// Ring depth: 3 stages (two in flight), 4 for one tile, whose stages are
// 8 KiB (measured on MI355X, graph replay, M = 4 / 8: 3072 x 8704 8.89 /
// 8.84 us against 9.74 / 9.74, 2048 x 5120 6.31 / 6.36 against 6.59 / 6.60;
// with two tiles a fourth stage was 2-5% slower, a fifth 5-8%; with 32
// staged activation rows a one-tile ring stays at 3 stages, 122 KiB).
template <bool SW, int NT, int MX>
hipError_t dispatch_row_wide_half(const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y,
                                  int64_t ldy, int M, int N, int K, int groups, hipStream_t stream) {
    if (K <= 4096) return launch_row_wide<16, SW, NT, MX, kRowD, 256>(x, codes, scales, y, ldy, M, N, K, groups, stream);
    if constexpr (NT <= 2)
        if (K > kWideMaxK)
            return launch_row_wide<36, SW, NT, MX, kRowD, 256>(x, codes, scales, y, ldy, M, N, K, groups, stream);
    return launch_row_wide<20, SW, NT, MX, kRowD, 256>(x, codes, scales, y, ldy, M, N, K, groups, stream);
}

template <bool SW, int NT, int MX>
hipError_t dispatch_row_wide(const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y,
                             int64_t ldy, int M, int N, int K, int groups, hipStream_t stream) {
    constexpr int D = NT == 1 && MX < 32 ? 4 : kRowD;
    if (K <= 4096) return launch_row_wide<8, SW, NT, MX, D>(x, codes, scales, y, ldy, M, N, K, groups, stream);
    if constexpr (NT <= 2)
        if (K > kWideMaxK)
            return launch_row_wide<18, SW, NT, MX, D>(x, codes, scales, y, ldy, M, N, K, groups, stream);
    return launch_row_wide<10, SW, NT, MX, D>(x, codes, scales, y, ldy, M, N, K, groups, stream);
}

template <bool SW>
hipError_t dispatch_row_wide(int nt, const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y,
                             int64_t ldy, int M, int N, int K, int groups, hipStream_t stream) {
    if (M > 32) {
        if (nt == 1) return dispatch_row_wide_half<SW, 1, 64>(x, codes, scales, y, ldy, M, N, K, groups, stream);
        return dispatch_row_wide_half<SW, 2, 64>(x, codes, scales, y, ldy, M, N, K, groups, stream);
    }
    if (M > 16) {
        if (nt == 1) return dispatch_row_wide<SW, 1, 32>(x, codes, scales, y, ldy, M, N, K, groups, stream);
        if (nt == 2) return dispatch_row_wide<SW, 2, 32>(x, codes, scales, y, ldy, M, N, K, groups, stream);
        if (nt == 3) return dispatch_row_wide_half<SW, 3, 32>(x, codes, scales, y, ldy, M, N, K, groups, stream);
        if (nt == 4) return dispatch_row_wide_half<SW, 4, 32>(x, codes, scales, y, ldy, M, N, K, groups, stream);
        return dispatch_row_wide_half<SW, 5, 32>(x, codes, scales, y, ldy, M, N, K, groups, stream);
    }
    if (M > kRowMaxM) {
        if (nt == 5) return dispatch_row_wide_half<SW, 5, 16>(x, codes, scales, y, ldy, M, N, K, groups, stream);
        if (nt == 1) return dispatch_row_wide<SW, 1, 16>(x, codes, scales, y, ldy, M, N, K, groups, stream);
        if (nt == 2) return dispatch_row_wide<SW, 2, 16>(x, codes, scales, y, ldy, M, N, K, groups, stream);
        if (nt == 3) return dispatch_row_wide<SW, 3, 16>(x, codes, scales, y, ldy, M, N, K, groups, stream);
        return dispatch_row_wide<SW, 4, 16>(x, codes, scales, y, ldy, M, N, K, groups, stream);
    }
    if (nt == 1) return dispatch_row_wide<SW, 1, 8>(x, codes, scales, y, ldy, M, N, K, groups, stream);
    if (nt == 2) return dispatch_row_wide<SW, 2, 8>(x, codes, scales, y, ldy, M, N, K, groups, stream);
    if (nt == 3) return dispatch_row_wide<SW, 3, 8>(x, codes, scales, y, ldy, M, N, K, groups, stream);
    if (nt == 4) return dispatch_row_wide<SW, 4, 8>(x, codes, scales, y, ldy, M, N, K, groups, stream);
    return dispatch_row_wide<SW, 5, 8>(x, codes, scales, y, ldy, M, N, K, groups, stream);
}

}  // namespace

hipError_t launch_small_m_candidates(const uint16_t* x, const uint8_t* codes, const float* scales, int M, int N,
                                     int K, uint32_t* part, int64_t& groups, hipStream_t stream) {
    int nb = 0, per = 0;
    if (!stream_form(M, N, K, nb, per)) return hipErrorNotSupported;
    groups = (N + per - 1) / per;
    return dispatch_stream<false, true>(nb, x, codes, scales, nullptr, 0, M, N, K, per, stream, part);
}

// The kernel is chosen from the weight geometry alone, the same for the plain
// and the SwiGLU form, so the SwiGLU outputs are those of the plain form's
// sums.
hipError_t launch_small_m(const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y,
                          int64_t ldy, int M, int N, int K, int /*split*/, bool swiglu, hipStream_t stream) {
    const int cus = compute_units();
    int nb = 0, per_rows = 0, wide_groups = 0;
    if (const int nt = row_wide_tiles(M, N, K, swiglu, wide_groups)) {
        if (swiglu) return dispatch_row_wide<true>(nt, x, codes, scales, y, ldy, M, N, K, wide_groups, stream);
        return dispatch_row_wide<false>(nt, x, codes, scales, y, ldy, M, N, K, wide_groups, stream);
    }
    if (M > 32) return hipErrorNotSupported;  // only the row-staged form stages 33..64 rows
    if (stream_form(M, N, K, nb, per_rows)) {
        if (swiglu)
            return dispatch_stream<true, false>(nb, x, codes, scales, y, ldy, M, N, K, (N / 2 + cus - 1) / cus,
                                                stream, nullptr);
        return dispatch_stream<false, false>(nb, x, codes, scales, y, ldy, M, N, K, per_rows, stream, nullptr);
    }
    // Rows per tile: about two tiles per CU, 8..16 rows (4..8 pairs), so
    // every CU streams about the same number of rows in one round (16-row
    // tiles left the 5120-row down projection at 1.25 per CU, a quarter of
    // the CUs streaming a second one alone).
    const int units = swiglu ? N / 2 : N;
    const int per = std::clamp((units + 2 * cus - 1) / (2 * cus), swiglu ? 4 : 8, swiglu ? 8 : 16);
    if (M > kMaxM) {
        // 17..32 rows off the row-range form: the same tiles with two
        // activation tiles (32 rows staged per chunk, 1 chunk ahead; each
        // code word feeds both).  Down at M = 24 / 32: 19.8 / 20.0 us with
        // two row tiles per workgroup, against 30.8 / 31.0 with one (two
        // workgroups per CU fit up to M = 21), 29.2 / 32.1 for two passes
        // of 16 rows and 36 in the split-K GEMM.
        if (M > kStreamMaxM) return hipErrorNotSupported;
        if (swiglu) return launch<8, 3, 1, 1, 32, true, 2>(x, codes, scales, y, ldy, M, N, K, per, stream);
        return launch<8, 3, 1, 1, 32, false, 2>(x, codes, scales, y, ldy, M, N, K, per, stream);
    }
    // 9..16 rows: activations 2 chunks ahead (down / QKV-gate at M = 16:
    // 15.8 / 12.7 us with two row tiles per workgroup, against 18.6 / 13.9
    // with one tile per workgroup and two workgroups per CU).
    if (swiglu) {
        if (M <= 8) return launch<8, 3, 1, 2, 8, true, 2>(x, codes, scales, y, ldy, M, N, K, per, stream);
        return launch<8, 3, 1, 2, 16, true, 2>(x, codes, scales, y, ldy, M, N, K, per, stream);
    }
    if (M <= 8) return launch<8, 3, 1, 2, 8, false, 2>(x, codes, scales, y, ldy, M, N, K, per, stream);
    return launch<8, 3, 1, 2, 16, false, 2>(x, codes, scales, y, ldy, M, N, K, per, stream);
}

}  // namespace fp8lin
