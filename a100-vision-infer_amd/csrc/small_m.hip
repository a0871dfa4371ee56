// Small-M (2..8 activation rows) block-FP8 linear on the matrix cores.
//
// Contract of fp8_tensor_small (src/fp8_tensor.cu:18-71): K % 128 == 0, block
// scales [N, K/128], each weight is decoded to BF16 with the reference
// rounding point bf16(decode(c) * s) before the BF16 matrix multiply, FP32
// accumulation.  The reference's split (1 or 4) only partitions its work
// (src/fp8_tensor.cu:41-51); here the K partition is the kernel's own and the
// same for both values, so both give the same bits.
//
// MI355X design: the path is an HBM stream of FP8 codes (M <= 8 rows reuse
// each code at most 8 times), so the kernel is built around keeping enough
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
#include <utility>

#include "gemm_fp8.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

using gemm_fp8::barrier;
using gemm_fp8::dma16;
using gemm_fp8::i32x4;
using gemm_fp8::make_desc;
using gemm_fp8::wait_vm;

constexpr int kRowX = 1040;  // LDS stride of an activation row (1 KiB + 16 B)
constexpr int kMaxM = 8;

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
template <int W, int D, int NBW, int XA>
struct SmallCfg {
    static constexpr bool KSPLIT = NBW < 4;
    static constexpr int ROWS = KSPLIT ? 16 : 16 * W;
    static constexpr int XBUFS = XA + 1;
    static constexpr int XQ = kMaxM / W;  // activation rows DMA'd per wave per chunk
    static constexpr int CS = XQ + 1;
    static constexpr int W0 = wait0(D, CS, NBW, XA), W1 = wait1(D, CS, NBW, XA);
    static_assert(W * NBW == 4 || NBW == 4, "a chunk's blocks are split evenly");
    static_assert(D % NBW == 0 && W0 <= 63 && W1 <= 63, "ring depth");
    static constexpr size_t lds(int M) {
        return (size_t)W * D * 2048 + (size_t)XBUFS * (M + 1) * kRowX + (size_t)W * XBUFS * 256;
    }
};

// Requirements (checked by the host): 2 <= M <= 8, K % 128 == 0,
// 32 * K < 2^31.
template <int W, int D, int NBW, int XA>
__global__ __launch_bounds__(64 * W) void small_m_kernel(const uint16_t* __restrict__ x,
                                                         const uint8_t* __restrict__ codes,
                                                         const float* __restrict__ scales,
                                                         uint16_t* __restrict__ y, int64_t ldy, int M, int N,
                                                         int K) {
    using C = SmallCfg<W, D, NBW, XA>;
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds0 = (uint32_t)(uintptr_t)lds;
    const int KB = K >> 7;
    const int nchunks = (KB + 3) >> 2;
    const int64_t nw = (int64_t)blockIdx.x * C::ROWS + (C::KSPLIT ? 0 : 16 * wave);  // this wave's first row
    const int rows_here = (int)max((int64_t)0, min((int64_t)16, (int64_t)N - nw));
    const int xbuf = (M + 1) * kRowX;
    const uint32_t o_codes = (uint32_t)(wave * D * 2048);
    const uint32_t o_x = (uint32_t)(W * D * 2048);
    const uint32_t o_sc = o_x + C::XBUFS * xbuf + wave * (C::XBUFS * 256);
    // the partial-sum exchange reuses the code rings once every wave is done
    static_assert(W * 1024 <= W * D * 2048, "reduction buffer fits in the code rings");
    const uint32_t o_red = 0;

    // row M of every activation buffer stays zero: lanes for rows >= M read it
    for (int e = threadIdx.x; e < C::XBUFS * 64; e += 64 * W)
        *reinterpret_cast<u32x4*>(lds + o_x + (e >> 6) * xbuf + M * kRowX + (e & 63) * 16) = u32x4{0, 0, 0, 0};
    __syncthreads();

    const i32x4 dw = make_desc(codes + (rows_here ? nw * K : 0), (uint32_t)(rows_here * K));
    const i32x4 ds = make_desc(scales + (rows_here ? nw * KB : 0), (uint32_t)(rows_here * KB * 4));
    const i32x4 dx = make_desc(x, (uint32_t)(M * K * 2));

    // Own block j of this wave -> global block index.
    auto gblk = [&](int j) __attribute__((always_inline)) -> int {
        const int c = j / NBW, p = j % NBW;
        return 4 * c + (C::KSPLIT ? wave + W * p : p);
    };
    // DMA lane offsets.  Codes, instruction q: lane -> row 8q + lane/8, LDS
    // position lane%8 <- chunk (lane%8) ^ sw(row) of the block's 128 codes.
    uint32_t cvoff[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int r = 8 * q + (lane >> 3);
        cvoff[q] = (uint32_t)(r * K + 16 * ((lane & 7) ^ sw(r)));
    }
    // Scales of chunk c: lane -> row lane/4, block 4c + lane%4 (LDS [row][4]).
    const uint32_t svoff = (uint32_t)((lane >> 2) * KB * 4 + 4 * (lane & 3));
    auto dma_codes = [&](int j) __attribute__((always_inline)) {
        const int blk = gblk(j);
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds0 + o_codes + (uint32_t)(j % D) * 2048u);
        const bool ok = blk < KB;
#pragma unroll
        for (int q = 0; q < 2; ++q) dma16(m0 + q * 1024, ok ? cvoff[q] + (uint32_t)blk * 128u : kBufferOob, dw, 0);
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
        const bool ok = 4 * c + (lane & 3) < KB;
        dma4(__builtin_amdgcn_readfirstlane(sb), ok ? svoff + (uint32_t)(16 * c) : kBufferOob, ds);
    };

    // Read side, lane (row = lane%16, g = lane/16).
    const int row = lane & 15, g = lane >> 4;
    const uint32_t c0off = (uint32_t)(row * 128 + 16 * (g ^ sw(row)));
    const uint32_t c1off = (uint32_t)(row * 128 + 16 * ((4 + g) ^ sw(row)));
    const uint32_t xrow = (uint32_t)((row < M ? row : M) * kRowX + 32 * g);

    // ---- prologue: XA chunks of activations and scales, own blocks 0..D-1
#pragma unroll
    for (int c = 0; c < XA; ++c) dma_chunk(c);
#pragma unroll
    for (int j = 0; j < D; ++j) dma_codes(j);
    wait_vm<0>();
    barrier();

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c = 0; c < nchunks; ++c) {
        const uint32_t xb = o_x + (uint32_t)((c % C::XBUFS) * xbuf);
        const uint32_t sb = o_sc + (uint32_t)((c % C::XBUFS) * 256);
        [&]<int... P>(std::integer_sequence<int, P...>) __attribute__((always_inline)) {
            ([&]() __attribute__((always_inline)) {
                constexpr int p = P;
                const int j = NBW * c + p;
                const int b = C::KSPLIT ? wave + W * p : p;  // block within the chunk
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
                u32x4 xf[4];
#pragma unroll
                for (int f = 0; f < 4; ++f)
                    xf[f] = *reinterpret_cast<const u32x4*>(lds + xb + xrow + b * 256 + (f >> 1) * 128 +
                                                            (f & 1) * 16);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const u32x4 cw = h ? c1 : c0;
                    uint32_t wv[8];
                    dequant4(cw.x, s, wv[0], wv[1]);
                    dequant4(cw.y, s, wv[2], wv[3]);
                    dequant4(cw.z, s, wv[4], wv[5]);
                    dequant4(cw.w, s, wv[6], wv[7]);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xf[2 * h]),
                                                                   as_bf16x8(wv[0], wv[1], wv[2], wv[3]), acc,
                                                                   0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xf[2 * h + 1]),
                                                                   as_bf16x8(wv[4], wv[5], wv[6], wv[7]), acc,
                                                                   0, 0, 0);
                }
                // the slot's codes are in registers; refill it D own blocks ahead
                gemm_fp8::wait_lgkm<0>();
                dma_codes(j + D);
            }(), ...);
        }(std::make_integer_sequence<int, NBW>{});
    }
    // DMAs past the end still target this workgroup's LDS
    wait_vm<0>();

    // acc[i] = C[m = 4g + i][n = row]
    float total[4];
    if constexpr (C::KSPLIT) {
        float* red = reinterpret_cast<float*>(lds + o_red);
        __syncthreads();  // every wave has read its last ring slot
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave * 256 + (4 * g + i) * 16 + row] = acc[i];
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float t = red[(4 * g + i) * 16 + row];
#pragma unroll
            for (int w = 1; w < W; ++w) t = t + red[w * 256 + (4 * g + i) * 16 + row];
            total[i] = t;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) total[i] = acc[i];
    }
    if (row < rows_here) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 4 * g + i;
            if (m < M) y[(int64_t)m * ldy + nw + row] = f32_to_bf16_bits(total[i]);
        }
    }
}

template <int W, int D, int NBW, int XA>
hipError_t launch(const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y, int64_t ldy, int M,
                  int N, int K, hipStream_t stream) {
    using C = SmallCfg<W, D, NBW, XA>;
    auto kern = small_m_kernel<W, D, NBW, XA>;
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       (int)C::lds(kMaxM));
    if (attr != hipSuccess) return attr;
    const int groups = (N + C::ROWS - 1) / C::ROWS;
    const size_t lds = C::lds(M);
    hipLaunchKernelGGL(kern, dim3(groups), dim3(64 * W), lds, stream, x, codes, scales, y, ldy, M, N, K);
    return hipGetLastError();
}

}  // namespace

// Four waves share 16 weight rows and split every chunk's 4 blocks, with a
// 4-block ring each.  Activations are prefetched 3 chunks ahead for M > 4
// (73 KiB of LDS at M = 8, two workgroups per CU) and 2 chunks ahead for
// M <= 4, which brings the LDS under 54 KiB and fits three workgroups per CU:
// 7% faster on the 75968-row head at M = 2 and 4, the same elsewhere.  The
// prefetch distance does not change the arithmetic.  Measured on MI355X at
// the decode shapes (M = 2..8) this beats 64-row workgroups (the NBW == 4
// form) for every shape, and deeper rings that leave one workgroup per CU.
hipError_t launch_small_m(const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y,
                          int64_t ldy, int M, int N, int K, int /*split*/, hipStream_t stream) {
    if (M <= 4) return launch<4, 4, 1, 2>(x, codes, scales, y, ldy, M, N, K, stream);
    return launch<4, 4, 1, 3>(x, codes, scales, y, ldy, M, N, K, stream);
}

}  // namespace fp8lin
