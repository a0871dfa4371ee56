// Small-M (2..8 activation rows) block-FP8 linear on the matrix cores.
//
// Contract of fp8_tensor_small (src/fp8_tensor.cu:18-71): K % 128 == 0, block
// scales [N, K/128], the weight tile is decoded to BF16 with the reference
// rounding point bf16(decode(c) * s) before the BF16 matrix multiply, FP32
// accumulation.  split == 4 divides the K blocks into four ranges exactly as
// the reference does (steps = ceil(blocks/4), range i = [i*steps, ...)) and
// reduces the FP32 partials in the order ((p0+p1)+p2)+p3 (:48-51).
//
// MI355X design: one workgroup of 4 waves owns 16 weight rows.  The 4 waves
// take interleaved 128-wide K blocks of the workgroup's range and their 16x16
// accumulators are added in LDS in a fixed order.  Per 128-K block a lane
// loads 2x16 codes of its row with 128-bit loads (lane l: row l%16, K offset
// 16*(l/16) + 64*h), converts them in registers and feeds them straight into
// v_mfma_f32_16x16x32_bf16 as the B operand; the activations (rows >= M are
// zero) are the A operand loaded with the same K permutation.  No LDS staging
// of the weights: FP8 bytes go HBM -> VGPR -> BF16 -> MFMA.
#include "device.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

constexpr int kSmallThreads = 256;
constexpr int kSmallWaves = kSmallThreads / kWave;

__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4 v{a, b, c, d};
    return __builtin_bit_cast(bf16x8, v);
}

__global__ __launch_bounds__(kSmallThreads) void small_m_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ codes,
    const float* __restrict__ scales, uint16_t* __restrict__ y, int64_t ldy,
    float* __restrict__ partial, int M, int N, int K) {
    __shared__ float red[kSmallWaves][256];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int n0 = blockIdx.x * 16;
    const int split = gridDim.y, sidx = blockIdx.y;
    const int KB = K >> 7;
    const int steps = (KB + split - 1) / split;
    const int begin = sidx * steps;
    const int end = min(KB, begin + steps);

    const int col = lane & 15, g = lane >> 4;
    const int64_t row = min(n0 + col, N - 1);
    const uint8_t* wrow = codes + row * (int64_t)K;
    const float* srow = scales + row * (int64_t)KB;
    const bool xrow_valid = col < M;
    const uint16_t* xrow = x + (int64_t)(xrow_valid ? col : 0) * K;

    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    int kb = begin + wave;
    u32x4 c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
    float s = 0.0f;
    if (kb < end) {
        c0 = load_u32x4_stream(wrow + kb * 128 + 16 * g);
        c1 = load_u32x4_stream(wrow + kb * 128 + 64 + 16 * g);
        s = srow[kb];
    }
    for (; kb < end; kb += kSmallWaves) {
        const int kn = kb + kSmallWaves;
        u32x4 n0c = {0, 0, 0, 0}, n1c = {0, 0, 0, 0};
        float sn = 0.0f;
        if (kn < end) {
            n0c = load_u32x4_stream(wrow + kn * 128 + 16 * g);
            n1c = load_u32x4_stream(wrow + kn * 128 + 64 + 16 * g);
            sn = srow[kn];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const u32x4 cw = h ? c1 : c0;
            uint32_t wv[8];
            dequant4(cw.x, s, wv[0], wv[1]);
            dequant4(cw.y, s, wv[2], wv[3]);
            dequant4(cw.z, s, wv[4], wv[5]);
            dequant4(cw.w, s, wv[6], wv[7]);
            u32x4 xa = {0, 0, 0, 0}, xb = {0, 0, 0, 0};
            if (xrow_valid) {
                xa = load_u32x4(xrow + kb * 128 + 64 * h + 16 * g);
                xb = load_u32x4(xrow + kb * 128 + 64 * h + 16 * g + 8);
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, xa), as_bf16x8(wv[0], wv[1], wv[2], wv[3]), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, xb), as_bf16x8(wv[4], wv[5], wv[6], wv[7]), acc, 0, 0, 0);
        }
        c0 = n0c;
        c1 = n1c;
        s = sn;
    }
    // acc[r] = C[4*g + r][col]
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][(4 * g + r) * 16 + col] = acc[r];
    __syncthreads();
    const int t = threadIdx.x;  // 256 outputs: m = t/16, n = t%16
    const int m = t >> 4, n = n0 + (t & 15);
    const float total = ((red[0][t] + red[1][t]) + red[2][t]) + red[3][t];
    if (m < M && n < N) {
        if (partial)
            partial[((int64_t)sidx * M + m) * N + n] = total;
        else
            y[(int64_t)m * ldy + n] = f32_to_bf16_bits(total);
    }
}

// y = bf16(((p0 + p1) + p2) + ...) in index order (src/fp8_tensor.cu:48-51).
__global__ __launch_bounds__(256) void reduce_partials_kernel(const float* __restrict__ p,
                                                              uint16_t* __restrict__ y,
                                                              int64_t ldy, int M, int N,
                                                              int split) {
    const int64_t elements = (int64_t)M * N;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < elements;
         i += (int64_t)gridDim.x * blockDim.x) {
        float t = p[i];
        for (int s = 1; s < split; ++s) t = t + p[s * elements + i];
        const int64_t m = i / N, n = i % N;
        y[m * ldy + n] = f32_to_bf16_bits(t);
    }
}

}  // namespace

hipError_t launch_small_m(const uint16_t* x, const uint8_t* codes, const float* scales,
                          uint16_t* y, int64_t ldy, int M, int N, int K, int split,
                          float* partial, hipStream_t stream) {
    dim3 grid((N + 15) / 16, split);
    hipLaunchKernelGGL(small_m_kernel, grid, dim3(kSmallThreads), 0, stream, x, codes, scales, y,
                       ldy, split > 1 ? partial : nullptr, M, N, K);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || split == 1) return e;
    const int64_t elements = (int64_t)M * N;
    int blocks = (int)((elements + 255) / 256);
    if (blocks > 65535) blocks = 65535;
    hipLaunchKernelGGL(reduce_partials_kernel, dim3(blocks), dim3(256), 0, stream, partial, y, ldy,
                       M, N, split);
    return hipGetLastError();
}

}  // namespace fp8lin
