// Elementwise kernels: block-FP8 dequantization, SwiGLU, the deterministic
// synthetic-input generators and a streaming-read probe.
#include "device.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

// ---------------------------------------------------------------------------
// Dequantization y[r,c] = bf16(decode(q[r,c]) * s[r, c/128]) (src/kernels.cu:13-16).
// Fast path: 16 codes per thread with one 128-bit load and two 128-bit
// stores (cols % 16 == 0, 16-byte aligned); otherwise one element per thread.
__global__ __launch_bounds__(256) void dequant16_kernel(const uint8_t* __restrict__ q,
                                                        const float* __restrict__ s, int64_t S,
                                                        uint16_t* __restrict__ y, int64_t ldy,
                                                        int64_t rows, int64_t cols) {
    const int64_t per_row = cols >> 4;
    const int64_t total = rows * per_row;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / per_row, c = (i % per_row) << 4;
        const u32x4 codes = load_u32x4_stream(q + r * cols + c);
        const float sc = s[r * S + (S == 1 ? 0 : c >> 7)];
        uint32_t wv[8];
        dequant4(codes.x, sc, wv[0], wv[1]);
        dequant4(codes.y, sc, wv[2], wv[3]);
        dequant4(codes.z, sc, wv[4], wv[5]);
        dequant4(codes.w, sc, wv[6], wv[7]);
        u32x4* dst = reinterpret_cast<u32x4*>(y + r * ldy + c);
        dst[0] = u32x4{wv[0], wv[1], wv[2], wv[3]};
        dst[1] = u32x4{wv[4], wv[5], wv[6], wv[7]};
    }
}

__global__ __launch_bounds__(256) void dequant1_kernel(const uint8_t* __restrict__ q,
                                                       const float* __restrict__ s, int64_t S,
                                                       uint16_t* __restrict__ y, int64_t ldy,
                                                       int64_t rows, int64_t cols) {
    const int64_t total = rows * cols;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / cols, c = i % cols;
        const float v = fp8x2_to_f32<false>((uint32_t)q[i]).x;
        y[r * ldy + c] = f32_to_bf16_bits(v * s[r * S + (S == 1 ? 0 : c >> 7)]);
    }
}

// ---------------------------------------------------------------------------
// SwiGLU over [M, 2D] -> [M, D] (src/optimized.cu:73).
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t* __restrict__ in,
                                                     uint16_t* __restrict__ y, int64_t M,
                                                     int64_t D) {
    const int64_t total = M * D;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / D, j = i % D;
        y[i] = swiglu_bf16_bits(in[r * 2 * D + j], in[r * 2 * D + D + j]);
    }
}

// ---------------------------------------------------------------------------
// Bias add y[r,c] = bf16(y[r,c] + b[c]) in place over rows of stride ldy: the
// BF16 tensor sum `y + bias` of src/engine.cpp:240 (FP32 add, one RNE
// rounding).
__global__ __launch_bounds__(256) void bias_kernel(uint16_t* __restrict__ y, int64_t ldy,
                                                   const uint16_t* __restrict__ b, int64_t rows,
                                                   int64_t cols) {
    const int64_t total = rows * cols;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / cols, c = i % cols;
        uint16_t* p = y + r * ldy + c;
        *p = f32_to_bf16_bits(bf16_bits_to_f32(*p) + bf16_bits_to_f32(b[c]));
    }
}

// ---------------------------------------------------------------------------
// Deterministic normals.  Every multiply-add below is an explicit fmaf or two
// separately rounded operations (contraction is off), so the host checker can
// reproduce the bits exactly with IEEE arithmetic.
__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t h0 = __umulhi(0xD2511F53u, c[0]), l0 = 0xD2511F53u * c[0];
        const uint32_t h1 = __umulhi(0xCD9E8D57u, c[2]), l1 = 0xCD9E8D57u * c[2];
        const uint32_t n0 = h1 ^ c[1] ^ k0, n2 = h0 ^ c[3] ^ k1;
        c[0] = n0;
        c[1] = l1;
        c[2] = n2;
        c[3] = l0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

__device__ __forceinline__ float det_log(float u) {
#pragma clang fp contract(off)
    const uint32_t b = __float_as_uint(u);
    int e = (int)(b >> 23) - 127;
    uint32_t mb = (b & 0x007fffffu) | 0x3f800000u;
    if (mb > 0x3fb504f3u) {
        mb -= 0x00800000u;
        e += 1;
    }
    const float m = __uint_as_float(mb);
    const float t = (m - 1.0f) / (m + 1.0f);
    const float t2 = t * t;
    float p = __builtin_fmaf(t2, 0x1.3b13b2p-4f, 0x1.745d18p-4f);
    p = __builtin_fmaf(t2, p, 0x1.c71c72p-4f);
    p = __builtin_fmaf(t2, p, 0x1.24924ap-3f);
    p = __builtin_fmaf(t2, p, 0x1.99999ap-3f);
    p = __builtin_fmaf(t2, p, 0x1.555556p-2f);
    p = __builtin_fmaf(t2, p, 1.0f);
    const float lnm = (t + t) * p;
    return __builtin_fmaf((float)e, 0x1.62e430p-1f, lnm);
}

__device__ __forceinline__ float det_cos2pi(float u) {
#pragma clang fp contract(off)
    const float q4 = u * 4.0f;
    const int q = (int)q4;
    const float f = q4 - (float)q;
    const float th = f * 0x1.921fb6p+0f;
    const float t2 = th * th;
    float c = __builtin_fmaf(t2, 0x1.1eed8ep-29f, -0x1.27e4fcp-22f);
    c = __builtin_fmaf(t2, c, 0x1.a01a02p-16f);
    c = __builtin_fmaf(t2, c, -0x1.6c16c2p-10f);
    c = __builtin_fmaf(t2, c, 0x1.555556p-5f);
    c = __builtin_fmaf(t2, c, -0.5f);
    c = __builtin_fmaf(t2, c, 1.0f);
    float s = __builtin_fmaf(t2, 0x1.612462p-33f, -0x1.ae6456p-26f);
    s = __builtin_fmaf(t2, s, 0x1.71de3ap-19f);
    s = __builtin_fmaf(t2, s, -0x1.a01a02p-13f);
    s = __builtin_fmaf(t2, s, 0x1.111112p-7f);
    s = __builtin_fmaf(t2, s, -0x1.555556p-3f);
    s = __builtin_fmaf(t2, s, 1.0f);
    s = s * th;
    switch (q & 3) {
        case 0: return c;
        case 1: return -s;
        case 2: return -c;
        default: return s;
    }
}

__device__ __forceinline__ float det_normal(uint64_t seed, uint32_t tag, uint64_t index) {
#pragma clang fp contract(off)
    uint32_t c[4] = {(uint32_t)index, (uint32_t)(index >> 32), tag, 0x6a09e667u};
    philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    const float u1 = (float)((c[0] >> 8) + 1u) * 0x1p-24f;
    const float u2 = (float)(c[1] >> 8) * 0x1p-24f;
    const float rad = __builtin_sqrtf(-2.0f * det_log(u1));
    return rad * det_cos2pi(u2);
}

// Round to nearest even onto the E4M3FN grid; values rounding to 480 or above,
// +-Inf and NaN give the NaN code 0x7f|sign.
__device__ __forceinline__ uint32_t e4m3_rne(float v) {
    const uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
    const float a = fabsf(v);
    if (!(a < 480.0f)) return sign | 0x7fu;
    if (a < 0.015625f) return sign | (uint32_t)__builtin_rintf(a * 512.0f);
    int e2;
    const float f = frexpf(a, &e2);
    int E = e2 - 1;
    const float s = f * 2.0f;
    int mi = (int)__builtin_rintf((s - 1.0f) * 8.0f);
    if (mi == 8) {
        mi = 0;
        E += 1;
    }
    int code = ((E + 7) << 3) | mi;
    if (code >= 0x7f) code = 0x7f;
    return sign | (uint32_t)code;
}

// One workgroup per 128x128 block (tools/make_tiny_fixture.py:56-61).
__global__ __launch_bounds__(256) void gen_weights_kernel(uint64_t seed, uint32_t tag, int64_t N,
                                                          int64_t K, float std_dev,
                                                          uint8_t* __restrict__ codes,
                                                          float* __restrict__ scales) {
    __shared__ float red[4];
    const int64_t KB = (K + 127) / 128;
    const int64_t bn = blockIdx.x / KB, bk = blockIdx.x % KB;
    const int64_t r0 = bn * 128, c0 = bk * 128;
    const int t = threadIdx.x;
    float w[64];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 64; ++i) {
        const int e = t + 256 * i;
        const int64_t r = r0 + (e >> 7), c = c0 + (e & 127);
        float v = 0.0f;
        if (r < N && c < K) {
#pragma clang fp contract(off)
            v = std_dev * det_normal(seed, tag, (uint64_t)(r * K + c));
        }
        w[i] = v;
        amax = fmaxf(amax, fabsf(v));
    }
    for (int d = 32; d >= 1; d >>= 1) amax = fmaxf(amax, __shfl_xor(amax, d, kWave));
    if ((t & 63) == 0) red[t >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float scale = (amax > 1e-12f ? amax : 1e-12f) / 448.0f;
#pragma unroll
    for (int i = 0; i < 64; ++i) {
        const int e = t + 256 * i;
        const int64_t r = r0 + (e >> 7), c = c0 + (e & 127);
        if (r < N && c < K) codes[r * K + c] = (uint8_t)e4m3_rne(w[i] / scale);
    }
    if (t < 128 && r0 + t < N) scales[(r0 + t) * KB + bk] = scale;
}

__global__ __launch_bounds__(256) void gen_activations_kernel(uint64_t seed, uint32_t tag,
                                                              int64_t total,
                                                              uint16_t* __restrict__ x) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x)
        x[i] = f32_to_bf16_bits(det_normal(seed, tag, (uint64_t)i));
}

__global__ __launch_bounds__(256) void gen_normal_kernel(uint64_t seed, uint32_t tag,
                                                         uint64_t first, int64_t n,
                                                         float* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = det_normal(seed, tag, first + (uint64_t)i);
}

// ---------------------------------------------------------------------------
// Streaming read in the decode GEMV's access pattern: each wave reads one
// contiguous 10 KiB chunk with all ten 128-bit non-temporal loads issued
// before the first use (measured on MI355X: 6.4 TB/s at the gate/up size and
// 7.0 TB/s over 1 GiB, where a grid-stride loop with one load in flight per
// lane reached 5.4 and 6.8).  The XOR checksum is reduced over the wave, so
// every lane's loads stay live; a word of sink is written only if it takes an
// unlikely value.  Each workgroup's buffer bounds its own 40 KiB, so any size
// works and the tail reads zeros.
constexpr int kReadChunks = 10;  // 1 KiB loads per wave
constexpr uint64_t kReadBlock = 4 * kReadChunks * 1024;

__global__ __launch_bounds__(256) void stream_read_kernel(const uint8_t* __restrict__ src, uint64_t bytes,
                                                          float* __restrict__ sink) {
    const uint64_t base = (uint64_t)blockIdx.x * kReadBlock;
    const uint64_t left = bytes - base;
    const rsrc_t r = make_rsrc(src + base, (uint32_t)(left < kReadBlock ? left : kReadBlock));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    u32x4 v[kReadChunks];
#pragma unroll
    for (int j = 0; j < kReadChunks; ++j)
        v[j] = buf_load16<2>(r, (uint32_t)((wave * kReadChunks + j) * 1024 + lane * 16));
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < kReadChunks; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    for (int d = 32; d >= 1; d >>= 1) acc ^= __shfl_xor(acc, d, kWave);
    if (lane == 0 && acc == 0x7fc00001u) sink[blockIdx.x & 4095] = 1.0f;
}

// MFMA ceiling: 16 independent 32x32x16 BF16 accumulators per wave, operands
// in registers, so the loop is bound by MFMA issue alone (32 cycles each).
__global__ __launch_bounds__(256) void mfma_ceiling_kernel(int64_t iters, float* __restrict__ sink,
                                                           uint64_t* __restrict__ clocks) {
    typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
    f32x16 acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
    bf16x8_t a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (__bf16)(0.001f * (float)(threadIdx.x + i));
        b[i] = (__bf16)(0.002f * (float)i);
    }
    const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[i], 0, 0, 0);
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[i][r];
    if (s == 1234.5f) sink[0] = s;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        clocks[0] = t1 - t0;
        clocks[1] = r1 - r0;
    }
}

int grid_for(int64_t items, int64_t per_block, int64_t cap) {
    int64_t g = (items + per_block - 1) / per_block;
    if (g < 1) g = 1;
    return (int)(g < cap ? g : cap);
}

}  // namespace

hipError_t launch_dequant(const uint8_t* codes, const float* scales, int64_t S, uint16_t* y,
                          int64_t ldy, int64_t rows, int64_t cols, hipStream_t stream) {
    const bool wide = (cols % 16 == 0) && (ldy % 8 == 0) &&
                      (reinterpret_cast<uintptr_t>(codes) % 16 == 0) &&
                      (reinterpret_cast<uintptr_t>(y) % 16 == 0);
    if (wide) {
        const int64_t items = rows * (cols / 16);
        hipLaunchKernelGGL(dequant16_kernel, dim3(grid_for(items, 256, 8192)), dim3(256), 0, stream,
                           codes, scales, S, y, ldy, rows, cols);
    } else {
        hipLaunchKernelGGL(dequant1_kernel, dim3(grid_for(rows * cols, 256, 65535)), dim3(256), 0,
                           stream, codes, scales, S, y, ldy, rows, cols);
    }
    return hipGetLastError();
}

hipError_t launch_swiglu(const uint16_t* in, uint16_t* y, int64_t M, int64_t D, hipStream_t stream) {
    hipLaunchKernelGGL(swiglu_kernel, dim3(grid_for(M * D, 256, 65535)), dim3(256), 0, stream, in, y,
                       M, D);
    return hipGetLastError();
}

hipError_t launch_bias(uint16_t* y, int64_t ldy, const uint16_t* bias, int64_t rows, int64_t cols,
                       hipStream_t stream) {
    hipLaunchKernelGGL(bias_kernel, dim3(grid_for(rows * cols, 256, 65535)), dim3(256), 0, stream, y, ldy,
                       bias, rows, cols);
    return hipGetLastError();
}

hipError_t launch_gen_weights(uint64_t seed, uint32_t tag, int64_t N, int64_t K, float std_dev,
                              uint8_t* codes, float* scales, hipStream_t stream) {
    const int64_t blocks = ((N + 127) / 128) * ((K + 127) / 128);
    hipLaunchKernelGGL(gen_weights_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, seed, tag,
                       N, K, std_dev, codes, scales);
    return hipGetLastError();
}

hipError_t launch_gen_activations(uint64_t seed, uint32_t tag, int64_t M, int64_t K, uint16_t* x,
                                  hipStream_t stream) {
    hipLaunchKernelGGL(gen_activations_kernel, dim3(grid_for(M * K, 256, 16384)), dim3(256), 0,
                       stream, seed, tag, M * K, x);
    return hipGetLastError();
}

hipError_t launch_gen_normal(uint64_t seed, uint32_t tag, uint64_t first, int64_t n, float* out,
                             hipStream_t stream) {
    hipLaunchKernelGGL(gen_normal_kernel, dim3(grid_for(n, 256, 16384)), dim3(256), 0, stream, seed,
                       tag, first, n, out);
    return hipGetLastError();
}

hipError_t launch_mfma_ceiling(int64_t iters, float* sink, uint64_t* clocks, hipStream_t stream) {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(mfma_ceiling_kernel, dim3(cus), dim3(256), 0, stream, iters, sink, clocks);
    return hipGetLastError();
}

hipError_t launch_stream_read(const void* src, size_t bytes, float* sink, hipStream_t stream) {
    const uint64_t blocks = (bytes + kReadBlock - 1) / kReadBlock;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const uint8_t*>(src), (uint64_t)bytes, sink);
    return hipGetLastError();
}

}  // namespace fp8lin
