// Device-side helpers shared by the fp8lin kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fp8lin {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Two E4M3FN bytes of `word` (bytes 0,1 when hi == false, bytes 2,3 when
// hi == true) to two exact floats.  gfx950's v_cvt_pk_f32_fp8 uses the OCP
// E4M3FN encoding: bias 7, subnormals m*2^-9, 0x7f/0xff NaN -- the decode of
// include/avi/fp8_codec.cuh:5-10 (checked over all 256 codes by the tests).
template <bool HI>
__device__ __forceinline__ f32x2 fp8x2_to_f32(uint32_t word) {
    return __builtin_amdgcn_cvt_pk_f32_fp8(word, HI);
}

// Two floats to packed BF16 with round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(f32x2 v) {
    bf16x2 p = __builtin_convertvector(v, bf16x2);
    return __builtin_bit_cast(uint32_t, p);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
    __bf16 b = (__bf16)v;
    return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
    return __builtin_bit_cast(float, bits16 << 16);
}

// Four E4M3FN codes (one dword) times `s`, rounded to BF16 at the reference's
// rounding point bf16(decode(c) * s) (src/optimized.cu:22), as two packed
// BF16 pairs: out0 = (c0, c1), out1 = (c2, c3).
__device__ __forceinline__ void dequant4(uint32_t codes, float s, uint32_t& out0, uint32_t& out1) {
    f32x2 lo = fp8x2_to_f32<false>(codes);
    f32x2 hi = fp8x2_to_f32<true>(codes);
    lo.x *= s;
    lo.y *= s;
    hi.x *= s;
    hi.y *= s;
    out0 = pack_bf16x2(lo);
    out1 = pack_bf16x2(hi);
}

// acc + a.lo*b.lo + a.hi*b.hi over packed BF16 pairs (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), acc, false);
}

// ---- vocabulary candidates ----
// (value, id) order: larger value first, then the smaller id.  It is a total
// order on the pairs, so any reduction tree gives the reference's result
// (torch.max over a row, src/dual_path.cu:37-55).
__device__ __forceinline__ void pick(float& v, uint32_t& id, float ov, uint32_t oid) {
    if (ov > v || (ov == v && oid < id)) {
        v = ov;
        id = oid;
    }
}

// The best pair of the 64 lanes of a wave (every lane gets it).
__device__ __forceinline__ void wave_pick(float& v, uint32_t& id) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const float ov = __shfl_xor(v, d, kWave);
        const uint32_t oid = __shfl_xor(id, d, kWave);
        pick(v, id, ov, oid);
    }
}

// NaN counts as +inf: the row's candidate becomes non-finite and the merge
// rejects it, as torch.max's NaN propagation does in the reference.
__device__ __forceinline__ void pick_bf16(float& v, uint32_t& id, uint32_t bits, uint32_t i) {
    float f = bf16_bits_to_f32(bits);
    if (f != f) f = __builtin_inff();
    pick(v, id, f, i);
}

// Butterfly sum over the 64 lanes of a wave; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
    return v;
}

__device__ __forceinline__ u32x4 load_u32x4(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

// Non-temporal 128-bit load for data that is read exactly once (weights).
__device__ __forceinline__ u32x4 load_u32x4_stream(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Raw buffer resources (V#) for branch-free loads: a lane whose byte offset is
// at or beyond `num_records` reads zeros instead of faulting, so a guarded load
// needs no branch and the compiler's wait counting stays exact.  Dword 3 is the
// gfx9-family raw-buffer format word.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kBufferOob = 0x80000000u;  // offset used for masked lanes

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_bytes,
                                             0x00020000);
}

// AUX: cache policy bits of the load (2 = non-temporal on gfx950).
template <int AUX>
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, AUX));
}
__device__ __forceinline__ float buf_load_f32(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

}  // namespace fp8lin

namespace fp8lin {

// SwiGLU of one (gate, up) pair, with the reference's rounding points
// (src/optimized.cu:73): a and u are BF16 values (BF16 tensors in the
// reference), g = bf16(a / (1 + exp(-a))), y = bf16(g * u), with an accurate
// expf and an IEEE division so g stays within 1 BF16 ulp of the exact value.
// Shared by the standalone kernel and every GEMM and GEMV epilogue, so the
// fused and unfused paths agree bit for bit.
//
// g is computed first with the hardware exp2 and reciprocal
// (exp(-a) = 2^(-a*log2(e)), then a * rcp(1 + e)).  For a >= -64 that value
// is within 53 FP32 ulp of the accurate one (the argument's rounding, up to
// 2^-18 absolute below 128, dominates).  g depends on a alone and a is BF16,
// so the 65 536 inputs can be enumerated: for every a >= -64 the BF16
// rounding of the fast value differs from the accurate quotient's only where
// the fast value's low 16 bits lie within 4 of the rounding midpoint 0x8000.
// Values within 8 of it (about 0.02% of typical gates, so under 2% of
// 64-lane groups need the slow path at all), and a < -64 (where
// 1 / (1 + e) is an FP32 denormal that the reciprocal flushes to zero), take
// the accurate expf and division.  The tests check all 65 536 gate values.
__device__ __forceinline__ float swiglu_gate_exact(float a) {
    return a / (1.0f + expf(-a));
}

// The fast quotient, and whether this input must take the accurate path.
__device__ __forceinline__ float swiglu_gate_fast(float a, bool& need) {
    const float e = __builtin_amdgcn_exp2f(a * -1.44269504088896340736f);
    const float gf = a * __builtin_amdgcn_rcpf(1.0f + e);
    const uint32_t low = __builtin_bit_cast(uint32_t, gf) & 0xffffu;
    need = !(a >= -64.0f) || (low > 0x8000u - 8u && low < 0x8000u + 8u);
    return gf;
}

// y = bf16(bf16(g) * u) from the FP32 gate quotient.
__device__ __forceinline__ uint16_t swiglu_finish(float gf, float u) {
    const float g = bf16_bits_to_f32(f32_to_bf16_bits(gf));
    return f32_to_bf16_bits(g * u);
}

__device__ __forceinline__ uint16_t swiglu_bf16_bits(uint16_t a_bits, uint16_t u_bits) {
    const float a = bf16_bits_to_f32(a_bits);
    bool need;
    float gf = swiglu_gate_fast(a, need);
    if (need) gf = swiglu_gate_exact(a);
    return swiglu_finish(gf, bf16_bits_to_f32(u_bits));
}

// NB SwiGLU outputs at once, each from a packed (gate | up << 16) BF16 pair:
// the same arithmetic as swiglu_bf16_bits, laid out for a wave that runs
// alone on its SIMD (a GEMM epilogue).  The NB fast quotients are
// independent, so their instructions interleave instead of waiting on each
// other's latency, and the rare accurate path is one branch per batch.
template <int NB>
__device__ __forceinline__ void swiglu_bf16_batch(const uint32_t (&gu)[NB], uint16_t (&out)[NB]) {
    float gf[NB];
    uint32_t need = 0;
#pragma unroll
    for (int k = 0; k < NB; ++k) {
        bool n;
        gf[k] = swiglu_gate_fast(bf16_bits_to_f32(gu[k] & 0xffffu), n);
        need |= (uint32_t)n << k;
    }
    if (need) {
#pragma unroll
        for (int k = 0; k < NB; ++k)
            if ((need >> k) & 1u) gf[k] = swiglu_gate_exact(bf16_bits_to_f32(gu[k] & 0xffffu));
    }
#pragma unroll
    for (int k = 0; k < NB; ++k) out[k] = swiglu_finish(gf[k], bf16_bits_to_f32(gu[k] >> 16));
}

}  // namespace fp8lin
