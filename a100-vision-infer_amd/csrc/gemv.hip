// Decode GEMV dispatch for 1..8 activation rows (kernels in gemv_kernel.hpp).
//
// Reference numerics (src/optimized.cu:20-23, :42-60; src/deep_kernels.cu:23-63):
//   y[m,n] = bf16( sum_k x[m,k] * bf16(decode(code[n,k]) * scale[n, k/128]) )
// with FP32 accumulation.  The reference runs one 32-lane warp per weight row;
// here 64-lane waves stream the weights with 128-bit loads, convert the codes
// with v_cvt_pk_f32_fp8, multiply by the block scale, round to BF16 with
// v_cvt_pk_bf16_f32 (the reference's rounding point) and accumulate with
// v_dot2_f32_bf16.
//
// Accumulation order: for K <= 9216 every path sums a row's steps in order
// inside one wave (the "W = 1" order); above that, and for M > 2 against at
// most 1024 weight rows, four waves split the steps (W = 4).  The choice
// depends only on M, N and K, never on the weight type, on pointer alignment
// or on which kernel runs, so the byte-load fallback and the BF16-weight
// (decoded cache) variant give bit-identical results to the 128-bit FP8 path,
// as the reference's tests require (tests/optimized_test.cpp:11-12, :57-62).
//
// Kernel choice for the 128-bit path, FP8 or BF16 weights (measured on
// MI355X, decode shapes): the unrolled ring kernel with the row group's loads
// all in flight, four waves per workgroup -- R = 1 rows for K <= 4096, R = 2
// for K <= 5120, R = 1 for K <= 9216 (R = 2 for the SwiGLU form, whose rows
// come in gate/up pairs); below 16384 rows with K <= 5120, R = 2 and two
// waves per workgroup; up to 1024 weight rows, one wave per workgroup.
#include "gemv_kernel.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

constexpr int kRingMaxK = 9216;  // 9 steps of 1024
constexpr int kNT = 2;           // non-temporal weight loads (gfx950 cache policy)

// Up to this many weight rows the ring kernel runs one wave per workgroup
// and, outside SwiGLU, one row per wave: a few rows then spread over as many
// CUs as there are rows (the GDN in_proj_all group's 48 BF16 rows took 6 µs
// on 12 CUs).  R and the waves per workgroup change no result: each row is
// summed by one wave in step order either way.
constexpr int kFewRows = 1024;

template <int MR, bool FP8, bool SWIGLU>
hipError_t ring(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y, int64_t ldy, int M,
                int N, int K, hipStream_t stream) {
    using namespace gemv;
    if (N <= kFewRows) {
        constexpr int R = SWIGLU ? 2 : 1;
        if (K <= 4096) return launch_ring<MR, R, 4, FP8, SWIGLU, kNT, 1>(x, w, scales, S, y, ldy, M, N, K, stream);
        if (K <= 5120) return launch_ring<MR, R, 5, FP8, SWIGLU, kNT, 1>(x, w, scales, S, y, ldy, M, N, K, stream);
        return launch_ring<MR, R, 9, FP8, SWIGLU, kNT, 1>(x, w, scales, S, y, ldy, M, N, K, stream);
    }
    // Up to kSharedXRows rows with K <= 5120 (the 7168-row QKV-gate, the
    // 8192-row in_proj_all group, config 1's 4096 rows): two rows per wave and
    // two waves per workgroup, about 3% faster than one row per wave or
    // four-wave workgroups at those shapes (graph-replayed medians).
    if (N < gemv::kSharedXRows && K <= 5120) {
        if (K <= 4096) return launch_ring<MR, 2, 4, FP8, SWIGLU, kNT, 2>(x, w, scales, S, y, ldy, M, N, K, stream);
        return launch_ring<MR, 2, 5, FP8, SWIGLU, kNT, 2>(x, w, scales, S, y, ldy, M, N, K, stream);
    }
    if (K <= 4096) {
        if constexpr (SWIGLU)
            return launch_ring<MR, 2, 4, FP8, SWIGLU, kNT>(x, w, scales, S, y, ldy, M, N, K, stream);
        else
            return launch_ring<MR, 1, 4, FP8, SWIGLU, kNT>(x, w, scales, S, y, ldy, M, N, K, stream);
    }
    if (K <= 5120) return launch_ring<MR, 2, 5, FP8, SWIGLU, kNT>(x, w, scales, S, y, ldy, M, N, K, stream);
    if constexpr (SWIGLU)
        return launch_ring<MR, 2, 9, FP8, SWIGLU, kNT>(x, w, scales, S, y, ldy, M, N, K, stream);
    else
        return launch_ring<MR, 1, 9, FP8, SWIGLU, kNT>(x, w, scales, S, y, ldy, M, N, K, stream);
}

// General kernel with the same W as the ring path for this K.
template <int MR, int R, bool FP8, bool SWIGLU>
hipError_t general(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
                   int64_t ldy, int M, int N, int K, bool wide, hipStream_t stream) {
    using namespace gemv;
    // More than 2 rows against a few weight rows: no ring form exists for
    // these M, so the 128-bit, byte-load, FP8 and BF16 forms all run this
    // kernel, and the four-wave step split (one row per workgroup) is free to
    // choose: 4x the waves on a 48-row group.
    if (M > 2 && N <= kFewRows) {
        constexpr int R1 = SWIGLU ? 2 : 1;
        return launch<MR, R1, 4, FP8, SWIGLU, true>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
    }
    if (K <= kRingMaxK) return launch<MR, R, 1, FP8, SWIGLU, true>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
    return launch<MR, R, 4, FP8, SWIGLU, true>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
}

// Whether the 128-bit path runs the ring kernel (raw-buffer kernels take
// 32-bit byte offsets).
bool ring_path(bool fp8, bool wide, int M, int N, int K) {
    if (!(wide && K <= kRingMaxK && (int64_t)N * K * (fp8 ? 1 : 2) < ((int64_t)1 << 31) &&
          (int64_t)M * K * 2 < ((int64_t)1 << 31)))
        return false;
    return M <= 1 || (M <= 2 && K <= 5120);
}

template <bool FP8, bool SWIGLU>
hipError_t dispatch(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
                    int64_t ldy, int M, int N, int K, bool wide, hipStream_t stream) {
    if (ring_path(FP8, wide, M, N, K)) {
        if (M <= 1) return ring<1, FP8, SWIGLU>(x, w, scales, S, y, ldy, M, N, K, stream);
        return ring<2, FP8, SWIGLU>(x, w, scales, S, y, ldy, M, N, K, stream);
    }
    if (M <= 1) return general<1, 4, FP8, SWIGLU>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
    if (M <= 2) return general<2, 4, FP8, SWIGLU>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
    if (M <= 4) return general<4, 2, FP8, SWIGLU>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
    return general<8, 2, FP8, SWIGLU>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
}

// The ring kernel with the candidate epilogue (the same per-row totals as
// ring<MR, true, false>: one wave sums each row in step order).
template <int MR>
hipError_t ring_cand(const uint16_t* x, const uint8_t* w, const float* scales, int S, int M, int N, int K,
                     uint32_t* part, uint32_t* counters, int64_t& chunks, hipStream_t stream) {
    using namespace gemv;
    if (K <= 4096) {
        chunks = ring_cand_blocks<MR, 1, 4, kNT>(N);
        return launch_ring_cand<MR, 1, 4, kNT>(x, w, scales, S, M, N, K, part, counters, stream);
    }
    if (K <= 5120) {
        chunks = ring_cand_blocks<MR, 2, 5, kNT>(N);
        return launch_ring_cand<MR, 2, 5, kNT>(x, w, scales, S, M, N, K, part, counters, stream);
    }
    chunks = ring_cand_blocks<MR, 1, 9, kNT>(N);
    return launch_ring_cand<MR, 1, 9, kNT>(x, w, scales, S, M, N, K, part, counters, stream);
}

// Workspace of the candidate form: the workgroup pairs (at most one per 4
// columns: R = 1, four waves per workgroup), 256-byte aligned, then the
// finishing launch's slice pairs and arrival counters.
size_t pairs_bytes(int M, int N) { return ((size_t)M * (size_t)((N + 3) / 4 + 7) * 8 + 255) / 256 * 256; }

}  // namespace

bool gemv_candidates_supported(int M, int N, int K, bool wide) { return ring_path(true, wide, M, N, K); }

size_t gemv_candidates_ws_bytes(int M, int N) {
    return pairs_bytes(M, N) + (size_t)M * kCandSlices * 8 + (size_t)M * 4;
}

hipError_t launch_gemv_candidates(const uint16_t* x, const uint8_t* codes, const float* scales, int S, int M,
                                  int N, int K, int64_t offset, void* ws, double* out, hipStream_t stream) {
    auto* part = static_cast<uint32_t*>(ws);
    auto* slices = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + pairs_bytes(M, N));
    uint32_t* counters = slices + (size_t)M * kCandSlices * 2;
    int64_t chunks = 0;
    const hipError_t e = M <= 1 ? ring_cand<1>(x, codes, scales, S, M, N, K, part, counters, chunks, stream)
                                : ring_cand<2>(x, codes, scales, S, M, N, K, part, counters, chunks, stream);
    if (e != hipSuccess) return e;
    return launch_candidates_finish_sliced(part, M, chunks, slices, counters, offset, out, stream);
}

hipError_t launch_gemv_rows(const uint16_t* x, const void* w, bool fp8, const float* scales, int S, uint16_t* y,
                            int64_t ldy, int M, int N, int K, bool wide, bool swiglu, hipStream_t stream) {
    using namespace gemv;
    if (fp8)
        return swiglu ? launch<8, 4, 4, true, true, true>(x, w, scales, S, y, ldy, M, N, K, wide, stream)
                      : launch<8, 4, 4, true, false, true>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
    return swiglu ? launch<8, 4, 4, false, true, true>(x, w, nullptr, 1, y, ldy, M, N, K, wide, stream)
                  : launch<8, 4, 4, false, false, true>(x, w, nullptr, 1, y, ldy, M, N, K, wide, stream);
}

hipError_t launch_gemv(const uint16_t* x, const void* w, bool fp8, const float* scales, int S,
                       uint16_t* y, int64_t ldy, int M, int N, int K, bool wide,
                       hipStream_t stream) {
    if (fp8) return dispatch<true, false>(x, w, scales, S, y, ldy, M, N, K, wide, stream);
    return dispatch<false, false>(x, w, nullptr, 1, y, ldy, M, N, K, wide, stream);
}

// The FP8 weight (kFewRows < na < kSharedXRows rows: the ring kernel's
// two-row, two-wave form) and the BF16 weight (nb <= kFewRows rows: one row
// per wave) of one activation row, K <= 5120, 128-bit operands, in one launch
// (gemv_ring_pair_kernel); hipErrorNotSupported outside that.
hipError_t launch_gemv_pair(const uint16_t* x, const uint8_t* codes, const float* scales, int S, uint16_t* ya,
                            int na, const uint16_t* wb, uint16_t* yb, int nb, int64_t ldy, int K,
                            hipStream_t stream) {
    using namespace gemv;
    if (!(na > kFewRows && na < kSharedXRows && nb >= 1 && nb <= kFewRows && K >= 16 && K <= 5120 &&
          K % 16 == 0))
        return hipErrorNotSupported;
    const int blocks_a = ((na + 1) / 2 + 1) / 2;
    const int blocks = blocks_a + (nb + 1) / 2;
    if (K <= 4096)
        hipLaunchKernelGGL((gemv_ring_pair_kernel<4, kNT>), dim3((unsigned)blocks), dim3(128), 0, stream, x, codes,
                           scales, S, ya, na, wb, yb, nb, ldy, K, blocks_a);
    else
        hipLaunchKernelGGL((gemv_ring_pair_kernel<5, kNT>), dim3((unsigned)blocks), dim3(128), 0, stream, x, codes,
                           scales, S, ya, na, wb, yb, nb, ldy, K, blocks_a);
    return hipGetLastError();
}

hipError_t launch_gemv_swiglu(const uint16_t* x, const uint8_t* codes, const float* scales, int S,
                              uint16_t* y, int64_t ldy, int M, int N, int K, bool wide,
                              hipStream_t stream) {
    return dispatch<true, true>(x, codes, scales, S, y, ldy, M, N, K, wide, stream);
}

}  // namespace fp8lin
