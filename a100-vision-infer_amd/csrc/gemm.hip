// Prefill GEMM dispatch.  FP8 weights with K % 256 == 0 (every benchmark
// shape) run gemm_fp8_kernel (gemm_fp8.hpp); other K, unaligned operands and
// BF16 weights run the general template of gemm_kernel.hpp.
//
// General template, as measured on MI355X at the prefill shapes (M =
// 512..4096, N = 17408, K = 5120, fused SwiGLU): a 256x256 workgroup tile of 8 waves
// (2 along M x 4 along N, 128x64 per wave as 4x2 accumulators of
// v_mfma_f32_32x32x16_bf16), K step 64, global loads issued two K steps ahead,
// the next stage's FP8 dequantization and LDS store placed after the second
// MFMA group, and the scheduler's MFMA/LDS interleave strategy 1.
#include <algorithm>
#include <atomic>

#include "gemm_fp8.hpp"
#include "gemm_kernel.hpp"
#include "internal.hpp"

namespace fp8lin {
namespace {

using Tile = gemm::Cfg<256, 256, 64, 2, 4>;
constexpr int kGroupM = 8;   // XCD-local tile patch height
constexpr int kIglp = 1;     // MFMA / LDS interleave strategy
constexpr int kPrefetch = 2; // global loads two K steps ahead
constexpr int kStoreAt = 1;  // next-stage store after MFMA sub-step 1

template <bool FP8, bool SWIGLU>
hipError_t run(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
               int64_t ldy, int M, int N, int K, hipStream_t stream) {
    return gemm::launch<Tile, FP8, SWIGLU, kGroupM, kIglp, kPrefetch, kStoreAt>(x, w, scales, S, y, ldy,
                                                                             M, N, K, stream);
}

// Work plan of the persistent FP8 GEMM (see gemm_fp8.hpp).  Without a
// workspace every tile is computed whole.  With one, K is split where the
// tile count leaves CUs idle:
//  - fewer tiles than half the CUs (e.g. the prefill QKV-gate and down
//    projections at M = 512): every tile, into min(G / T, K / 256, 8)
//    ranges;
//  - otherwise a last round of at most half the CUs (M = 1024: 16 of 272
//    tiles; M = 4096: 64 of 1088; the M = 512 output head: 82 of 594): those
//    tiles, into min(G / R, K / 256, 8) ranges.  A last round over more than
//    half the CUs stays whole: splitting it would not shorten the CUs that
//    run an unsplit tile.
gemm_fp8::Plan plan_for(int bm, int M, int N, int K, bool swiglu, int G, bool split) {
    using namespace gemm_fp8;
    Plan p;
    p.bm = bm;
    p.mtiles = (M + bm - 1) / bm;
    p.ntiles = swiglu ? ((N >> 1) + BN / 2 - 1) / (BN / 2) : (N + BN - 1) / BN;
    const int T = p.mtiles * p.ntiles;
    p.full = T;
    p.rtiles = 0;
    p.splits = 1;
    if (split) {
        const int chunks = K / 256;
        if (2 * T <= G) {
            const int s = std::min(std::min(G / T, chunks), kMaxSplits);
            if (s > 1) {
                p.full = 0;
                p.rtiles = T;
                p.splits = s;
            }
        } else if (T > G && T % G != 0 && 2 * (T % G) <= G) {
            const int R = T % G;
            const int s = std::min(std::min(G / R, chunks), kMaxSplits);
            if (s > 1) {
                p.full = T - R;
                p.rtiles = R;
                p.splits = s;
            }
        }
    }
    p.fpad = (p.full + kXcds - 1) / kXcds * kXcds;
    p.units = p.fpad + p.rtiles * p.splits;
    return p;
}

size_t plan_bytes(const gemm_fp8::Plan& p) {
    return (size_t)p.rtiles * p.splits * p.bm * gemm_fp8::BN * sizeof(float);
}

// The plan of a launch.  M <= 128 (one tile row) takes 128-row tiles: the
// same outputs at half the MFMA work of a 256-row tile that is at least half
// padding.  Above that the 256-row tile stays: measured on MI355X, a 128-row
// tile costs 0.62 (whole chip) to 0.77 (one partial round) of a 256-row tile
// (its K loop issues 4 dequant VALU per MFMA instead of 2, with the same
// per-step waits), so two of them cost more than the one they replace.
// Both heights give each output the same FP32 sum over a K range.
gemm_fp8::Plan make_plan(int M, int N, int K, bool swiglu, int G, bool split) {
    return plan_for(M <= 128 ? 128 : 256, M, N, K, swiglu, G, split);
}

template <int MT, bool SWIGLU>
hipError_t run_fp8_mt(const uint16_t* x, const uint8_t* w, const float* scales, int S, uint16_t* y, int64_t ldy,
                      int M, int N, int K, const gemm_fp8::Plan& plan, int G, float* part, hipStream_t stream) {
    using namespace gemm_fp8;
    using Gm = Geo<MT>;
    auto kern = gemm_fp8_kernel<MT, SWIGLU>;
    static const hipError_t attr = gemm::allow_lds(reinterpret_cast<const void*>(kern), Gm::LDS_BYTES);
    if (attr != hipSuccess) return attr;
    const int grid = std::min(plan.units, G);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(THREADS), Gm::LDS_BYTES, stream, x, w, scales, S, y, (int)ldy, M, N,
                       K, plan, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || plan.rtiles == 0) return e;
    const int64_t threads = (int64_t)plan.rtiles * Gm::BM * (SWIGLU ? 32 : 64);
    hipLaunchKernelGGL((tail_reduce_kernel<MT, SWIGLU>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       stream, part, plan, M, N, y, ldy);
    return hipGetLastError();
}

template <bool SWIGLU>
hipError_t run_fp8(const uint16_t* x, const uint8_t* w, const float* scales, int S, uint16_t* y, int64_t ldy,
                   int M, int N, int K, const gemm_fp8::Plan& plan, int G, float* part, hipStream_t stream) {
    return plan.bm == 128 ? run_fp8_mt<4, SWIGLU>(x, w, scales, S, y, ldy, M, N, K, plan, G, part, stream)
                          : run_fp8_mt<8, SWIGLU>(x, w, scales, S, y, ldy, M, N, K, plan, G, part, stream);
}

// Shapes and alignments the FP8 kernel takes.
bool fp8_kernel_ok(const uint16_t* x, const void* w, int S, int64_t ldy, int M, int N, int K) {
    return gemm_fp8::supported(x, w, S, ldy, M, N, K);
}

// A few weight rows (N <= kSkinnyRows, as the GDN in_proj_all group's 48 BF16
// rows): 256x256 tiles would run M/256 workgroups, so the skinny MFMA kernel
// takes them (16 x 16 output tiles, K split over 4 waves; skinny.hip), or,
// for K % 32 != 0 or unaligned operands, the GEMV's prefill form (8
// activation rows per workgroup row).  N counts weight rows in both forms, so
// the fused SwiGLU GEMM and the plain GEMM of one weight take the same kernel
// (and give the same sums).
bool skinny(int M, int N, bool /*swiglu*/) { return M > 8 && N <= kSkinnyRows; }

hipError_t launch_skinny(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y, int64_t ldy,
                         int M, int N, int K, bool swiglu, hipStream_t stream) {
    if (skinny_mfma_supported(x, w, scales != nullptr, S, M, N, K))
        return launch_skinny_mfma(x, w, scales != nullptr, scales, S, y, ldy, M, N, K, swiglu, stream);
    const bool wide = K % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(w) % 16 == 0;
    return launch_gemv_rows(x, w, scales != nullptr, scales, S, y, ldy, M, N, K, wide, swiglu, stream);
}

// 9..16 activation rows of a block-FP8 weight of more than 1024 rows: the
// small-M matrix-core kernels (small_m.hip), whose 16x16 MFMA tile holds all
// of them, stream the codes once with each dequantized once (the wide
// row-staged form up to 64 rows per CU, else the row-range form or the
// K-split 16-row tiles); a GEMM tile would be at least seven eighths
// padding.  17..32 rows in the wide row-staged form with 32 staged
// activation rows (up to 32 weight rows per CU), else in the row-range form
// with two activation tiles (K <= 5120) or the K-split 16-row tiles with two
// activation tiles.  33..64 rows where the row-staged form holds them (64
// staged rows in 256-byte stages, up to 32 weight rows per CU), else the
// GEMM.  Its geometry limits are those of the decode routing (block scales
// [N, K/128], 16-byte aligned x and codes).
bool mid_rows(const uint16_t* x, const void* w, int S, int64_t M, int64_t N, int64_t K) {
    const int64_t lim = (int64_t)1 << 31;
    if (M > 32 && !(M <= 64 && N < lim && K < lim && small_m_wide_rows((int)M, (int)N, (int)K))) return false;
    return M > 8 && N > 1024 && K % 128 == 0 && S == K / 128 &&
           reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 && 16 * K < lim &&
           N * S * 4 < lim && M * K * 2 < lim;
}

}  // namespace

bool gemm_mid_rows(const uint16_t* x, const void* w, int S, int64_t M, int64_t N, int64_t K) {
    return mid_rows(x, w, S, M, N, K);
}

namespace {

// 65..128 rows where both halves are mid rows (narrow weights) and the GEMM
// would run its tiles whole (no split-K workspace): two passes of the small-M
// kernels, each half as a call of its own rows.  Whole tiles run one
// workgroup per 128x256 tile (20 on the 5120-row down projection: 144 us
// against about 50 for the halves); where a workspace lets the GEMM split K
// it stays, being faster (29-38 us there).
bool halves(const uint16_t* x, const void* w, int S, int M, int N, int K) {
    return M > 64 && M <= 128 && mid_rows(x, w, S, M / 2, N, K) && mid_rows(x, w, S, M - M / 2, N, K);
}

hipError_t launch_halves(const uint16_t* x, const uint8_t* codes, const float* scales, uint16_t* y, int64_t ldy,
                         int M, int N, int K, bool swiglu, hipStream_t stream) {
    const int h = M - M / 2;
    const hipError_t e = launch_small_m(x, codes, scales, y, ldy, h, N, K, 1, swiglu, stream);
    if (e != hipSuccess) return e;
    return launch_small_m(x + (int64_t)h * K, codes, scales, y + (int64_t)h * ldy, ldy, M - h, N, K, 1, swiglu,
                          stream);
}

}  // namespace

// Compute units of the current device (cached per device), rounded down to a
// multiple of the 8 XCDs: the persistent kernels' grid size.
int compute_units() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 8) cus = 256;
        v = cus / gemm_fp8::kXcds * gemm_fp8::kXcds;
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

size_t gemm_workspace_bytes(int S, int64_t ldy, int M, int N, int K, bool swiglu) {
    if (skinny(M, N, swiglu) || mid_rows(nullptr, nullptr, S, M, N, K) ||
        !fp8_kernel_ok(nullptr, nullptr, S, ldy, M, N, K))
        return 0;
    return plan_bytes(make_plan(M, N, K, swiglu, compute_units(), true));
}

hipError_t launch_gemm_ws(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y, int64_t ldy,
                          int M, int N, int K, bool swiglu, void* ws, size_t ws_bytes, hipStream_t stream) {
    if (skinny(M, N, swiglu)) return launch_skinny(x, w, scales, S, y, ldy, M, N, K, swiglu, stream);
    const bool fp8 = scales != nullptr;
    if (fp8 && mid_rows(x, w, S, M, N, K))
        return launch_small_m(x, static_cast<const uint8_t*>(w), scales, y, ldy, M, N, K, 1, swiglu, stream);
    if (fp8 && fp8_kernel_ok(x, w, S, ldy, M, N, K)) {
        const uint8_t* codes = static_cast<const uint8_t*>(w);
        const int G = compute_units();
        gemm_fp8::Plan plan = make_plan(M, N, K, swiglu, G, ws != nullptr);
        if (plan_bytes(plan) > ws_bytes || reinterpret_cast<uintptr_t>(ws) % 16 != 0)
            plan = make_plan(M, N, K, swiglu, G, false);
        if (plan.rtiles == 0 && halves(x, w, S, M, N, K))
            return launch_halves(x, codes, scales, y, ldy, M, N, K, swiglu, stream);
        float* part = static_cast<float*>(ws);
        return swiglu ? run_fp8<true>(x, codes, scales, S, y, ldy, M, N, K, plan, G, part, stream)
                      : run_fp8<false>(x, codes, scales, S, y, ldy, M, N, K, plan, G, part, stream);
    }
    return launch_gemm(x, w, scales, S, y, ldy, M, N, K, swiglu, stream);
}

hipError_t launch_gemm(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y,
                       int64_t ldy, int M, int N, int K, bool swiglu, hipStream_t stream) {
    if (skinny(M, N, swiglu)) return launch_skinny(x, w, scales, S, y, ldy, M, N, K, swiglu, stream);
    const bool fp8 = scales != nullptr;
    if (fp8 && mid_rows(x, w, S, M, N, K))
        return launch_small_m(x, static_cast<const uint8_t*>(w), scales, y, ldy, M, N, K, 1, swiglu, stream);
    if (fp8 && halves(x, w, S, M, N, K))
        return launch_halves(x, static_cast<const uint8_t*>(w), scales, y, ldy, M, N, K, swiglu, stream);
    if (fp8 && fp8_kernel_ok(x, w, S, ldy, M, N, K)) {
        const uint8_t* codes = static_cast<const uint8_t*>(w);
        const int G = compute_units();
        const gemm_fp8::Plan plan = make_plan(M, N, K, swiglu, G, false);
        return swiglu ? run_fp8<true>(x, codes, scales, S, y, ldy, M, N, K, plan, G, nullptr, stream)
                      : run_fp8<false>(x, codes, scales, S, y, ldy, M, N, K, plan, G, nullptr, stream);
    }
    if (fp8)
        return swiglu ? run<true, true>(x, w, scales, S, y, ldy, M, N, K, stream)
                      : run<true, false>(x, w, scales, S, y, ldy, M, N, K, stream);
    return swiglu ? run<false, true>(x, w, nullptr, 1, y, ldy, M, N, K, stream)
                  : run<false, false>(x, w, nullptr, 1, y, ldy, M, N, K, stream);
}

}  // namespace fp8lin
