// Host-side launchers shared between the kernel files and the C ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fp8lin {

// Decode GEMV, 1 <= M <= 8 (gemv.hip).  `w` is E4M3FN codes when fp8, else
// BF16.  `wide` selects 128-bit loads (caller checked alignment and K % 16).
hipError_t launch_gemv_pair(const uint16_t* x, const uint8_t* codes, const float* scales, int S, uint16_t* ya,
                            int na, const uint16_t* wb, uint16_t* yb, int nb, int64_t ldy, int K,
                            hipStream_t stream);
hipError_t launch_gemv(const uint16_t* x, const void* w, bool fp8, const float* scales, int S,
                       uint16_t* y, int64_t ldy, int M, int N, int K, bool wide,
                       hipStream_t stream);
// Decode GEMV with the SwiGLU epilogue: N weight rows (gate [0,N/2), up
// [N/2,N)), y is [M, N/2].
hipError_t launch_gemv_swiglu(const uint16_t* x, const uint8_t* codes, const float* scales, int S,
                              uint16_t* y, int64_t ldy, int M, int N, int K, bool wide,
                              hipStream_t stream);

// Any number of activation rows against a few weight rows (gemv.hip): the
// GEMV over blocks of 8 activation rows, four waves splitting K (the prefill
// form for N <= kSkinnyRows, where 256x256 MFMA tiles leave most CUs idle).
constexpr int kSkinnyRows = 256;
// MFMA form for few weight rows (skinny.hip): 16 x 16 output tiles, K split
// over 4 waves; the requirements in skinny_mfma_supported.
bool skinny_mfma_supported(const uint16_t* x, const void* w, bool fp8, int S, int64_t M, int64_t N, int64_t K);
hipError_t launch_skinny_mfma(const uint16_t* x, const void* w, bool fp8, const float* scales, int S, uint16_t* y,
                              int64_t ldy, int M, int N, int K, bool swiglu, hipStream_t stream);
hipError_t launch_gemv_rows(const uint16_t* x, const void* w, bool fp8, const float* scales, int S, uint16_t* y,
                            int64_t ldy, int M, int N, int K, bool wide, bool swiglu, hipStream_t stream);

// Compute units of the current device, rounded down to a multiple of the 8
// XCDs (cached per device): the grid of the persistent kernels (gemm.hip).
int compute_units();

// Small-M matrix-core kernel, 2 <= M <= 32 (17..32: two 16-row MFMA tiles,
// in the row-range form where small_m_candidates_supported), K % 128 == 0, block scales
// (small_m.hip).  The K partition is the kernel's own, so split 1 and 4 give
// the same bits; no workspace.  M * K * 2 and 16 * K must be below 2^31.
// swiglu: N weight rows (gate [0, N/2), up [N/2, N)), y is [M, N/2], bit-equal
// to fused_swiglu of the plain form's output; also needs N * K / 32 < 2^31.
hipError_t launch_small_m(const uint16_t* x, const uint8_t* codes, const float* scales,
                          uint16_t* y, int64_t ldy, int M, int N, int K, int split, bool swiglu,
                          hipStream_t stream);
// The output head's candidates where launch_small_m (plain form) runs its
// row-range kernel (small_m_candidates_supported): the same logits, reduced
// per workgroup and activation row to one {value bits, column} pair, part
// [M][groups] pairs (groups <= CUs), for launch_candidates_finish.  No logits
// written.
// Supported: K / 128 in 25..40 with at least 32 weight rows per CU for M <=
// 16 (24 for 17..32 rows), or K / 128 in 65..72 with 32 rows per CU for M <= 16.
bool small_m_candidates_supported(int M, int N, int K);
// Whether fp8lin_linear runs the small-M kernel at two rows and K <= 5120
// (where it measured faster than the two-row ring GEMV for this weight).
bool small_m_two_rows(int N, int K);
// Whether the row-staged small-M form runs M rows against an N x K weight.
bool small_m_wide_rows(int M, int N, int K);
hipError_t launch_small_m_candidates(const uint16_t* x, const uint8_t* codes, const float* scales, int M, int N,
                                     int K, uint32_t* part, int64_t& groups, hipStream_t stream);
// out[2m] = value, out[2m + 1] = column + offset of the best of the `chunks`
// pairs of row m in part [M][chunks] (epilogue.hip; one workgroup per row).
hipError_t launch_candidates_finish(const uint32_t* part, int M, int64_t chunks, int64_t offset, double* out,
                                    hipStream_t stream);

// MFMA GEMM (gemm.hip).  B is E4M3FN codes (scales != nullptr, dequantized
// to BF16 in LDS) or BF16 (scales == nullptr).  When swiglu, N is the number
// of weight rows (gate rows [0,N/2), up rows [N/2,N)) and y is [M, N/2].
hipError_t launch_gemm(const uint16_t* x, const void* w, const float* scales, int S,
                       uint16_t* y, int64_t ldy, int M, int N, int K, bool swiglu,
                       hipStream_t stream);
// The FP8 GEMM with a workspace for K-split partials: where the tile count
// leaves CUs idle (few tiles, or a small last round) K is split and a second
// launch adds the FP32 partials.  gemm_workspace_bytes() is what that needs
// (0 when nothing splits); a smaller or unaligned workspace, unaligned x or
// w, or another kernel's shape run unsplit.
size_t gemm_workspace_bytes(int S, int64_t ldy, int M, int N, int K, bool swiglu);
// Whether the GEMM dispatch sends this FP8 call (9..32 rows) to the small-M
// matrix-core kernel instead of a GEMM tile.
bool gemm_mid_rows(const uint16_t* x, const void* w, int S, int64_t M, int64_t N, int64_t K);
hipError_t launch_gemm_ws(const uint16_t* x, const void* w, const float* scales, int S, uint16_t* y, int64_t ldy,
                          int M, int N, int K, bool swiglu, void* ws, size_t ws_bytes, hipStream_t stream);

// Elementwise kernels (elementwise.hip).
hipError_t launch_dequant(const uint8_t* codes, const float* scales, int64_t S, uint16_t* y,
                          int64_t ldy, int64_t rows, int64_t cols, hipStream_t stream);
hipError_t launch_swiglu(const uint16_t* in, uint16_t* y, int64_t M, int64_t D,
                         hipStream_t stream);
// y[r, c] = bf16(y[r, c] + bias[c]) for r < rows, c < cols (row stride ldy).
hipError_t launch_bias(uint16_t* y, int64_t ldy, const uint16_t* bias, int64_t rows, int64_t cols,
                       hipStream_t stream);
hipError_t launch_gen_weights(uint64_t seed, uint32_t tag, int64_t N, int64_t K, float std_dev,
                              uint8_t* codes, float* scales, hipStream_t stream);
hipError_t launch_gen_activations(uint64_t seed, uint32_t tag, int64_t M, int64_t K,
                                  uint16_t* x, hipStream_t stream);
hipError_t launch_gen_normal(uint64_t seed, uint32_t tag, uint64_t first, int64_t n,
                             float* out, hipStream_t stream);
hipError_t launch_stream_read(const void* src, size_t bytes, float* sink, hipStream_t stream);

// Decode epilogue and output head (epilogue.hip).  launch_rms: RMSNorm of x
// (update == nullptr) or of residual = bf16(x + update), also stored.
hipError_t launch_rms(const uint16_t* x, const uint16_t* update, const uint16_t* w, uint16_t* residual,
                      uint16_t* y, int64_t M, int D, float eps, bool centered, hipStream_t stream);
// Row-parallel reduce folded into the residual add: update = bf16(sum over
// `ranks` partials [ranks][M][D] in order), then as launch_rms.
hipError_t launch_reduce_rms(const uint16_t* x, const uint16_t* partials, int ranks, const uint16_t* w,
                             uint16_t* residual, uint16_t* y, int64_t M, int D, float eps, bool centered,
                             hipStream_t stream);
// Candidates of logits [M, N] -> out [M, 2] doubles {value, id + offset};
// part: M * vocab_chunks(N) {float bits, id} pairs.
int64_t vocab_chunks(int64_t N);
// Per row m, the best pair of the `chunks` workgroups of the GEMV candidate
// kernel (8 XCD runs of ceil(chunks / 8) slots per row) as out[2m] = value,
// out[2m + 1] = column + offset (epilogue.hip): kCandSlices workgroups per row
// each reduce a slice into slices[(m * kCandSlices + s) * 2], and the last to
// arrive (per-row counters[m], zero at launch) reduces the slices.
constexpr int kCandSlices = 16;
hipError_t launch_candidates_finish_sliced(const uint32_t* part, int M, int64_t chunks, uint32_t* slices,
                                           uint32_t* counters, int64_t offset, double* out, hipStream_t stream);
// The output head's GEMV with the candidate epilogue (gemv.hip): for the calls
// where fp8lin_linear runs the ring kernel (gemv_candidates_supported), the
// candidates of its logits without writing them, in a workspace of
// gemv_candidates_ws_bytes(M, N) (16-byte aligned; no cleared bytes needed).
bool gemv_candidates_supported(int M, int N, int K, bool wide);
size_t gemv_candidates_ws_bytes(int M, int N);
hipError_t launch_gemv_candidates(const uint16_t* x, const uint8_t* codes, const float* scales, int S, int M,
                                  int N, int K, int64_t offset, void* ws, double* out, hipStream_t stream);
hipError_t launch_vocab_candidates(const uint16_t* logits, int M, int N, int64_t offset, uint32_t* part,
                                   double* out, hipStream_t stream);
hipError_t launch_merge_candidates(const double* gathered, int ranks, int64_t rows, int64_t* out,
                                   hipStream_t stream);

// Multi-axis rotary embedding of x [T, H, D] (D <= kRopeMaxD), and the fused
// per-head RMSNorm + rotary embedding of the QKV-gate output (D <= 512).
constexpr int kRopeMaxD = 4096;
hipError_t launch_rope(const uint16_t* x, const int64_t* pos, uint16_t* y, int T, int H, int D, int R, float theta,
                       int hs, int ws, hipStream_t stream);
hipError_t launch_qk_norm_rope(const uint16_t* p, int64_t ld, const uint16_t* qw, const uint16_t* kw,
                               const int64_t* pos, uint16_t* q, uint16_t* k, int T, int H, int HK, int D, int R,
                               float theta, int hs, int ws, float eps, bool centered, hipStream_t stream);

hipError_t launch_mfma_ceiling(int64_t iters, float* sink, uint64_t* clocks, hipStream_t stream);

// Decode chain (chain.hip): one-row linear links in one launch; link L waits
// for link `after` (or nothing when after < 0) before it reads x.  sync:
// chain_sync_words(nlinks) 64-bit words, zero before the first call of a
// chain shape: word 0 counts waits that gave up, word 1 the chain's shape,
// then per-link slot counters and per-XCD call words (chain.hip).
constexpr int kChainMaxLinks = 8;  // FP8LIN_CHAIN_MAX_LINKS
struct ChainLink {
    const uint8_t* codes;
    const float* scales;
    int64_t S, N, K;
    const uint16_t* x;
    uint16_t* y;
    bool swiglu;
    int after;
};
bool chain_link_supported(int64_t N, int64_t K, int64_t S, bool swiglu);
size_t chain_sync_words(int nlinks);
hipError_t launch_chain(const ChainLink* links, int nlinks, uint64_t* sync, hipStream_t stream);

}  // namespace fp8lin
