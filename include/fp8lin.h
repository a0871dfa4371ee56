/*
 * fp8lin -- MI355X (gfx950) block-FP8 linear layers, C ABI.
 *
 * E4M3FN weight codes [N,K] (uint8, row-major) with FP32 scales, times BF16
 * activations [M,K] (row-major), FP32 accumulation, BF16 output [M,N].
 * Scales are either per row ([N], scale_cols == 1) or 128x128 block scales
 * expanded along rows ([N, ceil(K/128)], scale_cols == ceil(K/128)); the
 * weight used for element (n,k) is bf16(decode(code[n,k]) * scale[n, k/128]).
 *
 * Conventions for every entry point:
 *  - all tensors are device pointers owned by the caller; the library never
 *    allocates or frees them and never synchronises the stream;
 *  - BF16 data is passed as uint16_t bit patterns;
 *  - `stream` is a hipStream_t (NULL = the null stream); work is enqueued
 *    on it and is capturable into a HIP graph;
 *  - a workspace (16-byte aligned device memory of at least the size the
 *    matching *_workspace_bytes function reports) belongs to the call's
 *    launches until they complete on `stream`: calls that may run at the same
 *    time (other streams) need their own workspaces;
 *  - the return value is FP8LIN_OK or one of the FP8LIN_ERR_* codes below;
 *    fp8lin_last_error() gives a message for the calling thread's last
 *    failure.  No C++ exception crosses this boundary.
 *
 * Each declaration names the reference (laoyin/a100-vision-infer) interface it
 * replaces.  The reference takes at::Tensor arguments, allocates its outputs
 * and reports errors with TORCH_CHECK; here the same checks become status
 * codes and the caller passes the output buffer.
 */
#ifndef FP8LIN_H
#define FP8LIN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2.0.0: fp8lin_weight gained its `bias` member (a record built against a
 * 1.x header has another size and stride) and fp8lin_linear_ws was added. */
#define FP8LIN_VERSION 200 /* 2.0.0 */

enum fp8lin_status {
    FP8LIN_OK = 0,
    FP8LIN_ERR_SHAPE = 1,       /* invalid or inconsistent dimensions */
    FP8LIN_ERR_ARGUMENT = 2,    /* null pointer, bad scale layout, bad flag value */
    FP8LIN_ERR_UNSUPPORTED = 3, /* valid request outside this entry point's contract */
    FP8LIN_ERR_WORKSPACE = 4,   /* workspace missing or smaller than required */
    FP8LIN_ERR_LAUNCH = 5,      /* HIP runtime or kernel launch failure */
    FP8LIN_ERR_DEVICE = 6       /* the current device is not a gfx950 GPU */
};

typedef void* fp8lin_stream_t; /* hipStream_t */

int fp8lin_version(void);
/* Message for the calling thread's most recent failure ("" if none). */
const char* fp8lin_last_error(void);
/* Checks that the current device is gfx950 and, once per device, queries
 * its properties and looks up the device address of the library's static
 * scratch.  Every entry point does the same on its first call on a device,
 * but those runtime queries must not run inside a HIP stream capture: call
 * fp8lin_init() with each device current before the first capture that
 * records fp8lin calls on it (the Python host mirror does so for every
 * device it is handed).  Idempotent and thread-safe.  TileLang plugin
 * precedent: init()/get_last_error() of src/tilelang.cpp:80-82. */
int fp8lin_init(void);

/* ---------------------------------------------------------------------------
 * Dequantization: y[r,c] = bf16(decode(codes[r,c]) * scales[r, c/128]).
 * Replaces `Tensor fp8_decode(Tensor codes, Tensor scales)`
 * (include/avi/engine.h:13, src/kernels.cu:17-27).  rows == 0 or cols == 0
 * is a no-op, as in the reference.
 */
int fp8lin_decode(const uint8_t* codes, const float* scales, int64_t scale_cols,
                  uint16_t* y, int64_t rows, int64_t cols, fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * y[M,N] = x[M,K] * W^T.  Replaces
 * `at::Tensor fp8_linear(at::Tensor x, at::Tensor codes, at::Tensor scales,
 *                        bool vector_gemv=false)`
 * (include/avi/ops.h:18, src/optimized.cu:61-70).  M <= 8 runs the decode
 * GEMV (128-bit loads when K, x and codes are 16-byte aligned, otherwise
 * byte loads with bit-identical results; vector_gemv changes nothing), except
 * that 3..8 rows (2 rows at K > 5120; at K <= 5120 on weights of its
 * row-range form: more than 80 rows per compute unit at K = 4224..5120, more
 * than 40 at K = 3200..4096, as the output heads; or 25..40 rows per compute
 * unit on its row-staged form) against more than 1024 weight rows with
 * block scales, K % 128 == 0 and 16-byte aligned x and codes run the small-M
 * matrix-core kernel of fp8lin_tensor_small (one pass over the weights for
 * all rows; same parity bar, another FP32 summation order, so such a call and
 * an unaligned view of the same data may differ in the last bit, which the
 * reference allows: it checks bit-equality only on one-row views,
 * tests/optimized_test.cpp:57-62); M > 8 runs the MFMA GEMM that dequantizes
 * FP8 tiles to BF16 (128-row tiles for M <= 128, 256-row tiles above), except
 * that 9..16 rows under the same conditions as the 3..8-row case run the
 * small-M matrix-core kernel too (its 16-row MFMA tile holds them all),
 * 17..32 rows (two such tiles), and 33..64 rows on weights of at most 32
 * rows per compute unit (four such tiles; no split-K workspace needed);
 * 65..128 rows on such weights run as two row halves of those kernels (each
 * half the bits of a call of its own rows) instead of whole GEMM tiles.
 * Requires M, N, K > 0 and scale_cols in {1, ceil(K/128)}.
 */
int fp8lin_linear(const uint16_t* x, const uint8_t* codes, const float* scales,
                  int64_t scale_cols, uint16_t* y, int64_t M, int64_t N, int64_t K,
                  int vector_gemv, fp8lin_stream_t stream);

/* Same as fp8lin_linear with an output row stride ldy >= N (elements), so a
 * caller can write into a column slice of a wider output (the mixed-group
 * concatenation of src/engine.cpp:199 without a copy). */
int fp8lin_linear_ld(const uint16_t* x, const uint8_t* codes, const float* scales,
                     int64_t scale_cols, uint16_t* y, int64_t ldy, int64_t M, int64_t N,
                     int64_t K, int vector_gemv, fp8lin_stream_t stream);

/* fp8lin_linear with a workspace for the prefill GEMM's K-split partials:
 * when M > 8 and the GEMM's 256x256 (128-row for M <= 128) tiles number
 * fewer than half the CUs (e.g. the 7168-row QKV-gate and 5120-row down
 * projections at M = 512, or the 5120-row down projection at M = 65..128),
 * or leave a last round on at most half of them, those tiles are cut into
 * K ranges and a second launch adds their FP32 sums in order and rounds
 * once.  Within the parity bar of fp8lin_linear (only the FP32 summation
 * order of the split tiles differs); every other call is fp8lin_linear bit
 * for bit.  The workspace is what fp8lin_linear_workspace_bytes reports for
 * (M, N, K) (0: none needed; 256 KiB per split tile and K range), 16-byte
 * aligned, any content.  Replaces the same `fp8_linear` as fp8lin_linear;
 * the reference allocates such partials inside its own operator
 * (src/fp8_tensor.cu:65), here the caller passes them.
 */
size_t fp8lin_linear_workspace_bytes(int64_t M, int64_t N, int64_t K);
int fp8lin_linear_ws(const uint16_t* x, const uint8_t* codes, const float* scales, int64_t scale_cols,
                     uint16_t* y, int64_t M, int64_t N, int64_t K, int vector_gemv, void* workspace,
                     size_t workspace_bytes, fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * Fused gate/up projection + SwiGLU: with G = fp8lin_linear(x, W) of shape
 * [M, N] (N even, rows [0, N/2) = gate, [N/2, N) = up, the row concatenation
 * of src/engine.cpp:116,167), y[M, N/2] = fused_swiglu(G) bit for bit: the
 * kernel fp8lin_linear picks for the same arguments runs with a SwiGLU
 * epilogue.  Replaces the pair linear(gate_up) -> fused_swiglu at
 * src/engine.cpp:415.
 */
int fp8lin_linear_swiglu(const uint16_t* x, const uint8_t* codes, const float* scales,
                         int64_t scale_cols, uint16_t* y, int64_t M, int64_t N, int64_t K,
                         fp8lin_stream_t stream);

/* The same with a workspace, which lets the prefill GEMM (M > 8) split K
 * where whole tiles would leave CUs idle: when the 256x256 tiles number
 * fewer than half the CUs, or leave a last round on at most a quarter of
 * them (M = 1024 and M = 4096 at N = 17408, K = 5120), those tiles are cut
 * into K ranges whose FP32 sums a second launch adds in order before the
 * SwiGLU rounding points.  Within the parity bar of the unsplit call (only
 * the FP32 summation order of the split tiles differs).  The workspace is
 * what fp8lin_linear_swiglu_workspace_bytes reports (0: none needed), 16-byte
 * aligned.  Same replacement as fp8lin_linear_swiglu.
 */
size_t fp8lin_linear_swiglu_workspace_bytes(int64_t M, int64_t N, int64_t K);
int fp8lin_linear_swiglu_ws(const uint16_t* x, const uint8_t* codes, const float* scales, int64_t scale_cols,
                            uint16_t* y, int64_t M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                            fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * Bias add in place: y[r,c] = bf16(y[r,c] + bias[c]) for r < rows, c < N, y
 * with row stride ldy >= N; the BF16 `y + b` of Engine::linear
 * (src/engine.cpp:240), for callers that reduce an output across ranks before
 * adding its bias.  rows == 0 or N == 0 is a no-op.
 */
int fp8lin_add_bias(uint16_t* y, int64_t ldy, const uint16_t* bias, int64_t rows, int64_t N,
                    fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * SwiGLU: y[r,j] = bf16(bf16(a/(1+exp(-a))) * u), a = in[r,j], u = in[r,D+j],
 * in is [M, 2D].  Replaces `at::Tensor fused_swiglu(at::Tensor gate_up)`
 * (include/avi/ops.h:20, src/optimized.cu:73-74).
 */
int fp8lin_swiglu(const uint16_t* gate_up, uint16_t* y, int64_t M, int64_t D,
                  fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * Shared-weight multi-row GEMV, 1 <= M <= 8: every row of x is multiplied
 * against one pass over the weights.  `scales == NULL` means `weight` is BF16
 * [N,K] (a decoded-weight cache); otherwise it is E4M3FN codes.  The FP8 and
 * the BF16-decoded forms give bit-identical outputs.  Replaces
 * `at::Tensor small_linear_shared(at::Tensor x, at::Tensor weight,
 *                                 at::Tensor scales={})`
 * (include/avi/ops.h:11, src/deep_kernels.cu:134-157).
 */
int fp8lin_linear_shared(const uint16_t* x, const void* weight, const float* scales,
                         int64_t scale_cols, uint16_t* y, int64_t M, int64_t N, int64_t K,
                         fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * Small-M matrix-core path, 2 <= M <= 8, K % 128 == 0, block scales
 * [N, K/128], split in {1, 4}.  The K partition is the kernel's own, so
 * split 1 and split 4 give the same bits and no workspace is needed: the
 * workspace size is 0 and the workspace arguments are accepted and ignored.
 * Like the reference, any contiguous x and codes are accepted: when either
 * is not 16-byte aligned (a view at an odd offset) or 16*K >= 2^31, the call
 * runs the multi-row decode GEMV instead (same parity bar).  Replaces
 * `at::Tensor fp8_tensor_small(at::Tensor x, at::Tensor codes,
 *                              at::Tensor scales, int split=1)`
 * (include/avi/ops.h:10, src/fp8_tensor.cu:53-71); the same contract serves
 * `tilelang_fp8_small` (include/avi/tilelang.h:11, src/tilelang.cpp:94-107).
 */
size_t fp8lin_tensor_small_workspace_bytes(int64_t M, int64_t N, int split);
int fp8lin_tensor_small(const uint16_t* x, const uint8_t* codes, const float* scales,
                        uint16_t* y, int64_t M, int64_t N, int64_t K, int split,
                        void* workspace, size_t workspace_bytes, fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * BF16 GEMM y[M,N] = x[M,K] * W^T with BF16 weights W [N,K] (the decoded-weight
 * cache and unquantized weights, `at::matmul(x, w.t())` at
 * src/engine.cpp:221,236).  MFMA kernel, FP32 accumulation, BF16 output.
 */
int fp8lin_gemm_bf16(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t ldy,
                     int64_t M, int64_t N, int64_t K, fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * Engine::linear dispatch (src/engine.cpp:196-242) over one weight, with the
 * EngineOptions linear-path flags (include/avi/engine.h:16).  The decision
 * order is the reference's: tensor-small (rows 2..8, K%128==0, block scales;
 * tilelang_fp8 additionally N%16==0) -> multi-token shared GEMV (rows 2..8)
 * -> cached BF16 GEMM (rows > 1) -> fp8_linear (optimized, unless
 * cublas_prefill and rows > 8) -> dequant-then-GEMM in 2048-row slabs
 * (src/engine.cpp:225-233) -> BF16 GEMM for unquantized weights.  Then, when
 * the weight has a bias, y = bf16(y + bias) (src/engine.cpp:240).
 * The tensor-parallel reduce that the reference runs between the product and
 * the bias (src/engine.cpp:239) is the caller's: for a weight whose output is
 * reduced across ranks, pass bias = NULL here and call fp8lin_add_bias after
 * the reduce.  Options that the reference's Engine constructor rejects
 * (fp8_tensor_small together with tilelang_fp8, either of them without
 * optimized, a split other than 1 or 4; src/engine.cpp:78-81) make every
 * engine entry point return FP8LIN_ERR_ARGUMENT (and the *_workspace_bytes
 * and *_path queries 0).
 * Records must be zero-initialised before their fields are set (C:
 * `fp8lin_weight w = {0};`, C++: `fp8lin_weight w{};`), so that a member a
 * caller does not know about, such as `bias` (added in 2.0.0), is NULL.
 */
typedef struct fp8lin_weight {
    const void* data;            /* uint8 codes [N,K], or BF16 [N,K] if scales == NULL */
    const float* scales;         /* [N] or [N, ceil(K/128)]; NULL for BF16 weights */
    int64_t scale_cols;          /* 1 or ceil(K/128); ignored for BF16 weights */
    const uint16_t* cached_bf16; /* optional decoded copy [N,K] (bounded cache) or NULL */
    int64_t N, K;
    const uint16_t* bias;        /* optional BF16 [N] (`name.bias`), or NULL */
} fp8lin_weight;

typedef struct fp8lin_linear_options {
    int optimized;        /* EngineOptions::optimized (false with --baseline) */
    int vector_gemv;      /* --vector-gemv */
    int cublas_prefill;   /* dequant-then-GEMM for rows > 8 */
    int fp8_tensor_small; /* small-M matrix-core path */
    int fp8_tensor_split; /* 1 or 4 */
    int tilelang_fp8;     /* same contract as fp8_tensor_small, N % 16 == 0 */
    int multi_token_gemv; /* shared-weight GEMV for rows 2..8 */
    int shared_gemv_fp8;  /* shared GEMV reads FP8 codes even if a cache exists */
} fp8lin_linear_options;

/* Workspace needed by fp8lin_engine_linear for this weight and row count;
 * 0 if none.  The FP8 GEMM branch (rows > 8) splits K where its 256x256
 * tiles would leave CUs idle (as fp8lin_linear_swiglu_ws does) and then needs
 * 256 KiB of FP32 partials per split tile and K range; the dequant-then-GEMM
 * branch needs a 2048-row BF16 slab. */
size_t fp8lin_engine_linear_workspace_bytes(const fp8lin_linear_options* options,
                                            const fp8lin_weight* weight, int64_t rows);
/* Id of the branch fp8lin_engine_linear takes for this weight, options and
 * row count (FP8LIN_PATH_*), without launching anything; 0 on bad arguments. */
int fp8lin_engine_linear_path(const fp8lin_linear_options* options, const fp8lin_weight* weight,
                              int64_t rows);
/* y has row stride ldy >= weight->N.  Writes the id of the path it took to
 * *path_out when path_out != NULL (FP8LIN_PATH_*). */
int fp8lin_engine_linear(const fp8lin_linear_options* options, const fp8lin_weight* weight,
                         const uint16_t* x, int64_t rows, uint16_t* y, int64_t ldy,
                         void* workspace, size_t workspace_bytes, int* path_out,
                         fp8lin_stream_t stream);
/* Mixed projection groups (src/engine.cpp:198-199, fuse_weights :147-177):
 * each group's output is written to consecutive column slices of y, in
 * order, exactly like at::cat(parts, -1).  Two groups at one row that both
 * take the decode GEMV (an FP8 weight of 1025..16383 rows, then a BF16 weight
 * of at most 1024, K <= 5120, no bias: the GDN in_proj_all group) run in one
 * launch, with the bits of the two groups' own calls. */
int fp8lin_engine_linear_groups(const fp8lin_linear_options* options,
                                const fp8lin_weight* groups, int ngroups,
                                const uint16_t* x, int64_t rows, uint16_t* y, int64_t ldy,
                                void* workspace, size_t workspace_bytes,
                                fp8lin_stream_t stream);

enum fp8lin_path {
    FP8LIN_PATH_TENSOR_SMALL = 1,
    FP8LIN_PATH_SHARED_GEMV = 2,
    FP8LIN_PATH_CACHED_BF16 = 3,
    FP8LIN_PATH_FP8_GEMV = 4,
    FP8LIN_PATH_FP8_GEMM = 5,
    FP8LIN_PATH_DEQUANT_GEMM = 6,
    FP8LIN_PATH_BF16 = 7
};

/* ---------------------------------------------------------------------------
 * Decode epilogue: RMSNorm over the last dimension of x [rows, D] (BF16):
 *   inv = rsqrt(sum_i x_i^2 / D + eps)
 *   centered:  y_i = bf16(x_i * inv * (w_i + 1))
 *   otherwise: y_i = bf16(bf16(x_i * inv) * w_i)
 * with the sum in FP32.  Replaces
 * `at::Tensor fused_rms(at::Tensor x, at::Tensor weight, double eps, bool one_center)`
 * (include/avi/ops.h:19, src/optimized.cu:71-72).  rows == 0 is a no-op;
 * eps is used as given (the reference checks it only in the residual form).
 */
int fp8lin_rms(const uint16_t* x, const uint16_t* weight, uint16_t* y, int64_t rows, int64_t D,
               double eps, int centered, fp8lin_stream_t stream);

/* Fused residual add + RMSNorm: residual = bf16(x + update), y = RMSNorm of
 * residual as in fp8lin_rms.  Bit-identical to fp8lin_residual_rms's residual
 * fed to fp8lin_rms.  Replaces
 * `std::pair<at::Tensor, at::Tensor> residual_rms(at::Tensor residual,
 *     at::Tensor update, at::Tensor weight, double eps, bool centered=true)`
 * (include/avi/ops.h:6, src/dual_path.cu:68-78); the pair is (residual, y).
 * Requires rows > 0, 0 < D < 2^31, eps finite and > 0; the outputs must not
 * overlap the inputs.
 */
int fp8lin_residual_rms(const uint16_t* x, const uint16_t* update, const uint16_t* weight,
                        uint16_t* residual, uint16_t* y, int64_t rows, int64_t D, double eps,
                        int centered, fp8lin_stream_t stream);

/* The row-parallel reduce folded into the residual add (no single reference
 * counterpart; it fuses Engine::sum's BF16 reduce, src/engine.cpp:183-195,
 * with residual_rms, src/dual_path.cu:68-78): partials [ranks][rows][D] are
 * the per-rank outputs of a row-parallel projection, gathered on this GPU;
 * update = bf16(sum over ranks in rank order, in FP32), then residual =
 * bf16(x + update) and y = RMSNorm(residual) as fp8lin_residual_rms.  For
 * ranks <= 2 the update equals the reference's BF16 all-reduce
 * (tests/tp_reduce_test.cpp:25-32).  Requires 1 <= ranks <= 8 and the
 * requirements of fp8lin_residual_rms.
 */
int fp8lin_reduce_residual_rms(const uint16_t* x, const uint16_t* partials, int64_t ranks,
                               const uint16_t* weight, uint16_t* residual, uint16_t* y, int64_t rows,
                               int64_t D, double eps, int centered, fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * Multi-axis rotary embedding (interleaved mRoPE) of x [T, H, D] (BF16) at
 * positions [3, T] (int64: temporal, height, width), into y [T, H, D].  For
 * d < rotary, pair index f = d mod rotary/2 reads axis 1 when f mod 3 == 1
 * and f < 3*height_section, axis 2 when f mod 3 == 2 and f < 3*width_section,
 * else axis 0;
 *   angle = float(pos) * powf(float(theta), -2f*f/rotary)      (FP32;
 *           the power correctly rounded to FP32 but at near-halfway values)
 *   co = bf16(cos(angle)), si = bf16(sin(angle))
 *   y[d] = bf16(bf16(x[d]*co) - bf16(x[d+rotary/2]*si))  d < rotary/2
 *   y[d] = bf16(bf16(x[d]*co) + bf16(x[d-rotary/2]*si))  rotary/2 <= d < rotary
 * and y[d] = x[d] for d >= rotary.  Requires rotary even, 0 < rotary <= D,
 * D <= 4096; T == 0 is a no-op.  Replaces `at::Tensor fused_rope(at::Tensor x,
 * at::Tensor positions, int rotary, double theta, int height_section,
 * int width_section)` (include/avi/ops.h:25, src/optimized.cu:77-78).
 */
int fp8lin_rope(const uint16_t* x, const int64_t* positions, uint16_t* y, int64_t T, int64_t H, int64_t D,
                int64_t rotary, double theta, int64_t height_section, int64_t width_section,
                fp8lin_stream_t stream);

/* Q/K epilogue of the QKV-gate projection, read in place from projected
 * [T, ld] (ld >= H*2D + 2*HK*D elements; per token H heads of query then gate,
 * D each, then HK key heads and HK value heads): q [T, H, D] =
 * rope(rms(query), q_norm) and k [T, HK, D] = rope(rms(key), k_norm), with
 * the centered RMSNorm of fp8lin_rms and fp8lin_rope's rotation.  Bit-identical
 * to fp8lin_rms of the contiguous query (key) rows followed by fp8lin_rope.
 * The gate and value heads stay views of projected.  Requires H > 0, HK > 0,
 * D <= 512; eps is used as given, as by fp8lin_rms.
 * Replaces the optimized branch of src/engine.cpp:279-287 (norm(q_norm),
 * norm(k_norm), fused_rope(q), fused_rope(k)).
 */
int fp8lin_qk_norm_rope(const uint16_t* projected, int64_t ld, const uint16_t* q_norm, const uint16_t* k_norm,
                        const int64_t* positions, uint16_t* q, uint16_t* k, int64_t T, int64_t H, int64_t HK,
                        int64_t D, int64_t rotary, double theta, int64_t height_section, int64_t width_section,
                        double eps, fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * Output head.  Per row of BF16 logits [M, N], the largest value (NaN counts
 * as +inf so that a NaN row is rejected by the merge, ties go to the smaller
 * column) as out[m] = {value, column + offset} in doubles.  Replaces
 * `at::Tensor vocabulary_candidates(at::Tensor logits, int64_t offset=0)`
 * (include/avi/ops.h:7, src/dual_path.cu:79-85).  Requires 0 < M <= 65535,
 * N > 0, 0 <= offset <= INT32_MAX - N; workspace: the bytes below (one
 * {value, column} pair per 2048 columns and row, 16-byte aligned).
 */
size_t fp8lin_vocab_candidates_workspace_bytes(int64_t M, int64_t N);
int fp8lin_vocab_candidates(const uint16_t* logits, int64_t M, int64_t N, int64_t offset,
                            double* out, void* workspace, size_t workspace_bytes,
                            fp8lin_stream_t stream);

/* Token ids from gathered candidates [ranks, rows, 2] (doubles): per row the
 * best {value, id} over ranks (ties to the smaller id), or -1 if any rank's
 * value or id is non-finite or the id is not an integer in [0, INT32_MAX].
 * Replaces `at::Tensor merge_candidates(at::Tensor gathered)`
 * (include/avi/ops.h:8, src/dual_path.cu:86-92).  Requires 0 < ranks <= 8
 * and 0 < rows <= 65535.
 */
int fp8lin_merge_candidates(const double* gathered, int64_t ranks, int64_t rows, int64_t* out,
                            fp8lin_stream_t stream);

/* The head projection and its candidates in one call: out equals
 * fp8lin_vocab_candidates(fp8lin_linear(x, W), offset), the pair of
 * src/speculative.cpp:25-27 (Engine::local_candidates with gpu_candidates).
 * Where fp8lin_linear runs its ring GEMV (M <= 2, 16-byte aligned x and
 * codes, K % 16 == 0 and K <= 9216, K <= 5120 at M = 2) the GEMV's epilogue
 * emits one {max, column} pair per workgroup and no logits are written
 * (src/dual_path.cu:37-55 fused into the projection); where it runs the
 * small-M matrix-core kernel's row-range form (3..32 rows, or 2 at
 * K > 5120, against at least 32 weight rows per compute unit; 17..32 rows
 * at K <= 5120) that kernel does the same, one pair per workgroup and row;
 * otherwise the logits [M, N] and the chunk pairs go to the workspace.
 * Workspace: the bytes below, 16-byte aligned, any content.  Requirements
 * of fp8lin_linear and fp8lin_vocab_candidates.
 */
size_t fp8lin_linear_candidates_workspace_bytes(int64_t M, int64_t N, int64_t K);
int fp8lin_linear_candidates(const uint16_t* x, const uint8_t* codes, const float* scales,
                             int64_t scale_cols, int64_t M, int64_t N, int64_t K, int64_t offset,
                             double* out, void* workspace, size_t workspace_bytes,
                             fp8lin_stream_t stream);

/* Allocation-free form of fp8lin_linear_candidates.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory or call
 * hipMalloc (code under HIP graph capture such as the MTP draft step, tight
 * serving loops).  Same arguments, checks and result (bit for bit) as
 * fp8lin_linear_candidates, without the workspace: the logits and candidate
 * pairs go to a static device scratch of FP8LIN_STATIC_SCRATCH_BYTES that
 * each GPU holds from the library's first use on it until the process ends.
 * Requires fp8lin_linear_candidates_workspace_bytes(M, N, K) <= that size
 * (4 MiB: about 2.09 million logits, e.g. M x N up to 8 x 261632 or
 * 1 x 2093056), else FP8LIN_ERR_UNSUPPORTED.  Every call on one GPU shares that GPU's scratch:
 * calls that may overlap on one GPU (other streams, other threads) race, so
 * a caller serialises them.  The call allocates nothing and needs no cleared
 * memory (every scratch byte it reads is written first in the same call).
 */
#define FP8LIN_STATIC_SCRATCH_BYTES (4u << 20)
int fp8lin_linear_candidates_static(const uint16_t* x, const uint8_t* codes, const float* scales,
                                    int64_t scale_cols, int64_t M, int64_t N, int64_t K, int64_t offset,
                                    double* out, fp8lin_stream_t stream);

/* The head projection through Engine::linear's dispatch, then its candidates:
 * Engine::local_candidates with gpu_candidates (src/speculative.cpp:25-27).
 * out equals fp8lin_vocab_candidates of fp8lin_engine_linear's output for
 * the same options (so rows 2..8 take the small-M path when the options
 * select it).  On the FP8 GEMV branch without a bias this is
 * fp8lin_linear_candidates, and the tensor-small branch without a bias takes
 * the small-M kernel's candidate form where its row-range form runs (no
 * logits written in either).  Workspace: the bytes below
 * (the logits, the candidate pairs and the branch's own workspace), 16-byte
 * aligned.
 */
size_t fp8lin_engine_linear_candidates_workspace_bytes(const fp8lin_linear_options* options,
                                                       const fp8lin_weight* weight, int64_t rows);
int fp8lin_engine_linear_candidates(const fp8lin_linear_options* options, const fp8lin_weight* weight,
                                    const uint16_t* x, int64_t rows, int64_t offset, double* out,
                                    void* workspace, size_t workspace_bytes, int* path_out,
                                    fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * Decode chain: the one-row linear layers of one decode step in a single
 * launch.  Replaces the sequence of Engine::linear calls of Engine::step
 * (src/engine.cpp:401-421) at one token, which the reference replays as one
 * captured graph (src/engine.cpp:522-539): link L computes y = x * W^T (with
 * swiglu, the fused gate/up + SwiGLU of fp8lin_linear_swiglu) for one
 * activation row, and its output equals fp8lin_linear's
 * (fp8lin_linear_swiglu's) for M = 1 bit for bit.  A link whose `after` is
 * an earlier link's index reads x only once that link has stored all its
 * outputs, so x may be (part of) the output of link `after`; with
 * after = -1, x must be ready when the call is enqueued.  The workgroups of
 * the links run in link order, and each issues its weight loads before it
 * waits, so HBM stays busy across the links.
 * Requirements per link: K % 16 == 0, K <= 9216 (with swiglu, N even and
 * K <= 5120), scale_cols 1 or ceil(K/128), N * K < 2^31; the outputs of the
 * links do not overlap each other or any weight, and a link's output
 * overlaps only the x of links that wait for it.
 * Workspace: fp8lin_decode_chain_workspace_bytes(nlinks) bytes (16-byte
 * aligned) of 64-bit counters, all zero before the first call on it.  The
 * counters never reset, so one zeroed workspace serves any number of calls
 * of ONE chain shape (the links' N, K, swiglu and after) on one stream and
 * device; calls that may overlap, or a chain of another shape, need their
 * own (or a workspace zeroed again).  Word 0 counts the waits that gave up:
 * a link's input not complete after about 2^20 polls (which only a grid
 * that cannot stay resident, e.g. beside other kernels on a shared GPU, can
 * cause), or, at once, every wait of a chain given a workspace that counted
 * a chain of another shape (word 1 records the shape).  A call that adds to
 * word 0 has wrong outputs.  No counterpart in the reference's operator
 * set.
 */
#define FP8LIN_CHAIN_MAX_LINKS 8
typedef struct fp8lin_chain_link {
    const uint8_t* codes;  /* E4M3FN [N, K] */
    const float* scales;   /* [N] or [N, ceil(K/128)] */
    int64_t scale_cols;    /* 1 or ceil(K/128) */
    int64_t N, K;
    const uint16_t* x;     /* BF16 [1, K] */
    uint16_t* y;           /* BF16 [1, N], or [1, N/2] with swiglu */
    int swiglu;            /* rows [0, N/2) gate, [N/2, N) up; y = SwiGLU */
    int after;             /* index of an earlier link to wait for, or -1 */
} fp8lin_chain_link;
size_t fp8lin_decode_chain_workspace_bytes(int nlinks);
int fp8lin_decode_chain(const fp8lin_chain_link* links, int nlinks, void* workspace, size_t workspace_bytes,
                        fp8lin_stream_t stream);

/* ---------------------------------------------------------------------------
 * Deterministic synthetic inputs (no reference counterpart; used by the
 * benchmark and tests so that the device and a host checker see the same
 * bits).  Element i of stream `tag` is a standard normal from Philox4x32-10
 * (counter (i lo, i hi, tag, 0x6a09e667), key (seed lo, seed hi)) through
 * Box-Muller.  Weights are std * normal, quantized per 128x128 block with
 * scale = max(amax, 1e-12) / 448 and codes = E4M3FN(w / scale) (round to
 * nearest even), the recipe of tools/make_tiny_fixture.py:56-61; scales are
 * written row-expanded [N, ceil(K/128)].  Activations are bf16(normal).
 */
int fp8lin_gen_weights(uint64_t seed, uint32_t tag, int64_t N, int64_t K, float std_dev,
                       uint8_t* codes, float* scales, fp8lin_stream_t stream);
int fp8lin_gen_activations(uint64_t seed, uint32_t tag, int64_t M, int64_t K, uint16_t* x,
                           fp8lin_stream_t stream);
int fp8lin_gen_normal(uint64_t seed, uint32_t tag, uint64_t first, int64_t n, float* out,
                      fp8lin_stream_t stream);

/* Streaming-read probe (no reference counterpart): reads `bytes` bytes in
 * the decode GEMV's access pattern (each wave a contiguous 10 KiB with all
 * its 128-bit loads in flight) and may write checksum words into sink
 * (>= 4096 floats).  Used to measure the practical HBM read ceiling;
 * 16 <= bytes < 2^40. */
int fp8lin_stream_read(const void* src, size_t bytes, float* sink, fp8lin_stream_t stream);

/* MFMA-ceiling probe (no reference counterpart): one workgroup of 4 waves per
 * CU, each wave issuing iters x 16 independent v_mfma_f32_32x32x16_bf16 on
 * register operands (no memory traffic).  clocks[0] and clocks[1] receive the
 * shader-clock (s_memtime) and 100 MHz real-time (s_memrealtime) ticks that
 * workgroup 0 spent in that loop; sink (1 float) keeps the work alive.  Flops
 * per launch: CUs x 4 x iters x 16 x 32768.  Used to measure the practical
 * BF16 MFMA ceiling and the clock it runs at. */
int fp8lin_mfma_ceiling(int64_t iters, float* sink, uint64_t* clocks, fp8lin_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* FP8LIN_H */
