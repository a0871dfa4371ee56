/*
 * fp8lin CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference engine's block-FP8 linear numerics
 * (laoyin/a100-vision-infer).  It is the checker for the HIP library: only the
 * tests, the smoke check and the CPU-baseline leg of the benchmark may load it.
 * The product library never links, calls or falls back to it.
 *
 * Every function names the reference file:line it restates.  The checks that
 * pin each function (known-answer vectors, library routines, closed forms,
 * brute force) live in tests/test_oracle.py.
 *
 * Data layout (same as the reference):
 *   codes   uint8  [N, K] row-major, E4M3FN bytes
 *   scales  float  [N, S] row-major, S = 1 (per-row) or S = ceil(K/128)
 *                  (128x128 block scales expanded along rows)
 *   x, y    uint16 [M, K] / [M, N] row-major BF16 bit patterns
 */
#ifndef FP8LIN_ORACLE_H
#define FP8LIN_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* E4M3FN byte -> float, exact.  include/avi/fp8_codec.cuh:5-10. */
float oracle_fp8_e4m3_value(uint8_t code);
/* float -> BF16 bits, round-to-nearest-even; NaN -> quiet NaN (sign kept).
 * tools/format_utils.py:5-9 (finite values). */
uint16_t oracle_bf16_rne(float v);
float oracle_bf16_to_float(uint16_t b);
/* float -> E4M3FN byte, round-to-nearest-even, NaN/overflow -> 0x7f|sign.
 * The cast `(block/scale).to(torch.float8_e4m3fn)` of
 * tools/make_tiny_fixture.py:61. */
uint8_t oracle_e4m3_from_float(float v);

/* Batch helpers (n elements). */
void oracle_decode_table(float* out256);
void oracle_bf16_rne_array(const float* in, uint16_t* out, size_t n);
void oracle_e4m3_from_float_array(const float* in, uint8_t* out, size_t n);

/* Row expansion of [ceil(N/128), KB] block scales to [N, KB].
 * tools/fp8_import_utils.py:20 (np.repeat(scales,128,axis=0)[:n]). */
void oracle_expand_block_scales(const float* block, float* out, int64_t N, int64_t KB);

/* Per-element dequant y[i] = bf16(dec(q[i]) * s[row*S + (S==1 ? 0 : col/128)]).
 * src/kernels.cu:13-16. */
void oracle_dequant(const uint8_t* codes, const float* scales, int64_t scale_cols,
                    uint16_t* y, int64_t rows, int64_t cols);

/* Linear y[M,N] = bf16( sum_k double(x[m,k]) * double(bf16(dec(c[n,k]) * s)) ).
 * tests/fp8_tensor_test.cpp:11-22 (FP64 matmul, then BF16 via float).  Rows
 * n in [n_begin, n_end) only (the rest of y is untouched); threads <= 0 uses
 * the OpenMP default.  Returns 0, or -1 on bad arguments. */
int oracle_linear(const uint16_t* x, const uint8_t* codes, const float* scales,
                  int64_t scale_cols, uint16_t* y, int64_t M, int64_t N, int64_t K,
                  int64_t n_begin, int64_t n_end, int threads);
/* Same with BF16 weights [N,K] (decoded-weight cache / unquantized weights):
 * src/engine.cpp:220-221,234-237. */
int oracle_linear_bf16w(const uint16_t* x, const uint16_t* w, uint16_t* y,
                        int64_t M, int64_t N, int64_t K, int threads);
/* SwiGLU y[r,j] = bf16( float(bf16(a/(1+expf(-a)))) * u ), a = in[r,j],
 * u = in[r,D+j]; in is [M, 2D].  src/optimized.cu:73. */
void oracle_swiglu(const uint16_t* in, uint16_t* y, int64_t M, int64_t D);

/* ---- decode epilogue and output head ---- */
/* RMSNorm of BF16 rows: inv = 1/sqrt(sum_i x^2 / D + eps) (sum and root in
 * double), v = float(x) * inv, rounded to BF16 first when !centered, then
 * y = bf16(v * (w + (centered ? 1 : 0))).  src/optimized.cu:71 (`rms`). */
void oracle_rms(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t M, int64_t D, float eps,
                int centered);
/* Multi-axis rotary embedding of x [T, H, D] at pos [3, T] (src/optimized.cu:77-78). */
void oracle_rope(const uint16_t* x, const int64_t* pos, uint16_t* y, int64_t T, int64_t H, int64_t D, int64_t R,
                 float theta, int64_t hs, int64_t ws);
/* residual = bf16(float(x) + float(update)); y = oracle_rms(residual).
 * src/dual_path.cu:12-28 (`add_norm`). */
void oracle_residual_rms(const uint16_t* x, const uint16_t* update, const uint16_t* w, uint16_t* residual,
                         uint16_t* y, int64_t M, int64_t D, float eps, int centered);
/* Per row: the largest BF16 logit (NaN counts as +inf) and its column; ties
 * go to the smallest column.  out[2r] = value, out[2r+1] = column + offset.
 * src/dual_path.cu:29-59,80-89 (`vocabulary_candidates`). */
void oracle_vocab_candidates(const uint16_t* logits, int64_t M, int64_t N, int64_t offset, double* out);
/* gathered [ranks, rows, 2]: per row the best (value, id) over ranks, ties to
 * the smaller id; -1 when any rank's entry is non-finite or its id is not an
 * integer in [0, INT_MAX].  src/dual_path.cu:60-67 (`candidate_merge`). */
void oracle_merge_candidates(const double* gathered, int64_t ranks, int64_t rows, int64_t* out);

/* ---- deterministic synthetic inputs (seeded, counter based) ---- */
/* Philox4x32-10 (Salmon et al., SC'11): counter ctr[4], key key[2]. */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* Standard normal for element `index` of stream `tag` under `seed`. */
float oracle_normal(uint64_t seed, uint32_t tag, uint64_t index);
void oracle_normal_array(uint64_t seed, uint32_t tag, uint64_t first, float* out, size_t n);
/* W ~ std*N(0,1) [N,K] (tag 1), quantized per 128x128 block:
 * scale = max(amax, 1e-12)/448, code = e4m3(w/scale) (tools/make_tiny_fixture.py:56-61);
 * scales written row-expanded [N, ceil(K/128)].  w_out (optional) receives W. */
void oracle_gen_weights(uint64_t seed, uint32_t tag, int64_t N, int64_t K, float std_dev,
                        uint8_t* codes, float* scales, float* w_out);
/* x = bf16(N(0,1)) [M,K] (tag given by caller). */
void oracle_gen_activations(uint64_t seed, uint32_t tag, int64_t M, int64_t K, uint16_t* x);

int oracle_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
