/*
 * fp8lin CPU oracle -- TEST INFRASTRUCTURE ONLY (see fp8lin_oracle.h).
 *
 * Built by oracle/build_oracle.py with: gcc -O2 -march=x86-64-v3
 * -ffp-contract=off -fopenmp.  -ffp-contract=off matters: the synthetic-input
 * generator must produce the same float bits as the GPU generator, so every
 * multiply-add below is either an explicit fmaf() or two separately rounded
 * operations.
 */
#include "fp8lin_oracle.h"
#include <math.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* include/avi/fp8_codec.cuh:5-10: e=(c>>3)&15, m=c&7; NaN iff e==15 && m==7;
 * normal -> sign | (e+120)<<23 | m<<20; subnormal -> +-m * 2^-9. */
float oracle_fp8_e4m3_value(uint8_t code) {
    uint32_t e = (code >> 3) & 15u, m = code & 7u, sign = ((uint32_t)code & 128u) << 24;
    if (e == 15u && m == 7u) return u2f(sign | 0x7fc00000u);
    if (e) return u2f(sign | ((e + 120u) << 23) | (m << 20));
    return u2f(sign | f2u((float)m * 0.001953125f));
}

/* tools/format_utils.py:5-9: bits + 0x7fff + ((bits>>16)&1), keep the high
 * half.  That formula turns some NaN payloads into Inf; NaN is mapped to a
 * quiet NaN with the same sign instead (what the GPU's BF16 conversion and
 * CUDA's __float2bfloat16_rn both return for NaN). */
uint16_t oracle_bf16_rne(float v) {
    uint32_t bits = f2u(v);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

float oracle_bf16_to_float(uint16_t b) { return u2f((uint32_t)b << 16); }

/* Round-to-nearest-even onto the E4M3FN grid (bias 7, 3 mantissa bits,
 * subnormal step 2^-9).  A value that rounds to the 0x7f slot (480) or beyond,
 * +-Inf and NaN all give the NaN code 0x7f|sign: E4M3FN has no Inf and the
 * torch cast used by tools/make_tiny_fixture.py:61 does not saturate. */
uint8_t oracle_e4m3_from_float(float v) {
    uint8_t sign = signbit(v) ? 0x80 : 0x00;
    float a = fabsf(v);
    if (!(a < 480.0f)) return (uint8_t)(sign | 0x7f);
    if (a < 0.015625f) {                         /* below 2^-6: subnormal grid */
        float q = nearbyintf(a * 512.0f);        /* exact scaling, RNE */
        return (uint8_t)(sign | (uint8_t)q);     /* q == 8 encodes 2^-6 */
    }
    int e2;
    float f = frexpf(a, &e2);                    /* a = f * 2^e2, f in [0.5,1) */
    int E = e2 - 1;
    float s = f * 2.0f;                          /* [1,2) */
    float mant = nearbyintf((s - 1.0f) * 8.0f);  /* exact, then RNE */
    int mi = (int)mant;
    if (mi == 8) { mi = 0; E += 1; }
    int code = ((E + 7) << 3) | mi;
    if (code >= 0x7f) code = 0x7f;
    return (uint8_t)(sign | code);
}

void oracle_decode_table(float* out256) {
    for (int c = 0; c < 256; c++) out256[c] = oracle_fp8_e4m3_value((uint8_t)c);
}
void oracle_bf16_rne_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_bf16_rne(in[i]);
}
void oracle_e4m3_from_float_array(const float* in, uint8_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_e4m3_from_float(in[i]);
}

/* tools/fp8_import_utils.py:20: expanded = np.repeat(scales, 128, axis=0)[:n]. */
void oracle_expand_block_scales(const float* block, float* out, int64_t N, int64_t KB) {
    for (int64_t n = 0; n < N; n++)
        for (int64_t b = 0; b < KB; b++) out[n * KB + b] = block[(n / 128) * KB + b];
}

static inline float scale_at(const float* scales, int64_t S, int64_t row, int64_t col) {
    return scales[row * S + (S == 1 ? 0 : col / 128)];
}

/* src/kernels.cu:13-16. */
void oracle_dequant(const uint8_t* codes, const float* scales, int64_t S,
                    uint16_t* y, int64_t rows, int64_t cols) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        for (int64_t c = 0; c < cols; c++)
            y[r * cols + c] = oracle_bf16_rne(oracle_fp8_e4m3_value(codes[r * cols + c]) *
                                              scale_at(scales, S, r, c));
}

static int set_threads(int threads) {
#ifdef _OPENMP
    return threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

int oracle_max_threads(void) { return set_threads(0); }

/* tests/fp8_tensor_test.cpp:11-22: weight = bf16(decode(c) * s) (FP32
 * product, then BF16), matmul of double(x) and double(weight), then
 * `.to(kBFloat16)`, which converts double -> float -> BF16 (both RNE). */
int oracle_linear(const uint16_t* x, const uint8_t* codes, const float* scales,
                  int64_t S, uint16_t* y, int64_t M, int64_t N, int64_t K,
                  int64_t n_begin, int64_t n_end, int threads) {
    if (M <= 0 || N <= 0 || K <= 0 || n_begin < 0 || n_end > N || n_begin > n_end) return -1;
    if (!(S == 1 || S == (K + 127) / 128)) return -1;
    double* xd = (double*)malloc(sizeof(double) * (size_t)(M * K));
    if (!xd) return -1;
    for (int64_t i = 0; i < M * K; i++) xd[i] = (double)oracle_bf16_to_float(x[i]);
    int nt = set_threads(threads);
    int failed = 0;
#pragma omp parallel num_threads(nt)
    {
        double* w = (double*)malloc(sizeof(double) * (size_t)K);
        if (!w) {
#pragma omp atomic write
            failed = 1;
        } else {
#pragma omp for schedule(static)
            for (int64_t n = n_begin; n < n_end; n++) {
                const uint8_t* crow = codes + n * K;
                for (int64_t k = 0; k < K; k++)
                    w[k] = (double)oracle_bf16_to_float(
                        oracle_bf16_rne(oracle_fp8_e4m3_value(crow[k]) * scale_at(scales, S, n, k)));
                for (int64_t m = 0; m < M; m++) {
                    const double* xr = xd + m * K;
                    double acc = 0.0;
                    for (int64_t k = 0; k < K; k++) acc += xr[k] * w[k];
                    y[m * N + n] = oracle_bf16_rne((float)acc);
                }
            }
            free(w);
        }
    }
    free(xd);
    return failed ? -1 : 0;
}

/* src/engine.cpp:220-221 / :234-237: at::matmul(x, w.t()) with BF16 weights,
 * restated with the same FP64 accumulation and BF16 output rounding. */
int oracle_linear_bf16w(const uint16_t* x, const uint16_t* w, uint16_t* y,
                        int64_t M, int64_t N, int64_t K, int threads) {
    if (M <= 0 || N <= 0 || K <= 0) return -1;
    double* xd = (double*)malloc(sizeof(double) * (size_t)(M * K));
    if (!xd) return -1;
    for (int64_t i = 0; i < M * K; i++) xd[i] = (double)oracle_bf16_to_float(x[i]);
    int nt = set_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t n = 0; n < N; n++) {
        const uint16_t* wr = w + n * K;
        for (int64_t m = 0; m < M; m++) {
            const double* xr = xd + m * K;
            double acc = 0.0;
            for (int64_t k = 0; k < K; k++) acc += xr[k] * (double)oracle_bf16_to_float(wr[k]);
            y[m * N + n] = oracle_bf16_rne((float)acc);
        }
    }
    free(xd);
    return 0;
}

/* src/optimized.cu:73: gate = bf16(a/(1+expf(-a))); y = bf16(gate * u). */
void oracle_swiglu(const uint16_t* in, uint16_t* y, int64_t M, int64_t D) {
    for (int64_t r = 0; r < M; r++)
        for (int64_t j = 0; j < D; j++) {
            float a = oracle_bf16_to_float(in[r * 2 * D + j]);
            float u = oracle_bf16_to_float(in[r * 2 * D + D + j]);
            float g = oracle_bf16_to_float(oracle_bf16_rne(a / (1.0f + expf(-a))));
            y[r * D + j] = oracle_bf16_rne(g * u);
        }
}

/* ---------------- deterministic synthetic inputs ---------------- */

/* Philox4x32-10, Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
 * easy as 1, 2, 3" (SC'11): multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key
 * increments 0x9E3779B9 / 0xBB67AE85, ten rounds. */
void oracle_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int r = 0; r < 10; r++) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t h0 = (uint32_t)(p0 >> 32), l0 = (uint32_t)p0;
        uint32_t h1 = (uint32_t)(p1 >> 32), l1 = (uint32_t)p1;
        uint32_t n0 = h1 ^ c1 ^ k0, n2 = h0 ^ c3 ^ k1;
        c0 = n0; c1 = l1; c2 = n2; c3 = l0;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* ln(u) for u in (0,1], from +,*,/ and fmaf only, so that the CPU and the GPU
 * produce identical bits: u = m*2^e with m in [sqrt(1/2), sqrt(2)),
 * ln(m) = 2 atanh(t), t = (m-1)/(m+1), series to t^13. */
static float det_log(float u) {
    uint32_t b = f2u(u);
    int e = (int)(b >> 23) - 127;
    uint32_t mb = (b & 0x007fffffu) | 0x3f800000u;
    if (mb > 0x3fb504f3u) { mb -= 0x00800000u; e += 1; }
    float m = u2f(mb);
    float t = (m - 1.0f) / (m + 1.0f);
    float t2 = t * t;
    float p = fmaf(t2, 0x1.3b13b2p-4f, 0x1.745d18p-4f);
    p = fmaf(t2, p, 0x1.c71c72p-4f);
    p = fmaf(t2, p, 0x1.24924ap-3f);
    p = fmaf(t2, p, 0x1.99999ap-3f);
    p = fmaf(t2, p, 0x1.555556p-2f);
    p = fmaf(t2, p, 1.0f);
    float lnm = (t + t) * p;
    return fmaf((float)e, 0x1.62e430p-1f, lnm);
}

/* cos(2*pi*u) for u in [0,1): quadrant from 4u (exact), Taylor polynomials
 * of cos/sin on [0, pi/2] evaluated with fmaf. */
static float det_cos2pi(float u) {
    float q4 = u * 4.0f;
    int q = (int)q4;
    float f = q4 - (float)q;
    float th = f * 0x1.921fb6p+0f;
    float t2 = th * th;
    float c = fmaf(t2, 0x1.1eed8ep-29f, -0x1.27e4fcp-22f);
    c = fmaf(t2, c, 0x1.a01a02p-16f);
    c = fmaf(t2, c, -0x1.6c16c2p-10f);
    c = fmaf(t2, c, 0x1.555556p-5f);
    c = fmaf(t2, c, -0.5f);
    c = fmaf(t2, c, 1.0f);
    float s = fmaf(t2, 0x1.612462p-33f, -0x1.ae6456p-26f);
    s = fmaf(t2, s, 0x1.71de3ap-19f);
    s = fmaf(t2, s, -0x1.a01a02p-13f);
    s = fmaf(t2, s, 0x1.111112p-7f);
    s = fmaf(t2, s, -0x1.555556p-3f);
    s = fmaf(t2, s, 1.0f);
    s = s * th;
    switch (q & 3) {
        case 0: return c;
        case 1: return -s;
        case 2: return -c;
        default: return s;
    }
}

/* Box-Muller on one Philox block: counter (index lo, index hi, tag,
 * 0x6a09e667), key (seed lo, seed hi); u1 = (r0>>8 + 1)/2^24 in (0,1],
 * u2 = (r1>>8)/2^24 in [0,1); z = sqrt(-2 ln u1) * cos(2 pi u2). */
float oracle_normal(uint64_t seed, uint32_t tag, uint64_t index) {
    uint32_t ctr[4] = {(uint32_t)index, (uint32_t)(index >> 32), tag, 0x6a09e667u};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t r[4];
    oracle_philox4x32_10(ctr, key, r);
    float u1 = (float)((r[0] >> 8) + 1u) * 0x1p-24f;
    float u2 = (float)(r[1] >> 8) * 0x1p-24f;
    float rad = sqrtf(-2.0f * det_log(u1));
    return rad * det_cos2pi(u2);
}

void oracle_normal_array(uint64_t seed, uint32_t tag, uint64_t first, float* out, size_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; i++) out[i] = oracle_normal(seed, tag, first + (uint64_t)i);
}

/* tools/make_tiny_fixture.py:56-61: per 128x128 block,
 * scale = block.abs().max().clamp_min(1e-12)/448, codes = (block/scale) cast
 * to E4M3FN; the [ceil(N/128), ceil(K/128)] scales are then row-expanded as
 * tools/fp8_import_utils.py:20 does. */
void oracle_gen_weights(uint64_t seed, uint32_t tag, int64_t N, int64_t K, float std_dev,
                        uint8_t* codes, float* scales, float* w_out) {
    int64_t NB = (N + 127) / 128, KB = (K + 127) / 128;
#pragma omp parallel for schedule(dynamic)
    for (int64_t blk = 0; blk < NB * KB; blk++) {
        int64_t bn = blk / KB, bk = blk % KB;
        int64_t r0 = bn * 128, r1 = r0 + 128 < N ? r0 + 128 : N;
        int64_t c0 = bk * 128, c1 = c0 + 128 < K ? c0 + 128 : K;
        float w[128 * 128];
        float amax = 0.0f;
        for (int64_t r = r0; r < r1; r++)
            for (int64_t c = c0; c < c1; c++) {
                float v = std_dev * oracle_normal(seed, tag, (uint64_t)(r * K + c));
                w[(r - r0) * 128 + (c - c0)] = v;
                float a = fabsf(v);
                if (a > amax) amax = a;
            }
        float scale = (amax > 1e-12f ? amax : 1e-12f) / 448.0f;
        for (int64_t r = r0; r < r1; r++) {
            scales[r * KB + bk] = scale;
            for (int64_t c = c0; c < c1; c++) {
                float v = w[(r - r0) * 128 + (c - c0)];
                codes[r * K + c] = oracle_e4m3_from_float(v / scale);
                if (w_out) w_out[r * K + c] = v;
            }
        }
    }
}

void oracle_gen_activations(uint64_t seed, uint32_t tag, int64_t M, int64_t K, uint16_t* x) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M * K; i++) x[i] = oracle_bf16_rne(oracle_normal(seed, tag, (uint64_t)i));
}

/* ---------------- decode epilogue and output head ---------------- */

static void rms_row(const float* r, const uint16_t* w, uint16_t* y, int64_t D, float eps, int centered) {
    double ss = 0.0;
    for (int64_t i = 0; i < D; i++) ss += (double)r[i] * (double)r[i];
    const float inv = (float)(1.0 / sqrt(ss / (double)D + (double)eps));
    for (int64_t i = 0; i < D; i++) {
        float v = r[i] * inv;
        if (!centered) v = oracle_bf16_to_float(oracle_bf16_rne(v));
        y[i] = oracle_bf16_rne(v * (oracle_bf16_to_float(w[i]) + (centered ? 1.0f : 0.0f)));
    }
}

/* src/optimized.cu:71 */
void oracle_rms(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t M, int64_t D, float eps,
                int centered) {
    float* r = (float*)malloc((size_t)D * sizeof(float));
    for (int64_t m = 0; m < M; m++) {
        for (int64_t i = 0; i < D; i++) r[i] = oracle_bf16_to_float(x[m * D + i]);
        rms_row(r, w, y + m * D, D, eps, centered);
    }
    free(r);
}

/* src/optimized.cu:77 (rope_kernel), the multi-axis rotary embedding of
 * fused_rope (:78): x [T, H, D] BF16, pos [3, T] int64.  For d < R, pair
 * index f = d mod R/2 takes its position from axis 1 when f mod 3 == 1 and
 * f < 3*hs, from axis 2 when f mod 3 == 2 and f < 3*ws, else axis 0;
 *   angle = float(pos) * powf(theta, -2f*f/R)   (FP32)
 *   co = bf16(cos(angle)), si = bf16(sin(angle))
 *   y[d] = bf16(bf16(x[d]*co) + bf16(s*x[d'] * si))
 * with d' = d + R/2, s = -1 for d < R/2 and d' = d - R/2, s = +1 otherwise.
 * Elements d >= R are copied. */
void oracle_rope(const uint16_t* x, const int64_t* pos, uint16_t* y, int64_t T, int64_t H, int64_t D, int64_t R,
                 float theta, int64_t hs, int64_t ws) {
    const int64_t half = R / 2;
    for (int64_t t = 0; t < T; t++)
        for (int64_t h = 0; h < H; h++) {
            const uint16_t* xr = x + (t * H + h) * D;
            uint16_t* yr = y + (t * H + h) * D;
            for (int64_t d = 0; d < D; d++) {
                if (d >= R) {
                    yr[d] = xr[d];
                    continue;
                }
                const int64_t f = d % half;
                const int axis = (f % 3 == 1 && f < hs * 3) ? 1 : ((f % 3 == 2 && f < ws * 3) ? 2 : 0);
                const float angle = (float)pos[axis * T + t] * powf(theta, -2.0f * (float)f / (float)R);
                const float co = oracle_bf16_to_float(oracle_bf16_rne(cosf(angle)));
                const float si = oracle_bf16_to_float(oracle_bf16_rne(sinf(angle)));
                const float rotated = d < half ? -oracle_bf16_to_float(xr[d + half]) : oracle_bf16_to_float(xr[d - half]);
                const float a = oracle_bf16_to_float(oracle_bf16_rne(oracle_bf16_to_float(xr[d]) * co));
                const float b = oracle_bf16_to_float(oracle_bf16_rne(rotated * si));
                yr[d] = oracle_bf16_rne(a + b);
            }
        }
}

/* src/dual_path.cu:12-28 */
void oracle_residual_rms(const uint16_t* x, const uint16_t* update, const uint16_t* w, uint16_t* residual,
                         uint16_t* y, int64_t M, int64_t D, float eps, int centered) {
    float* r = (float*)malloc((size_t)D * sizeof(float));
    for (int64_t m = 0; m < M; m++) {
        for (int64_t i = 0; i < D; i++) {
            const uint16_t b = oracle_bf16_rne(oracle_bf16_to_float(x[m * D + i]) +
                                               oracle_bf16_to_float(update[m * D + i]));
            residual[m * D + i] = b;
            r[i] = oracle_bf16_to_float(b);
        }
        rms_row(r, w, y + m * D, D, eps, centered);
    }
    free(r);
}

/* src/dual_path.cu:29-59 */
void oracle_vocab_candidates(const uint16_t* logits, int64_t M, int64_t N, int64_t offset, double* out) {
    for (int64_t m = 0; m < M; m++) {
        float best = -INFINITY;
        int64_t id = -1;
        for (int64_t n = 0; n < N; n++) {
            float v = oracle_bf16_to_float(logits[m * N + n]);
            if (isnan(v)) v = INFINITY;
            if (id < 0 || v > best) {
                best = v;
                id = n;
            }
        }
        out[2 * m] = (double)best;
        out[2 * m + 1] = (double)(id + offset);
    }
}

/* src/dual_path.cu:60-67 */
void oracle_merge_candidates(const double* gathered, int64_t ranks, int64_t rows, int64_t* out) {
    for (int64_t r = 0; r < rows; r++) {
        double best = -INFINITY;
        int64_t id = INT64_MAX;
        int invalid = 0;
        for (int64_t k = 0; k < ranks; k++) {
            const double v = gathered[(k * rows + r) * 2], raw = gathered[(k * rows + r) * 2 + 1];
            if (!isfinite(v) || !isfinite(raw) || raw < 0 || raw > 2147483647.0 || raw != floor(raw)) {
                invalid = 1;
                continue;
            }
            const int64_t next = (int64_t)raw;
            if (v > best || (v == best && next < id)) {
                best = v;
                id = next;
            }
        }
        out[r] = invalid ? -1 : id;
    }
}
