/*
 * vxm_oracle.c -- scalar CPU restatement of the Q8_0 matmul path and the
 * MiniCPM4 / LocDiT / CFM math that surrounds it in the VoxCPM2 C runtime.
 *
 * TEST INFRASTRUCTURE ONLY: used by the test suite, the smoke check and the
 * CPU-baseline leg of the benchmark as the checker.  The product library
 * never links or calls it.
 *
 * Third-party algorithm: ggml-org/ggml v0.15.2 (CMakeLists.txt:54-70, not
 * vendored).  The Q8_0 functions restate ggml's published block_q8_0 format,
 * quantize_row_q8_0_ref, the x86 SIMD quantize_row_q8_0 and
 * vec_dot_q8_0_q8_0; the norm / rope / softmax functions restate
 * ggml_rms_norm, ggml_rope_ext (NEOX) and ggml_soft_max_ext as the reference
 * builds them.  Where ggml's exact floating-point order cannot be pinned
 * offline, the function says "parity unpinned" and the tests use tolerances.
 *
 * Build with -ffp-contract=off: every a*b+c below is two roundings, as in
 * ggml's scalar code compiled in ISO C mode.
 */
#include "vxm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Threading.  Large products run with OpenMP over independent outputs: every
 * output element is still formed by one thread, in the sequential order
 * written below, so results do not depend on the thread count. */
#define ORC_PAR_MIN 4096   /* outputs x blocks below which the loops stay serial */

/* ------------------------------------------------------------------------ */
/* number formats                                                            */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE-754 binary32 -> binary16, round to nearest even (ggml GGML_FP32_TO_FP16
 * on x86 is F16C _cvtss_sh(x, 0), i.e. RNE).  Pinned against numpy.float16. */
uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);     /* >= 65520 -> inf */
    uint32_t exp = ax >> 23;
    uint32_t man = (ax & 0x7fffffu) | 0x800000u;
    if (exp < 113) {                                                /* f16 subnormal / 0 */
        if (exp == 0) return (uint16_t)sign;                        /* f32 denormal -> 0 */
        uint32_t shift = 126 - exp;                                 /* >= 14 */
        if (shift > 24) return (uint16_t)sign;
        uint32_t q = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((exp - 112) << 10) | ((ax & 0x7fffffu) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float orc_fp16_to_fp32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        float v = (float)man * (1.0f / 16777216.0f);                /* man * 2^-24, exact */
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112) << 23) | (man << 13));
}

/* F32 -> BF16 -> F32, round to nearest even, quiet NaN.  Restates
 * ggml_fp32_to_bf16 as used by minicpm_bf16_round (src/minicpm4.c:39-42),
 * locdit_bf16_round (src/locdit.c:118-121) and bf16_scalar
 * (src/cfm_solver.c:23-25).  Pinned by tests/test_cfm_schedule.c:6-36.
 * f32 subnormal inputs: parity unpinned (ggml variants differ on flushing). */
float orc_bf16_round(float f) {
    uint32_t u = f2u(f);
    uint32_t h;
    if ((u & 0x7fffffffu) > 0x7f800000u) h = (u >> 16) | 64u;
    else h = (u + (0x7fffu + ((u >> 16) & 1u))) >> 16;
    return u2f(h << 16);
}

void orc_fp32_to_fp16_n(const float *x, uint16_t *h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = orc_fp32_to_fp16(x[i]);
}
void orc_fp16_to_fp32_n(const uint16_t *h, float *x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = orc_fp16_to_fp32(h[i]);
}
void orc_bf16_round_n(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_bf16_round(x[i]);
}

/* ------------------------------------------------------------------------ */
/* Q8_0                                                                      */
/* ------------------------------------------------------------------------ */

/* block_q8_0: fp16 d at byte 0, int8 qs[32] at bytes 2..33 (restated at
 * src/model_loader.c:317-331, src/gen_prompt.c:106-125, tools/bisect_q8.py:22-38).
 *
 * variant ORC_QUANT_REF: ggml quantize_row_q8_0_ref, used for weights by
 *   ggml_quantize_chunk (tools/quantize.c:292): d = amax/127, id = d ? 1/d : 0,
 *   qs = roundf(x*id) (half away from zero).
 * variant ORC_QUANT_X86: ggml's x86 SIMD quantize_row_q8_0, used for the
 *   activation (src1) of ggml_mul_mat on x86: d = amax/127,
 *   id = amax ? 127/amax : 0, qs = round-half-even(x*id).
 * Which variant a given ggml build uses for activations is parity unpinned
 * (it depends on the host ISA); both are provided and tested. */
void orc_quantize_row_q8_0(const float *x, uint8_t *y, int64_t k, int variant) {
    const int64_t nb = k / ORC_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        const float *xb = x + i * ORC_QK8_0;
        uint8_t *blk = y + i * ORC_Q8_0_BLOCK_BYTES;
        float amax = 0.0f;
        for (int j = 0; j < ORC_QK8_0; j++) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        uint16_t dh = orc_fp32_to_fp16(d);
        memcpy(blk, &dh, 2);
        int8_t *qs = (int8_t *)(blk + 2);
        if (variant == ORC_QUANT_REF) {
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            for (int j = 0; j < ORC_QK8_0; j++) qs[j] = (int8_t)roundf(xb[j] * id);
        } else {
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            for (int j = 0; j < ORC_QK8_0; j++) {
                float v = rintf(xb[j] * id);
                if (v > 127.0f) v = 127.0f;
                if (v < -128.0f) v = -128.0f;
                qs[j] = (int8_t)v;
            }
        }
    }
}

void orc_quantize_rows_q8_0(const float *x, uint8_t *y, int64_t rows, int64_t k, int variant) {
    const int64_t rb = k / ORC_QK8_0 * ORC_Q8_0_BLOCK_BYTES;
#pragma omp parallel for schedule(static) if (rows * k > 64 * ORC_PAR_MIN)
    for (int64_t r = 0; r < rows; r++) orc_quantize_row_q8_0(x + r * k, y + r * rb, k, variant);
}

/* dequantize_row_q8_0: x = fp32(d) * qs (src/model_loader.c:317-331). */
void orc_dequantize_row_q8_0(const uint8_t *y, float *x, int64_t k) {
    const int64_t nb = k / ORC_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *blk = y + i * ORC_Q8_0_BLOCK_BYTES;
        uint16_t dh; memcpy(&dh, blk, 2);
        const float d = orc_fp16_to_fp32(dh);
        const int8_t *qs = (const int8_t *)(blk + 2);
        for (int j = 0; j < ORC_QK8_0; j++) x[i * ORC_QK8_0 + j] = d * (float)qs[j];
    }
}

static inline int32_t block_dot(const uint8_t *a, const uint8_t *b) {
    const int8_t *qa = (const int8_t *)(a + 2), *qb = (const int8_t *)(b + 2);
    int32_t s = 0;
    for (int j = 0; j < ORC_QK8_0; j++) s += (int32_t)qa[j] * (int32_t)qb[j];
    return s;
}


static inline float block_scale(const uint8_t *a, const uint8_t *b) {
    uint16_t da, db; memcpy(&da, a, 2); memcpy(&db, b, 2);
    return orc_fp16_to_fp32(da) * orc_fp16_to_fp32(db);
}

/* Per-block int32 sums of vec_dot_q8_0_q8_0 (ggml, called from ggml_mul_mat at
 * src/projections.h:24-29 and src/minicpm4.c:270-279,415,441-458).  Integer
 * and order-independent: any correct implementation is bit-exact. */
void orc_block_dots_q8_0(const uint8_t *w, const uint8_t *xq, int64_t N, int64_t K,
                         int64_t M, int32_t *out) {
    const int64_t nb = K / ORC_QK8_0, rb = nb * ORC_Q8_0_BLOCK_BYTES;
#pragma omp parallel for collapse(2) schedule(static) if (M * N * nb > ORC_PAR_MIN)
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++)
            for (int64_t b = 0; b < nb; b++)
                out[(m * N + n) * nb + b] = block_dot(w + n * rb + b * ORC_Q8_0_BLOCK_BYTES,
                                                      xq + m * rb + b * ORC_Q8_0_BLOCK_BYTES);
}

/* ggml generic vec_dot_q8_0_q8_0: sumf += sumi * (d_w * d_x) block by block.
 * The x86 SIMD build accumulates in 8 fp32 lanes instead; the exact fp32
 * order of a given ggml build is parity unpinned, so callers compare with a
 * tolerance and with orc_mul_mat_q8_0_f64. */
void orc_mul_mat_q8_0(const uint8_t *w, const uint8_t *xq, int64_t N, int64_t K,
                      int64_t M, float *y) {
    const int64_t nb = K / ORC_QK8_0, rb = nb * ORC_Q8_0_BLOCK_BYTES;
#pragma omp parallel for collapse(2) schedule(static) if (M * N * nb > ORC_PAR_MIN)
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            float sumf = 0.0f;
            for (int64_t b = 0; b < nb; b++) {
                const uint8_t *wb = w + n * rb + b * ORC_Q8_0_BLOCK_BYTES;
                const uint8_t *xb = xq + m * rb + b * ORC_Q8_0_BLOCK_BYTES;
                float term = (float)block_dot(wb, xb) * block_scale(wb, xb);
                sumf = sumf + term;
            }
            y[m * N + n] = sumf;
        }
}

void orc_mul_mat_q8_0_f64(const uint8_t *w, const uint8_t *xq, int64_t N, int64_t K,
                          int64_t M, double *y) {
    const int64_t nb = K / ORC_QK8_0, rb = nb * ORC_Q8_0_BLOCK_BYTES;
#pragma omp parallel for collapse(2) schedule(static) if (M * N * nb > ORC_PAR_MIN)
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            double s = 0.0;
            for (int64_t b = 0; b < nb; b++) {
                const uint8_t *wb = w + n * rb + b * ORC_Q8_0_BLOCK_BYTES;
                const uint8_t *xb = xq + m * rb + b * ORC_Q8_0_BLOCK_BYTES;
                s += (double)((float)block_dot(wb, xb) * block_scale(wb, xb));
            }
            y[m * N + n] = s;
        }
}

/* When this file is included by the timed CPU baseline, the baseline swaps in
 * its SIMD mul_mat and attention through these pointers and threads the
 * attention heads of a single token; the oracle build leaves the pointers NULL
 * and threads only multi-token attention (its results do not depend on it). */
#ifdef ORC_MUL_MAT_HOOK
static void (*g_mul_mat_hook)(const uint8_t *, const float *, int64_t, int64_t, int64_t, float *,
                              int) = NULL;
static void (*g_attend_hook)(const float *, const uint16_t *, const uint16_t *, int64_t, int64_t, int64_t,
                             float *, float *) = NULL;
#endif
#ifndef ORC_ATTN_PAR_MIN
#define ORC_ATTN_PAR_MIN 16
#endif

/* ggml_mul_mat(W_q8_0, x_f32): quantize each x row (activation variant), then
 * the Q8_0 x Q8_0 dot per output.  Output y[m*N + n]. */
static void mul_mat_f32_in(const uint8_t *w, const float *x, int64_t N, int64_t K, int64_t M,
                           float *y, int variant) {
#ifdef ORC_MUL_MAT_HOOK
    if (g_mul_mat_hook) { g_mul_mat_hook(w, x, N, K, M, y, variant); return; }
#endif
    const int64_t rb = K / ORC_QK8_0 * ORC_Q8_0_BLOCK_BYTES;
    uint8_t *xq = (uint8_t *)malloc((size_t)(M * rb));
    orc_quantize_rows_q8_0(x, xq, M, K, variant);
    orc_mul_mat_q8_0(w, xq, N, K, M, y);
    free(xq);
}

/* ------------------------------------------------------------------------ */
/* MiniCPM4 block (src/minicpm4.c)                                           */
/* ------------------------------------------------------------------------ */

/* vcpm_rms_norm (src/minicpm4.c:132-152): ggml_rms_norm then BF16, * gain,
 * BF16.  ggml_rms_norm: sum of float squares in double, mean = (float)(sum/n),
 * scale = 1/sqrtf(mean + eps), y = x * scale.  Pinned against the reference's
 * golden tests/fixtures/rms_norm_*.bin and tests/test_minicpm4.c:154-181. */
void orc_rms_norm(const float *x, const float *g, int64_t rows, int64_t n, float eps, float *y) {
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * n;
        float *yr = y + r * n;
        double sum = 0.0;
        for (int64_t i = 0; i < n; i++) sum += (double)(xr[i] * xr[i]);
        const float mean = (float)(sum / (double)n);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t i = 0; i < n; i++) {
            float v = orc_bf16_round(xr[i] * scale);
            yr[i] = g ? orc_bf16_round(v * g[i]) : v;
        }
    }
}

/* vcpm_rope (src/minicpm4.c:165-223): ggml_rope_ext NEOX, n_dims = head_dim,
 * freq_scale 1, ext_factor 0, attn_factor 1, optional per-pair freq factors,
 * then BF16.  ggml builds theta iteratively: theta_0 = pos,
 * theta_{i+1} = theta_i * base^(-2/n_dims), and rotates pair (i, i + n/2) by
 * theta_i / ff_i.  cosf/sinf last-ulp behaviour is parity unpinned. */
void orc_rope_neox(float *x, int64_t n_heads, int64_t head_dim, int32_t pos,
                   float theta_base, const float *ff) {
    const int64_t half = head_dim / 2;
    const float theta_scale = powf(theta_base, -2.0f / (float)head_dim);
    float *cs = (float *)malloc(sizeof(float) * (size_t)head_dim);
    float theta = (float)pos;
    for (int64_t i = 0; i < half; i++) {
        const float f = ff ? ff[i] : 1.0f;
        const float th = theta / f;
        cs[2 * i] = cosf(th);
        cs[2 * i + 1] = sinf(th);
        theta *= theta_scale;
    }
    for (int64_t h = 0; h < n_heads; h++) {
        float *v = x + h * head_dim;
        for (int64_t i = 0; i < half; i++) {
            const float c = cs[2 * i], s = cs[2 * i + 1];
            const float x0 = v[i], x1 = v[i + half];
            v[i] = orc_bf16_round(x0 * c - x1 * s);
            v[i + half] = orc_bf16_round(x0 * s + x1 * c);
        }
    }
    free(cs);
}

/* ggml_silu_f32: x / (1 + expf(-x)).  ggml's SIMD builds use their own exp
 * approximation; last-ulp behaviour is parity unpinned. */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* gqa_group_attn (src/minicpm4.c:232-248) for one query head over kv_len
 * positions: scores = k.q * (1/sqrt(hd)), ggml_soft_max_ext (max, expf,
 * sum in double, scale by (float)(1/sum)), out = sum_j v_j p_j. */
static void attend_one(const float *q, const uint16_t *k, const uint16_t *v, int64_t kv_len,
                       int64_t hd, int64_t stride, float *out, float *scratch) {
    const float sc = 1.0f / sqrtf((float)hd);
    float mx = -INFINITY;
    for (int64_t j = 0; j < kv_len; j++) {
        float s = 0.0f;
        for (int64_t d = 0; d < hd; d++) s += orc_fp16_to_fp32(k[j * stride + d]) * q[d];
        s *= sc;
        scratch[j] = s;
        if (s > mx) mx = s;
    }
    double sum = 0.0;
    for (int64_t j = 0; j < kv_len; j++) {
        float e = expf(scratch[j] - mx);
        scratch[j] = e;
        sum += (double)e;
    }
    const float inv = (float)(1.0 / sum);
    for (int64_t j = 0; j < kv_len; j++) scratch[j] *= inv;
    for (int64_t d = 0; d < hd; d++) {
        float o = 0.0f;
        for (int64_t j = 0; j < kv_len; j++) o += orc_fp16_to_fp32(v[j * stride + d]) * scratch[j];
        out[d] = o;
    }
}

/* ggml_mul_mat(W, x) for a block weight: Q8_0 rows (wtype 0) or F32 rows
 * [N][K] (wtype 1, the F32 path the reference's op fixtures use,
 * tests/fixtures/gen_op_fixtures.py:35-235; fp32 sequential dot). */
static void layer_mul_mat(const orc_layer *w, const void *wp, const float *x, int64_t N, int64_t K,
                          int64_t M, float *y, int var) {
    if (w->wtype == 0) { mul_mat_f32_in((const uint8_t *)wp, x, N, K, M, y, var); return; }
    const float *wf = (const float *)wp;
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            float s = 0.0f;
            for (int64_t i = 0; i < K; i++) s += wf[n * K + i] * x[m * K + i];
            y[m * N + n] = s;
        }
}

/* vcpm_attention (src/minicpm4.c:250-428) over M tokens at positions
 * pos..pos+M-1: Q/K/V projections (BF16), NEOX RoPE (BF16), KV append, GQA
 * attention per token (q head h reads kv head h / (n_heads/n_kv_heads)),
 * O projection (BF16).  KV cache: f16 [n_kv][capacity][head_dim] (the
 * reference keeps F32, src/minicpm4.c:107-116; K and V are BF16-rounded
 * before the copy, so f16 storage is exact for normal-range values).
 * no_causal = 1 attends over the M fresh tokens only, as LocDiT/LocEnc do
 * (src/minicpm4.c:342-355).  xn: normed input [M][hidden]; out: [M][hidden]. */
int orc_attention(const orc_cfg *cfg, const orc_layer *w, const float *xn, int64_t M,
                  uint16_t *k_cache, uint16_t *v_cache, int64_t capacity, int32_t pos,
                  int no_causal, float *out) {
    const int64_t H = cfg->hidden, hd = cfg->head_dim, nh = cfg->n_heads, nkv = cfg->n_kv_heads;
    const int64_t qd = nh * hd, kvd = nkv * hd, qpk = nh / nkv;
    const int var = cfg->quant_variant;
    if (!no_causal && pos + M > capacity) return -1;
    float *q = (float *)malloc(sizeof(float) * (size_t)(M * qd));
    float *k = (float *)malloc(sizeof(float) * (size_t)(M * kvd));
    float *v = (float *)malloc(sizeof(float) * (size_t)(M * kvd));
    float *att = (float *)malloc(sizeof(float) * (size_t)(M * qd));
    const int64_t kvcap = no_causal ? M : capacity;
    uint16_t *lk = NULL, *lv = NULL;
    if (no_causal) {
        lk = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(nkv * M * hd));
        lv = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(nkv * M * hd));
    }
    float *scratch = (float *)malloc(sizeof(float) * (size_t)(kvcap + 1));
    layer_mul_mat(w, w->wq, xn, qd, H, M, q, var);
    layer_mul_mat(w, w->wk, xn, kvd, H, M, k, var);
    layer_mul_mat(w, w->wv, xn, kvd, H, M, v, var);
    for (int64_t i = 0; i < M * qd; i++) q[i] = orc_bf16_round(q[i]);
    for (int64_t i = 0; i < M * kvd; i++) { k[i] = orc_bf16_round(k[i]); v[i] = orc_bf16_round(v[i]); }
    if (!cfg->no_rope) {
        for (int64_t t = 0; t < M; t++) {
            orc_rope_neox(q + t * qd, nh, hd, pos + (int32_t)t, cfg->rope_theta, cfg->rope_ff);
            orc_rope_neox(k + t * kvd, nkv, hd, pos + (int32_t)t, cfg->rope_theta, cfg->rope_ff);
        }
    }
    uint16_t *kc = no_causal ? lk : k_cache, *vc = no_causal ? lv : v_cache;
    const int64_t base = no_causal ? 0 : pos;
    for (int64_t t = 0; t < M; t++)
        for (int64_t hh = 0; hh < nkv; hh++)
            for (int64_t d = 0; d < hd; d++) {
                kc[(hh * kvcap + base + t) * hd + d] = orc_fp32_to_fp16(k[t * kvd + hh * hd + d]);
                vc[(hh * kvcap + base + t) * hd + d] = orc_fp32_to_fp16(v[t * kvd + hh * hd + d]);
            }
    /* every (token, head) output is formed by one thread with its own scores */
#pragma omp parallel if (M * nh > ORC_ATTN_PAR_MIN)
    {
        float *sc = (float *)malloc(sizeof(float) * (size_t)(kvcap + 1));
#pragma omp for collapse(2) schedule(dynamic, 4)
        for (int64_t t = 0; t < M; t++)
            for (int64_t h = 0; h < nh; h++) {
                const int64_t kv_len = no_causal ? M : pos + t + 1;
                const int64_t gi = h / qpk;
#ifdef ORC_MUL_MAT_HOOK
                if (g_attend_hook) {
                    g_attend_hook(q + t * qd + h * hd, kc + gi * kvcap * hd, vc + gi * kvcap * hd, kv_len, hd, hd,
                                  att + t * qd + h * hd, sc);
                    continue;
                }
#endif
                attend_one(q + t * qd + h * hd, kc + gi * kvcap * hd, vc + gi * kvcap * hd, kv_len, hd,
                           hd, att + t * qd + h * hd, sc);
            }
        free(sc);
    }
    (void)scratch;
    layer_mul_mat(w, w->wo, att, H, qd, M, out, var);
    for (int64_t i = 0; i < M * H; i++) out[i] = orc_bf16_round(out[i]);
    free(q); free(k); free(v); free(att); free(lk); free(lv); free(scratch);
    return 0;
}

/* vcpm_mlp (src/minicpm4.c:432-463): down(bf16(bf16(silu(bf16(gate x))) *
 * bf16(up x))), BF16.  xn: [M][hidden]; out: [M][hidden]. */
void orc_mlp(const orc_cfg *cfg, const orc_layer *w, const float *xn, int64_t M, float *out) {
    const int64_t H = cfg->hidden, F = cfg->ffn;
    const int var = cfg->quant_variant;
    float *g = (float *)malloc(sizeof(float) * (size_t)(M * F));
    float *u = (float *)malloc(sizeof(float) * (size_t)(M * F));
    layer_mul_mat(w, w->wg, xn, F, H, M, g, var);
    layer_mul_mat(w, w->wu, xn, F, H, M, u, var);
    for (int64_t i = 0; i < M * F; i++) {
        float gs = orc_bf16_round(orc_silu(orc_bf16_round(g[i])));
        g[i] = orc_bf16_round(gs * orc_bf16_round(u[i]));
    }
    layer_mul_mat(w, w->wd, g, H, F, M, out, var);
    for (int64_t i = 0; i < M * H; i++) out[i] = orc_bf16_round(out[i]);
    free(g); free(u);
}

/* vcpm_minicpm4_block (src/minicpm4.c:467-532): pre-norm, attention,
 * residual (x + scale*attn, BF16), post-norm, MLP, residual (BF16). */
int orc_minicpm4_block(const orc_cfg *cfg, const orc_layer *w, float *x, int64_t M,
                       uint16_t *k_cache, uint16_t *v_cache, int64_t capacity,
                       int32_t pos, int no_causal) {
    const int64_t H = cfg->hidden;
    float *xn = (float *)malloc(sizeof(float) * (size_t)(M * H));
    float *o = (float *)malloc(sizeof(float) * (size_t)(M * H));
    orc_rms_norm(x, w->g_in, M, H, cfg->eps, xn);
    int rc = orc_attention(cfg, w, xn, M, k_cache, v_cache, capacity, pos, no_causal, o);
    if (rc) { free(xn); free(o); return rc; }
    for (int64_t i = 0; i < M * H; i++) {
        float oa = o[i];
        if (cfg->scale != 1.0f) oa = oa * cfg->scale;
        x[i] = orc_bf16_round(x[i] + oa);
    }
    orc_rms_norm(x, w->g_post, M, H, cfg->eps, xn);
    orc_mlp(cfg, w, xn, M, o);
    for (int64_t i = 0; i < M * H; i++) {
        float da = o[i];
        if (cfg->scale != 1.0f) da = da * cfg->scale;
        x[i] = orc_bf16_round(x[i] + da);
    }
    free(xn); free(o);
    return 0;
}

/* vcpm_minicpm4_forward (src/minicpm4.c:536-572): L causal blocks then the
 * final RMSNorm. */
int orc_minicpm4_forward(const orc_cfg *cfg, const orc_layer *layers, int32_t n_layers,
                         const float *final_norm, float *x, int64_t M,
                         uint16_t **k_caches, uint16_t **v_caches, int64_t capacity,
                         int32_t pos) {
    for (int32_t l = 0; l < n_layers; l++) {
        int rc = orc_minicpm4_block(cfg, &layers[l], x, M, k_caches[l], v_caches[l], capacity, pos, 0);
        if (rc) return rc;
    }
    if (final_norm) {
        float *t = (float *)malloc(sizeof(float) * (size_t)(M * cfg->hidden));
        orc_rms_norm(x, final_norm, M, cfg->hidden, cfg->eps, t);
        memcpy(x, t, sizeof(float) * (size_t)(M * cfg->hidden));
        free(t);
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* LocDiT (src/locdit.c) and the CFM loop (src/gen_step.c, src/cfm_solver.c) */
/* ------------------------------------------------------------------------ */

/* dit_sinusoidal_t_embed (src/locdit.c:163-188). */
void orc_sinusoid_embed(float t, int32_t dim, float *out) {
    const int32_t half = dim / 2;
    const float lmp = logf(10000.0f);
    const float denom = half > 1 ? (float)(half - 1) : 1.0f;
    const float st = orc_bf16_round(t * 1000.0f);
    for (int32_t i = 0; i < half; i++) {
        float e = orc_bf16_round(orc_bf16_round((float)i) * (-lmp / denom));
        float fr = orc_bf16_round(expf(e));
        float a = orc_bf16_round(fr * st);
        out[i] = orc_bf16_round(sinf(a));
        out[half + i] = orc_bf16_round(cosf(a));
    }
}

/* ggml_mul_mat(W, x) + bias, BF16 (dit_add_bias_2d then locdit_bf16_round). */
static void linear_bias_bf16(const uint8_t *w, const float *b, const float *x, int64_t N,
                             int64_t K, int64_t M, float *y, int var) {
    mul_mat_f32_in(w, x, N, K, M, y, var);
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            float v = y[m * N + n];
            if (b) v = v + b[n];
            y[m * N + n] = orc_bf16_round(v);
        }
}

/* vcpm_time_mlp_forward (src/locdit.c:140-159). */
static void time_mlp(const orc_locdit *w, int dt, const float *emb, int64_t H, float *out, int var) {
    const uint8_t *w1 = dt ? w->dt_w1 : w->t_w1, *w2 = dt ? w->dt_w2 : w->t_w2;
    const float *b1 = dt ? w->dt_b1 : w->t_b1, *b2 = dt ? w->dt_b2 : w->t_b2;
    float *h = (float *)malloc(sizeof(float) * (size_t)H);
    linear_bias_bf16(w1, b1, emb, H, H, 1, h, var);
    for (int64_t i = 0; i < H; i++) h[i] = orc_bf16_round(orc_silu(h[i]));
    linear_bias_bf16(w2, b2, h, H, H, 1, out, var);
    free(h);
}

/* vcpm_locdit_forward (src/locdit.c:216-400).  Sequence per branch:
 * [mu(2), t(1), cond(Pc), x(P)]; the reference uses Pc = P.  Blocks are
 * non-causal with positions from 0; the x slice is normed and projected. */
int orc_locdit_forward(const orc_cfg *cfg, const orc_locdit *w, const float *x,
                       const float *cond, int32_t P, int32_t Pc, float t, float dt,
                       const float *mu, float *out) {
    return orc_locdit_forward_states(cfg, w, x, cond, P, Pc, t, dt, mu, out, NULL);
}

/* orc_locdit_forward that also copies the sequence [S][hidden] entering each
 * block and leaving the last one into states[(n_layers + 1)][S][hidden]
 * (when non-NULL), for layer-by-layer comparisons. */
int orc_locdit_forward_states(const orc_cfg *cfg, const orc_locdit *w, const float *x,
                              const float *cond, int32_t P, int32_t Pc, float t, float dt,
                              const float *mu, float *out, float *states) {
    const int64_t H = cfg->hidden, F = w->feat;
    const int64_t S = 3 + Pc + P;
    const int var = cfg->quant_variant;
    float *seq = (float *)calloc((size_t)(S * H), sizeof(float));
    float *emb = (float *)malloc(sizeof(float) * (size_t)H);
    float *tf = (float *)malloc(sizeof(float) * (size_t)H);
    float *dtf = (float *)malloc(sizeof(float) * (size_t)H);
    if (mu) memcpy(seq, mu, sizeof(float) * (size_t)(2 * H));
    orc_sinusoid_embed(t, (int32_t)H, emb);
    time_mlp(w, 0, emb, H, tf, var);
    orc_sinusoid_embed(dt, (int32_t)H, emb);
    time_mlp(w, 1, emb, H, dtf, var);
    for (int64_t i = 0; i < H; i++) seq[2 * H + i] = orc_bf16_round(tf[i] + dtf[i]);
    linear_bias_bf16(w->cond_proj, w->cond_bias, cond, H, F, Pc, seq + 3 * H, var);
    linear_bias_bf16(w->in_proj, w->in_bias, x, H, F, P, seq + (3 + Pc) * H, var);
    for (int32_t l = 0; l < w->n_layers; l++) {
        if (states) memcpy(states + (size_t)l * S * H, seq, sizeof(float) * (size_t)(S * H));
        orc_minicpm4_block(cfg, &w->layers[l], seq, S, NULL, NULL, 0, 0, 1);
    }
    if (states) memcpy(states + (size_t)w->n_layers * S * H, seq, sizeof(float) * (size_t)(S * H));
    float *hn = (float *)malloc(sizeof(float) * (size_t)(P * H));
    orc_rms_norm(seq + (3 + Pc) * H, w->norm, P, H, cfg->eps, hn);
    linear_bias_bf16(w->out_proj, w->out_bias, hn, F, H, P, out, var);
    free(seq); free(emb); free(tf); free(dtf); free(hn);
    return 0;
}

/* vcpm_cfm_sway_t_bf16 (src/cfm_solver.c:27-37).  Pinned by
 * tests/test_cfm_schedule.c:7-18. */
float orc_cfm_sway_t_bf16(int step, int n_steps) {
    if (n_steps <= 0 || step < 0 || step > n_steps) return 0.0f;
    const float base = orc_bf16_round(1.0f - (float)step / (float)n_steps);
    const float half_pi = orc_bf16_round(1.57079632679489661923f);
    const float angle = orc_bf16_round(half_pi * base);
    const float cosine = orc_bf16_round(cosf(angle));
    const float inner = orc_bf16_round(orc_bf16_round(cosine - 1.0f) + base);
    return orc_bf16_round(base + inner);
}

/* Uniform grid t_k = 1 - k/n, BF16, descending like the sway schedule. */
float orc_cfm_uniform_t_bf16(int step, int n_steps) {
    if (n_steps <= 0 || step < 0 || step > n_steps) return 0.0f;
    return orc_bf16_round(1.0f - (float)step / (float)n_steps);
}

/* vcpm_cfm_cfg_zero_star (src/cfm_solver.c:65-93).  Pinned by
 * tests/test_cfm_schedule.c:20-34. */
float orc_cfm_cfg_zero_star(float *negative, const float *positive, int n, float cfg_value) {
    if (!negative || !positive || n <= 0) return 1.0f;
    double dot = 0.0, sq = 0.0;
    for (int i = 0; i < n; i++) {
        const float p = orc_bf16_round(positive[i]);
        const float q = orc_bf16_round(negative[i]);
        dot += orc_bf16_round(p * q);
        sq += orc_bf16_round(q * q);
    }
    const float dot_bf16 = orc_bf16_round((float)dot);
    const float norm_bf16 = orc_bf16_round((float)sq + 1.0e-8f);
    const float st = orc_bf16_round(dot_bf16 / norm_bf16);
    const float cfg_bf16 = orc_bf16_round(cfg_value);
    for (int i = 0; i < n; i++) {
        const float p = orc_bf16_round(positive[i]);
        const float q = orc_bf16_round(negative[i]);
        const float ns = orc_bf16_round(q * st);
        const float gd = orc_bf16_round(p - ns);
        const float gg = orc_bf16_round(cfg_bf16 * gd);
        negative[i] = orc_bf16_round(ns + gg);
    }
    return st;
}

/* vcpm_cfm_zero_star_steps (src/gen_step.c:50-54). */
int orc_cfm_zero_star_steps(int n_steps) {
    if (n_steps <= 1) return 0;
    int z = (int)(((float)n_steps + 1.0f) * 0.04f);
    return z > 1 ? z : 1;
}

/* The time step of Euler step `step` (src/gen_step.c:597-600): dt = bf16(-(t_k - t_{k+1}))
 * on the schedule (0 = sway, 1 = uniform). */
float orc_cfm_step_dt(int step, int n_steps, int schedule) {
    const float t = schedule ? orc_cfm_uniform_t_bf16(step, n_steps) : orc_cfm_sway_t_bf16(step, n_steps);
    const float nt = schedule ? orc_cfm_uniform_t_bf16(step + 1, n_steps) : orc_cfm_sway_t_bf16(step + 1, n_steps);
    return orc_bf16_round(-(t - nt));
}

/* The Euler update of the CFM loop (src/gen_step.c:626-629): x = bf16(x + bf16(dt * v)). */
void orc_cfm_euler_update(float *x, const float *v, int n, float dt) {
    for (int j = 0; j < n; j++) x[j] = orc_bf16_round(x[j] + orc_bf16_round(dt * v[j]));
}

/* The CFM Euler loop of vcpm_gen_step (src/gen_step.c:583-649): with CFG
 * (cfg_value != 1 and mu given, src/gen_step.c:475) the velocities of the
 * cond (mu) and uncond (mu = 0) branches and their CFG-Zero* blend, else the
 * cond velocity alone; then
 * x = bf16(x + bf16(step * v)).  schedule 0 = sway, 1 = uniform.  x is the
 * [P][feat] latent, updated in place. */
int orc_cfm_solve(const orc_cfg *cfg, const orc_locdit *w, float *x, const float *cond,
                  int32_t P, int32_t Pc, const float *mu, int n_steps, float cfg_value,
                  int schedule, int use_zero_star) {
    const int n = P * w->feat;
    float *vc = (float *)malloc(sizeof(float) * (size_t)n);
    float *vu = (float *)malloc(sizeof(float) * (size_t)n);
    const int zs = use_zero_star ? orc_cfm_zero_star_steps(n_steps) : 0;
    const int use_cfg = cfg_value != 1.0f && mu != NULL;   /* src/gen_step.c:475 */
    for (int step = 0; step < n_steps; step++) {
        if (step < zs) continue;
        const float t = schedule ? orc_cfm_uniform_t_bf16(step, n_steps) : orc_cfm_sway_t_bf16(step, n_steps);
        const float dtv = orc_cfm_step_dt(step, n_steps, schedule);
        orc_locdit_forward(cfg, w, x, cond, P, Pc, t, 0.0f, mu, vc);
        if (use_cfg) {
            orc_locdit_forward(cfg, w, x, cond, P, Pc, t, 0.0f, NULL, vu);
            orc_cfm_cfg_zero_star(vu, vc, n, cfg_value);
        } else {
            memcpy(vu, vc, sizeof(float) * (size_t)n);
        }
        orc_cfm_euler_update(x, vu, n, dtv);
    }
    free(vc); free(vu);
    return 0;
}

/* vcpm_locenc_forward (src/locenc.c:44-131): h = in_proj x + bias, F32 (the
 * reference adds no BF16 round here); the special token prepended as row 0
 * (src/locenc.c:65-85); n_layers bidirectional MiniCPM4 blocks with rope from
 * position 0, theta 10000, residual scale 1 (src/locenc.c:87-112); the final
 * RMSNorm (src/locenc.c:114-116); the special token's row is the output
 * (src/locenc.c:118-128), every row when there is no special token. */
int orc_locenc_forward(const orc_cfg *cfg, const orc_locenc *w, const float *x, int32_t P,
                       float *out, float *states) {
    const int64_t H = cfg->hidden, F = w->feat;
    const int64_t off = w->special ? 1 : 0, S = off + P;
    float *seq = (float *)calloc((size_t)(S * H), sizeof(float));
    if (w->special) memcpy(seq, w->special, sizeof(float) * (size_t)H);
    mul_mat_f32_in(w->in_proj, x, H, F, P, seq + off * H, cfg->quant_variant);
    if (w->in_bias)
        for (int64_t r = 0; r < P; r++)
            for (int64_t i = 0; i < H; i++) seq[(off + r) * H + i] = seq[(off + r) * H + i] + w->in_bias[i];
    for (int32_t l = 0; l < w->n_layers; l++) {
        if (states) memcpy(states + (size_t)l * S * H, seq, sizeof(float) * (size_t)(S * H));
        orc_minicpm4_block(cfg, &w->layers[l], seq, S, NULL, NULL, 0, 0, 1);
    }
    if (states) memcpy(states + (size_t)w->n_layers * S * H, seq, sizeof(float) * (size_t)(S * H));
    orc_rms_norm(seq, w->norm, off ? 1 : S, H, cfg->eps, out);
    free(seq);
    return 0;
}

/* vcpm_fsq_quantize (src/fsq.c:16-29): ggml_tanh, ggml_scale by s, ggml_round
 * (roundf: half away from zero), ggml_scale by 1.0f / s.  s <= 0 is the
 * identity (the reference returns x unchanged). */
void orc_fsq_quantize(const float *x, int64_t n, float quant_scale, float *y) {
    const float inv = quant_scale > 0.0f ? 1.0f / quant_scale : 0.0f;
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        if (quant_scale > 0.0f) {
            const float t = tanhf(v);
            const float sc = t * quant_scale;
            v = roundf(sc) * inv;
        }
        y[i] = v;
    }
}
