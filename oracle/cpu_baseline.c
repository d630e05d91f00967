/*
 * cpu_baseline.c -- the timed host-CPU baseline: a SIMD restatement of the
 * ggml CPU backend's Q8_0 path (ggml v0.15.2, not vendored; the reference
 * drives it through vcpm_backend_compute_graph -> ggml_graph_compute_with_ctx,
 * src/ggml_backend.c:557-599, with n_threads = 1 from src/gen_step.c:782).
 *
 * TEST / BENCHMARK INFRASTRUCTURE ONLY (the CPU-baseline leg of the
 * benchmark).  It restates ggml's x86 kernels: quantize_row_q8_0 (AVX2) for
 * the activation, vec_dot_q8_0_q8_0 with per-block int8 products summed to
 * int32 lanes and an fp32 fused multiply-add per block, and ggml's row split
 * of mul_mat over threads.  The glue (norm, rope, attention, SwiGLU) is the
 * scalar oracle, included below, whose cost is negligible next to the GEMVs.
 */
#include <immintrin.h>
#include <omp.h>
#include <stdint.h>
#include <string.h>

#define ORC_MUL_MAT_HOOK 1
#define ORC_ATTN_PAR_MIN 1
#include "vxm_oracle.c"

static int g_threads = 1;

/* the thread count of every parallel loop: the SIMD mul_mat and the glue */
void cb_set_threads(int n) {
    g_threads = n > 0 ? n : 1;
    omp_set_num_threads(g_threads);
}
int cb_get_threads(void) { return g_threads; }

/* ---- AVX2: sum of 32 int8 x int8 products into 8 int32 lanes, as float ---- */
__attribute__((target("avx2,fma,f16c")))
static inline __m256 dot32_avx2(const int8_t *a, const int8_t *b) {
    const __m256i qa = _mm256_loadu_si256((const __m256i *)a);
    const __m256i qb = _mm256_loadu_si256((const __m256i *)b);
    const __m256i ax = _mm256_sign_epi8(qa, qa);
    const __m256i sy = _mm256_sign_epi8(qb, qa);
    const __m256i p16 = _mm256_maddubs_epi16(ax, sy);
    const __m256i p32 = _mm256_madd_epi16(p16, _mm256_set1_epi16(1));
    return _mm256_cvtepi32_ps(p32);
}

__attribute__((target("avx2,fma,f16c")))
static float vec_dot_q8_0_avx2(int64_t nb, const uint8_t *w, const uint8_t *x) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *wb = w + b * 34, *xb = x + b * 34;
        uint16_t dw, dx; memcpy(&dw, wb, 2); memcpy(&dx, xb, 2);
        const __m256 d = _mm256_set1_ps(_cvtsh_ss(dw) * _cvtsh_ss(dx));
        acc = _mm256_fmadd_ps(d, dot32_avx2((const int8_t *)(wb + 2), (const int8_t *)(xb + 2)), acc);
    }
    __m128 lo = _mm256_castps256_ps128(acc), hi = _mm256_extractf128_ps(acc, 1);
    lo = _mm_add_ps(lo, hi);
    lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
    lo = _mm_add_ss(lo, _mm_movehdup_ps(lo));
    return _mm_cvtss_f32(lo);
}

/* ---- AVX512-VNNI (256-bit forms): dpbusd on |a| and sign(b, a) ---- */
__attribute__((target("avx2,fma,f16c,avx512f,avx512vl,avx512vnni")))
static float vec_dot_q8_0_vnni(int64_t nb, const uint8_t *w, const uint8_t *x) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *wb = w + b * 34, *xb = x + b * 34;
        uint16_t dw, dx; memcpy(&dw, wb, 2); memcpy(&dx, xb, 2);
        const __m256 d = _mm256_set1_ps(_cvtsh_ss(dw) * _cvtsh_ss(dx));
        const __m256i qa = _mm256_loadu_si256((const __m256i *)(wb + 2));
        const __m256i qb = _mm256_loadu_si256((const __m256i *)(xb + 2));
        const __m256i ax = _mm256_sign_epi8(qa, qa);
        const __m256i sy = _mm256_sign_epi8(qb, qa);
        const __m256i p = _mm256_dpbusd_epi32(_mm256_setzero_si256(), ax, sy);
        acc = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(p), acc);
    }
    __m128 lo = _mm256_castps256_ps128(acc), hi = _mm256_extractf128_ps(acc, 1);
    lo = _mm_add_ps(lo, hi);
    lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
    lo = _mm_add_ss(lo, _mm_movehdup_ps(lo));
    return _mm_cvtss_f32(lo);
}

typedef float (*dot_fn)(int64_t, const uint8_t *, const uint8_t *);

static dot_fn pick_dot(void) {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl")) return vec_dot_q8_0_vnni;
    return vec_dot_q8_0_avx2;
}

/* 1 = AVX512-VNNI, 0 = AVX2 */
int cb_isa(void) { return pick_dot() == vec_dot_q8_0_vnni; }

/* ggml_compute_forward_mul_mat for Q8_0 src0: rows of W split over threads,
 * one vec_dot per (row, column of x).  y[m*N + n]. */
void cb_mul_mat_q8_0(const uint8_t *w, const uint8_t *xq, int64_t N, int64_t K, int64_t M, float *y) {
    const int64_t nb = K / 32, rb = nb * 34;
    dot_fn dot = pick_dot();
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (int64_t n = 0; n < N; n++)
        for (int64_t m = 0; m < M; m++) y[m * N + n] = dot(nb, w + n * rb, xq + m * rb);
}

/* Hook used by the included oracle glue: quantize x rows (x86 variant) then
 * the SIMD mul_mat. */
static void cb_mul_mat_f32_in(const uint8_t *w, const float *x, int64_t N, int64_t K, int64_t M,
                              float *y, int variant) {
    const int64_t rb = K / 32 * 34;
    uint8_t *xq = (uint8_t *)malloc((size_t)(M * rb));
    orc_quantize_rows_q8_0(x, xq, M, K, variant);
    cb_mul_mat_q8_0(w, xq, N, K, M, y);
    free(xq);
}

/* One query head's attention over an f16 cache as ggml-cpu computes it with
 * F16C + FMA: f16 keys widened 8 at a time for the scores, the softmax of
 * ggml_soft_max_ext (max, expf, a double sum), then P.V accumulated row by row
 * over the f16 values.  hd % 8 == 0. */
__attribute__((target("avx2,fma,f16c")))
static void attend_one_f16c(const float *q, const uint16_t *k, const uint16_t *v, int64_t kv_len, int64_t hd,
                            int64_t stride, float *out, float *scratch) {
    const float sc = 1.0f / sqrtf((float)hd);
    float mx = -INFINITY;
    for (int64_t j = 0; j < kv_len; j++) {
        __m256 acc = _mm256_setzero_ps();
        for (int64_t d = 0; d < hd; d += 8) {
            const __m256 kf = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(k + j * stride + d)));
            acc = _mm256_fmadd_ps(kf, _mm256_loadu_ps(q + d), acc);
        }
        __m128 lo = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
        lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
        lo = _mm_add_ss(lo, _mm_movehdup_ps(lo));
        const float s = _mm_cvtss_f32(lo) * sc;
        scratch[j] = s;
        if (s > mx) mx = s;
    }
    double sum = 0.0;
    for (int64_t j = 0; j < kv_len; j++) {
        const float e = expf(scratch[j] - mx);
        scratch[j] = e;
        sum += (double)e;
    }
    const float inv = (float)(1.0 / sum);
    for (int64_t d = 0; d < hd; d++) out[d] = 0.0f;
    for (int64_t j = 0; j < kv_len; j++) {
        const __m256 p = _mm256_set1_ps(scratch[j] * inv);
        for (int64_t d = 0; d < hd; d += 8) {
            const __m256 vf = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(v + j * stride + d)));
            _mm256_storeu_ps(out + d, _mm256_fmadd_ps(p, vf, _mm256_loadu_ps(out + d)));
        }
    }
}

int cb_minicpm4_forward(const orc_cfg *cfg, const orc_layer *layers, int32_t n_layers,
                        const float *final_norm, float *x, int64_t M, uint16_t **k_caches,
                        uint16_t **v_caches, int64_t capacity, int32_t pos) {
    g_mul_mat_hook = cb_mul_mat_f32_in;
    if (cfg->head_dim % 8 == 0) g_attend_hook = attend_one_f16c;
    int rc = orc_minicpm4_forward(cfg, layers, n_layers, final_norm, x, M, k_caches, v_caches,
                                  capacity, pos);
    g_mul_mat_hook = NULL;
    g_attend_hook = NULL;
    return rc;
}
