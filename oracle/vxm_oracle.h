/*
 * vxm_oracle.h -- CPU oracle for the Q8_0 matmul hot path of the VoxCPM2 C
 * runtime (stevenke1981/voxcpm-cpp).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code.  Only the test suite, the smoke check and the CPU-baseline
 * leg of the benchmark use it, and only as the checker (or, for the baseline,
 * as the timed CPU restatement).
 *
 * The arithmetic of the path lives in ggml v0.15.2 (a third-party dependency
 * fetched by CMake FetchContent at CMakeLists.txt:54-70 and absent offline).
 * Every function below restates the published ggml algorithm or the
 * reference's own graph construction; each cites the reference call site it
 * follows.  Functions whose exact ggml behaviour cannot be pinned without
 * ggml itself are marked "parity unpinned" where they are defined.
 */
#ifndef VXM_ORACLE_H
#define VXM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK8_0 32
#define ORC_Q8_0_BLOCK_BYTES 34

/* Activation quantizer variants (see orc_quantize_row_q8_0). */
#define ORC_QUANT_REF 0   /* ggml quantize_row_q8_0_ref: id = 1/d, roundf()        */
#define ORC_QUANT_X86 1   /* ggml x86 SIMD quantize_row_q8_0: id = 127/amax, RNE    */

/* ---- number formats ---- */
uint16_t orc_fp32_to_fp16(float f);
float    orc_fp16_to_fp32(uint16_t h);
float    orc_bf16_round(float f);
void     orc_fp32_to_fp16_n(const float *x, uint16_t *h, int64_t n);
void     orc_fp16_to_fp32_n(const uint16_t *h, float *x, int64_t n);
void     orc_bf16_round_n(const float *x, float *y, int64_t n);

/* ---- Q8_0 blocks ---- */
void orc_quantize_row_q8_0(const float *x, uint8_t *y, int64_t k, int variant);
void orc_quantize_rows_q8_0(const float *x, uint8_t *y, int64_t rows, int64_t k, int variant);
void orc_dequantize_row_q8_0(const uint8_t *y, float *x, int64_t k);

/* int32 per-block dot sums: out[(m*N + n)*nb + b] */
void orc_block_dots_q8_0(const uint8_t *w, const uint8_t *xq, int64_t N, int64_t K,
                         int64_t M, int32_t *out);
/* y[m*N + n] = sum_b fp32(sumi_b) * (d_w * d_x), accumulated sequentially in fp32 */
void orc_mul_mat_q8_0(const uint8_t *w, const uint8_t *xq, int64_t N, int64_t K,
                      int64_t M, float *y);
/* same sum accumulated in fp64 (used to bound the fp32 rounding of any order) */
void orc_mul_mat_q8_0_f64(const uint8_t *w, const uint8_t *xq, int64_t N, int64_t K,
                          int64_t M, double *y);

/* ---- MiniCPM4 block pieces ---- */
void  orc_rms_norm(const float *x, const float *g, int64_t rows, int64_t n, float eps, float *y);
void  orc_rope_neox(float *x, int64_t n_heads, int64_t head_dim, int32_t pos,
                    float theta_base, const float *freq_factors);
float orc_silu(float x);

typedef struct orc_layer {
    const void *wq, *wk, *wv, *wo, *wg, *wu, *wd;      /* GGUF Q8_0 rows (or F32 rows) */
    const float *g_in, *g_post;                         /* RMSNorm gains  */
    int32_t wtype;                                      /* 0 = Q8_0, 1 = F32 [N][K] */
} orc_layer;

typedef struct orc_cfg {
    int32_t hidden, n_heads, n_kv_heads, head_dim, ffn;
    float   eps;
    float   rope_theta;
    int32_t no_rope;
    float   scale;                 /* DeepNorm residual scale (1 = none) */
    const float *rope_ff;          /* head_dim/2 frequency factors or NULL */
    int32_t quant_variant;         /* ORC_QUANT_* used for activations */
} orc_cfg;

int  orc_attention(const orc_cfg *cfg, const orc_layer *w, const float *xn, int64_t M,
                   uint16_t *k_cache, uint16_t *v_cache, int64_t capacity, int32_t pos,
                   int no_causal, float *out);
void orc_mlp(const orc_cfg *cfg, const orc_layer *w, const float *xn, int64_t M, float *out);
/* f16 KV cache for one layer: k and v are [n_kv_heads][capacity][head_dim]. */
int orc_minicpm4_block(const orc_cfg *cfg, const orc_layer *w, float *x, int64_t M,
                       uint16_t *k_cache, uint16_t *v_cache, int64_t capacity,
                       int32_t pos, int no_causal);
int orc_minicpm4_forward(const orc_cfg *cfg, const orc_layer *layers, int32_t n_layers,
                         const float *final_norm, float *x, int64_t M,
                         uint16_t **k_caches, uint16_t **v_caches, int64_t capacity,
                         int32_t pos);

/* ---- LocDiT + CFM ---- */
typedef struct orc_locdit {
    const orc_layer *layers;
    int32_t n_layers;
    const uint8_t *in_proj;  const float *in_bias;     /* hidden x feat */
    const uint8_t *cond_proj; const float *cond_bias;  /* hidden x feat */
    const uint8_t *out_proj; const float *out_bias;    /* feat x hidden */
    const float   *norm;                               /* hidden        */
    const uint8_t *t_w1, *t_w2, *dt_w1, *dt_w2;        /* hidden x hidden */
    const float   *t_b1, *t_b2, *dt_b1, *dt_b2;
    int32_t feat;
} orc_locdit;

void  orc_sinusoid_embed(float t, int32_t dim, float *out);
int   orc_locdit_forward(const orc_cfg *cfg, const orc_locdit *w, const float *x,
                         const float *cond, int32_t P, int32_t Pc, float t, float dt,
                         const float *mu, float *out);
int   orc_locdit_forward_states(const orc_cfg *cfg, const orc_locdit *w, const float *x,
                                const float *cond, int32_t P, int32_t Pc, float t, float dt,
                                const float *mu, float *out, float *states);
float orc_cfm_sway_t_bf16(int step, int n_steps);
float orc_cfm_uniform_t_bf16(int step, int n_steps);
float orc_cfm_cfg_zero_star(float *negative, const float *positive, int n, float cfg_value);
int   orc_cfm_zero_star_steps(int n_steps);
float orc_cfm_step_dt(int step, int n_steps, int schedule);
void  orc_cfm_euler_update(float *x, const float *v, int n, float dt);
int   orc_cfm_solve(const orc_cfg *cfg, const orc_locdit *w, float *x, const float *cond,
                    int32_t P, int32_t Pc, const float *mu, int n_steps, float cfg_value,
                    int schedule, int use_zero_star);

/* ---- LocEnc, FSQ ---- */
typedef struct orc_locenc {
    const orc_layer *layers;
    int32_t n_layers;
    const uint8_t *in_proj;  const float *in_bias;     /* hidden x feat (Q8_0 rows) */
    const float   *special;                            /* hidden, or NULL */
    const float   *norm;                               /* hidden */
    int32_t feat;
} orc_locenc;

/* out: the special token's row [hidden], or every row [P][hidden] without
 * one; states (optional): the sequence entering each block and leaving the
 * last, [(n_layers + 1)][P + has_special][hidden]. */
int  orc_locenc_forward(const orc_cfg *cfg, const orc_locenc *w, const float *x, int32_t P,
                        float *out, float *states);
void orc_fsq_quantize(const float *x, int64_t n, float quant_scale, float *y);

#ifdef __cplusplus
}
#endif
#endif
