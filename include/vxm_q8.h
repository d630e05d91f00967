/*
 * vxm_q8.h -- C ABI of the MI355X (gfx950) Q8_0 matmul path for the VoxCPM2
 * C runtime (stevenke1981/voxcpm-cpp).
 *
 * The reference executes every projection as ggml_mul_mat(W_q8_0, x_f32)
 * inside graphs run by vcpm_backend_compute_graph (src/ggml_backend.c:557-599).
 * This library replaces that arithmetic with hand-written HIP kernels behind
 * plain C entry points: no torch types, no C++ exceptions, int status codes.
 *
 * Conventions
 *  - Every entry point returns VXM_OK (0) or a vxm_status code; the message of
 *    the last failure on a context is returned by vxm_last_error().
 *  - Pointers named *_dev are device pointers (from vxm_malloc, or any HIP
 *    allocation on the context's device).  Host buffers are caller-owned.
 *  - Compute calls are asynchronous and ordered on the context's stream
 *    (vxm_get_stream); nothing synchronises the host except vxm_sync and the
 *    vxm_memcpy_* / upload / download calls, which are the host-boundary
 *    points the reference API implies (src/ggml_backend.c:356-457).
 *  - Activation matrices use the ggml layout of a [K, M] tensor: M rows of K
 *    contiguous floats, row m at x + m*K.  Outputs are [N, M]: y[m*N + n].
 *  - A quantized activation is two device arrays: xq int8 [M][K] and xd fp16
 *    bits [M][K/32] (the scale of block b of row m at xd[m*(K/32) + b]).
 *  - A context and the objects made on it are used by one host thread at a
 *    time (as a reference generation state is); separate contexts may be used
 *    from separate threads.
 */
#ifndef VXM_Q8_H
#define VXM_Q8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same values as vcpm_status (include/voxcpm.h:14-23). */
typedef enum vxm_status {
    VXM_OK = 0,
    VXM_ERR_INVALID_ARG = 1,
    VXM_ERR_IO = 2,
    VXM_ERR_MODEL_FORMAT = 3,
    VXM_ERR_UNSUPPORTED_ARCH = 4,
    VXM_ERR_BACKEND = 5,
    VXM_ERR_OOM = 6,
    VXM_ERR_NOT_IMPLEMENTED = 7
} vxm_status;

/* Activation quantizer variants (ggml-cpu quantize_row_q8_0 on x86 vs
 * quantize_row_q8_0_ref); the weights of a GGUF file use the _ref rule. */
#define VXM_QUANT_REF 0
#define VXM_QUANT_X86 1

/* Kernel path for vxm_mul_mat_*: AUTO picks by M. */
#define VXM_PATH_AUTO 0
#define VXM_PATH_GEMV 1   /* weight-streaming GEMV, any M (loops over rows of x) */
#define VXM_PATH_MFMA 2   /* int8 MFMA: register-fed small-M kernel up to 64 rows
                           * (N % 16 == 0, K % 256 == 0), else the LDS-tiled GEMM */
#define VXM_PATH_MFMA_TILED 3 /* the LDS-tiled MFMA GEMM for every M            */

typedef struct vxm_ctx vxm_ctx;
typedef struct vxm_weight vxm_weight;

/* ---- context -------------------------------------------------------------
 * Replaces vcpm_backend_init / vcpm_backend_free (src/ggml_backend.c:49-140)
 * for this path: one context = one device + one stream. */
int         vxm_open(int device, vxm_ctx **out);
int         vxm_close(vxm_ctx *ctx);
int         vxm_sync(vxm_ctx *ctx);
void       *vxm_get_stream(vxm_ctx *ctx);
const char *vxm_last_error(const vxm_ctx *ctx);
int         vxm_set_quant_variant(vxm_ctx *ctx, int variant);
int         vxm_set_path(vxm_ctx *ctx, int path);

/* HIP graph capture of the context's stream: no counterpart in the reference
 * (its host re-issues every graph each step, src/ggml_backend.c:557-599).  For
 * callers that replay one fixed sequence of vxm_* calls with new contents in
 * the same device buffers (matmuls, norms, an encoder pass).  Between begin
 * and end the calls on the context are recorded, not run; vxm_graph_launch
 * replays the recording on the context's stream.  Host scalars (a decode
 * position, a time step) are recorded with the values they had.  Run the
 * sequence once eagerly first: a call that would have to grow a scratch
 * buffer or set up a single-launch kernel's buffers (and so allocate and
 * synchronise) fails under capture with VXM_ERR_INVALID_ARG.
 * vxm_locdit_forward stages host-computed time embeddings and cannot be
 * captured; vxm_cfm_solve records and replays its own Euler loop.  Every tag
 * a kernel compares lives in device memory, so every replay is exact. */
typedef struct vxm_graph vxm_graph;
int vxm_capture_begin(vxm_ctx *ctx);
int vxm_capture_end(vxm_ctx *ctx, vxm_graph **out);
int vxm_graph_launch(vxm_ctx *ctx, const vxm_graph *g);
int vxm_graph_free(vxm_graph *g);

/* Device memory and host-boundary copies (ggml_backend_tensor_set/get,
 * src/ggml_backend.c:356-380,422-457).  The copies return when complete.  A
 * device-to-host copy of at most 64 KiB from a 16-byte aligned source (a
 * decode step's hidden state) is written by a copy kernel on the context's
 * stream into pinned host staging, which the call polls briefly before it
 * falls back to synchronising the stream. */
int vxm_malloc(vxm_ctx *ctx, size_t bytes, void **out_dev);
int vxm_free(vxm_ctx *ctx, void *dev);
int vxm_memcpy_h2d(vxm_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes);
int vxm_memcpy_d2h(vxm_ctx *ctx, void *dst_host, const void *src_dev, size_t bytes);

/* ---- Q8_0 weights --------------------------------------------------------
 * Upload of a GGUF Q8_0 tensor with ne = [k, n_rows] (34-byte blocks: fp16 d,
 * int8 qs[32]; rows of k/32 blocks), as vcpm_model_offload does
 * (src/model_loader.c:665-700).  The device copy is repacked (quants and
 * scales split) but vxm_download_q8_0 re-emits the exact GGUF bytes. */
int     vxm_upload_q8_0(vxm_ctx *ctx, const void *gguf_rows, int64_t n_rows, int64_t k,
                        vxm_weight **out);
int     vxm_download_q8_0(vxm_ctx *ctx, const vxm_weight *w, void *gguf_rows);
int     vxm_weight_free(vxm_ctx *ctx, vxm_weight *w);
int64_t vxm_weight_rows(const vxm_weight *w);
int64_t vxm_weight_cols(const vxm_weight *w);

/* ---- the matmul (ggml_mul_mat on Q8_0, src/projections.h:24-29) ---------- */
/* x (fp32 [M][K]) -> Q8_0 activation, per block d = amax/127. */
int vxm_quantize_q8_0(vxm_ctx *ctx, const float *x_dev, int64_t M, int64_t K, int variant,
                      int8_t *xq_dev, uint16_t *xd_dev);
/* y = W . x with x quantized internally (ggml_mul_mat(W, x) semantics). */
int vxm_mul_mat_q8_0(vxm_ctx *ctx, const vxm_weight *w, const float *x_dev, int64_t M,
                     float *y_dev);
/* y = W . x for an already quantized activation. */
int vxm_mul_mat_q8_0_q8_0(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq_dev,
                          const uint16_t *xd_dev, int64_t M, float *y_dev);
/* n independent products y_i = W_i . x_i of already quantized activations
 * (M rows each, every W_i of the same K) in one launch per 64 products.  They
 * are the mul_mat nodes of one reference graph that share no dependency (the
 * q/k/v projections, src/minicpm4.c:270-279; gate and up, src/minicpm4.c:
 * 441-458), which ggml runs one after another inside vcpm_backend_compute_graph
 * (src/ggml_backend.c:557-599).  Every y_i is bit-identical to
 * vxm_mul_mat_q8_0_q8_0's for the same operands.  Shapes that the chunked GEMV
 * does not take (M >= 8, K / 1024 not in {1, 2, 4, 6}) run one product per
 * launch on the kernel vxm_mul_mat_q8_0_q8_0 picks. */
int vxm_mul_mat_q8_0_q8_0_multi(vxm_ctx *ctx, int32_t n, const vxm_weight *const *w,
                                const int8_t *const *xq_dev, const uint16_t *const *xd_dev, int64_t M,
                                float *const *y_dev);
/* Measurement helper, no counterpart in the reference: reads n <= 128 device
 * ranges (16-byte aligned, sizes multiples of 16 B) once, in one launch, with
 * the GEMV's 128-bit streaming loads, and writes one XOR of 32-bit words per
 * wave to sink_dev, which holds vxm_stream_read_sink_words(n, bytes) words
 * (their XOR is the XOR of every word read).  The HBM read floor of a launch
 * that moves the same bytes. */
int vxm_stream_read(vxm_ctx *ctx, int32_t n, const void *const *ranges_dev, const int64_t *bytes,
                    uint32_t *sink_dev);
int64_t vxm_stream_read_sink_words(int32_t n, const int64_t *bytes);
/* vxm_mul_mat_q8_0 without any allocation: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * kernels, plans and results as vxm_mul_mat_q8_0; the quantized activation
 * and the K-split partials live in a fixed device array of
 * vxm_noalloc_scratch_bytes() per device (48 MiB 64 KiB), held until the
 * process ends.  A product whose quantized activation exceeds 32 MiB, or whose
 * K-split plan needs more than the array's 16 MiB of partial words (for
 * example 2048 x 6144 at M = 520, which vxm_mul_mat_q8_0 splits 3 ways), is
 * rejected with VXM_ERR_INVALID_ARG, never run on another plan.  All
 * calls on one device share the array: calls that overlap on a device (other
 * streams or threads) race. */
int vxm_mul_mat_q8_0_noalloc(vxm_ctx *ctx, const vxm_weight *w, const float *x_dev, int64_t M,
                             float *y_dev);
size_t vxm_noalloc_scratch_bytes(void);
/* Debug: int32 per-block sums of vec_dot_q8_0_q8_0, out[(m*N + n)*(K/32) + b]. */
int vxm_block_dots_q8_0(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq_dev,
                        const uint16_t *xd_dev, int64_t M, int32_t *out_dev);

/* ---- block ops -----------------------------------------------------------
 * vcpm_rms_norm (src/minicpm4.c:132-152) on rows x [rows][n]: y = BF16(BF16(
 * x / sqrt(mean(x^2) + eps)) * gain).  gain may be NULL (plain ggml_rms_norm
 * + BF16).  If xq/xd are non-NULL the output is also quantized to Q8_0 with
 * the context's activation rule (the input of the next ggml_mul_mat). */
int vxm_rms_norm(vxm_ctx *ctx, const float *x_dev, const float *gain_dev, int64_t rows, int64_t n,
                 float eps, float *y_dev, int8_t *xq_dev, uint16_t *xd_dev);

/* ---- MiniCPM4 stack ------------------------------------------------------
 * Mirrors vcpm_minicpm4_config (src/minicpm4.h:14-27). */
typedef struct vxm_minicpm4_config {
    int32_t hidden_size;
    int32_t n_layers;
    int32_t n_heads;
    int32_t n_kv_heads;
    int32_t intermediate_size;
    int32_t head_dim;
    float   rms_norm_eps;
    int32_t rope_theta;
    int32_t no_rope;          /* 1 for the residual LM (RALM), src/ralm.c:15-29 */
    float   scale_depth;      /* DeepNorm: residual scale = scale_depth/sqrt(n_layers) if > 0 */
    /* head_dim/2 rope frequency factors (host memory), or NULL for the
     * reference rule: the VoxCPM2 LongRoPE short factors when head_dim == 128
     * (src/minicpm4.c:49-66,183-190), none otherwise. */
    const float *rope_freq_factors;
} vxm_minicpm4_config;

/* One block's weights in host memory: GGUF Q8_0 rows for the seven
 * projections (vcpm_layer_weights, src/transformer.h:27-48) and F32 gains. */
typedef struct vxm_layer_weights_q8_0 {
    const void  *q_proj, *k_proj, *v_proj, *o_proj, *gate_proj, *up_proj, *down_proj;
    const float *input_layernorm, *post_attention_layernorm;
} vxm_layer_weights_q8_0;

typedef struct vxm_minicpm4 vxm_minicpm4;
typedef struct vxm_kv_cache vxm_kv_cache;

/* Uploads cfg->n_layers blocks (+ optional final norm, host F32 [hidden]). */
int vxm_minicpm4_create(vxm_ctx *ctx, const vxm_minicpm4_config *cfg,
                        const vxm_layer_weights_q8_0 *layers, const float *final_norm,
                        vxm_minicpm4 **out);
int vxm_minicpm4_free(vxm_minicpm4 *m);

/* f16 KV cache (the reference keeps F32, src/minicpm4.c:93-122): per layer,
 * K and V are [n_kv_heads][capacity][head_dim]. */
int     vxm_kv_cache_create(vxm_ctx *ctx, int32_t n_layers, int32_t n_kv_heads, int32_t head_dim,
                            int32_t capacity, vxm_kv_cache **out);
int     vxm_kv_cache_free(vxm_kv_cache *kv);
int     vxm_kv_cache_reset(vxm_kv_cache *kv);                 /* n_used = 0 (vcpm_gen_reset) */
int     vxm_kv_cache_set_used(vxm_kv_cache *kv, int32_t n_used);
int32_t vxm_kv_cache_used(const vxm_kv_cache *kv);
int     vxm_kv_cache_layer(vxm_kv_cache *kv, int32_t layer, uint16_t **k_dev, uint16_t **v_dev);

/* vcpm_minicpm4_block (src/minicpm4.c:467-532) for one layer, in place on
 * x [n_tokens][hidden].  Causal: tokens take positions pos.. and are appended
 * to the cache at the same rows.  no_causal: attention over the n_tokens
 * fresh tokens only (LocDiT/LocEnc use), positions from pos, cache untouched. */
int vxm_minicpm4_block(vxm_minicpm4 *m, vxm_kv_cache *kv, int32_t layer, float *x_dev,
                       int64_t n_tokens, int32_t pos, int no_causal);
/* vcpm_minicpm4_forward (src/minicpm4.c:536-572): all layers (causal) and
 * the final norm, in place on x [n_tokens][hidden]; positions and cache rows
 * pos..pos+n_tokens-1; sets the cache's n_used to pos + n_tokens. */
int vxm_minicpm4_forward(vxm_minicpm4 *m, vxm_kv_cache *kv, float *x_dev, int64_t n_tokens,
                         int32_t pos);

/* Decode (n_tokens == 1) strategy of vxm_minicpm4_forward:
 * VXM_DECODE_AUTO picks the fastest available, VXM_DECODE_KERNELS runs one
 * kernel per op, VXM_DECODE_PERSISTENT runs the whole stack in one launch
 * (all 256 workgroups resident).  No reference counterpart (ggml has one
 * graph path). */
#define VXM_DECODE_AUTO 0
#define VXM_DECODE_KERNELS 1
#define VXM_DECODE_PERSISTENT 2
int vxm_minicpm4_set_decode_mode(vxm_minicpm4 *m, int mode);
/* Synchronises the context's stream and reports a device-side failure of the
 * persistent decode (a workgroup that timed out waiting for its inputs) as
 * VXM_ERR_BACKEND, then clears it.  Decode calls themselves never block. */
int vxm_minicpm4_check(vxm_minicpm4 *m);
/* Debug read-back of every layer, as the reference's GPU path reads back every
 * graph node (src/ggml_backend.c:422-457) and VCPM_DEBUG_SHAPES dumps named
 * tensors (src/debug_dump.h:18-43).  With a non-null dump_dev, each later
 * vxm_minicpm4_forward writes the input of every layer l (after the previous
 * layer's residual) to dump_dev + l * n_tokens * hidden and the last layer's
 * output before the final norm to dump_dev + n_layers * n_tokens * hidden:
 * (n_layers + 1) * n_tokens * hidden floats, on every decode strategy (the
 * single launch writes them from workgroup 0).  Null turns it off. */
int vxm_minicpm4_set_layer_dump(vxm_minicpm4 *m, float *dump_dev);
/* Test hooks of the single-launch decode, no reference counterpart.  Its words
 * carry a 20-bit launch epoch kept in device memory (advanced by each launch,
 * so HIP graph replays tag anew); when it wraps, the launch resets every
 * exchange word.  set: the epoch of the next launch (1 .. 2^20 - 1; needs one
 * earlier single-launch decode on the model).  Both synchronise. */
int vxm_minicpm4_set_decode_epoch(vxm_minicpm4 *m, uint32_t epoch);
int vxm_minicpm4_decode_epoch(vxm_minicpm4 *m, uint32_t *epoch);

/* ---- LocDiT and the CFM solver -------------------------------------------
 * Mirrors vcpm_locdit_config (src/locdit.h:26-34) plus the projection widths. */
typedef struct vxm_locdit_config {
    int32_t hidden_size;
    int32_t n_layers;
    int32_t n_heads;
    int32_t n_kv_heads;
    int32_t intermediate_size;
    int32_t head_dim;
    int32_t feat_dim;         /* latent width of x and of the velocity (in_proj / out_proj) */
    int32_t cond_dim;         /* width of the cond tokens (cond_proj) */
    float   rms_norm_eps;
    int32_t rope_theta;       /* the reference uses 10000 (src/locdit.c:351) */
    /* head_dim/2 rope factors (host), or NULL for the MiniCPM4 rule (LongRoPE
     * short factors when head_dim == 128, none otherwise) */
    const float *rope_freq_factors;
} vxm_locdit_config;

/* vcpm_locdit_weights (src/locdit.h:41-68): GGUF Q8_0 rows and F32 vectors in host
 * memory.  Biases may be NULL. */
typedef struct vxm_locdit_weights_q8_0 {
    const vxm_layer_weights_q8_0 *layers;                   /* n_layers blocks */
    const void  *in_proj;   const float *in_bias;          /* [hidden][feat_dim]  */
    const void  *cond_proj; const float *cond_bias;        /* [hidden][cond_dim]  */
    const void  *out_proj;  const float *out_bias;         /* [feat_dim][hidden]  */
    const float *norm;                                     /* [hidden]            */
    const void  *t_w1, *t_w2, *dt_w1, *dt_w2;              /* [hidden][hidden]    */
    const float *t_b1, *t_b2, *dt_b1, *dt_b2;
} vxm_locdit_weights_q8_0;

typedef struct vxm_locdit vxm_locdit;

int vxm_locdit_create(vxm_ctx *ctx, const vxm_locdit_config *cfg, const vxm_locdit_weights_q8_0 *w,
                      vxm_locdit **out);
int vxm_locdit_free(vxm_locdit *m);

/* vcpm_locdit_forward (src/locdit.c:216-400): velocity of x for one branch.
 * x [P][feat_dim], cond [Pc][cond_dim], mu [2][hidden] or NULL (the
 * unconditional branch: zero rows), out [P][feat_dim]; t and dt are the
 * timestep scalars.  Sequence [mu(2), t(1), cond(Pc), x(P)], 12 non-causal
 * rope blocks from position 0, RMSNorm of the x rows, out_proj.  The
 * reference uses Pc == P. */
int vxm_locdit_forward(vxm_locdit *m, const float *x_dev, const float *cond_dev, int32_t P, int32_t Pc,
                       float t, float dt, const float *mu_dev, float *out_dev);

/* The CFM Euler loop of vcpm_gen_step (src/gen_step.c:583-649), on the
 * device with no host synchronisation: for each step past the zero-init
 * steps (when use_zero_star), t from the schedule, the conditional (mu) and
 * unconditional (no mu) velocities in ONE batch of 2 x (3 + Pc + P) rows,
 * CFG-Zero* (vcpm_cfm_cfg_zero_star, src/cfm_solver.c:65-93) and
 * x = bf16(x + bf16(dt * v)).  Without CFG (cfg_value == 1 or mu == NULL,
 * src/gen_step.c:475) only the conditional branch runs.  x [P][feat_dim] is
 * updated in place.  Where the single-launch blocks apply (see
 * vxm_locdit_set_block_mode) and feat_dim is 64 with at most 64 live steps,
 * every step -- its rows' assembly, the blocks, the final norm, out_proj,
 * CFG-Zero* and the Euler step -- runs inside one launch.
 * The first call with a given set of arguments (x, cond and mu pointers, P, Pc,
 * n_steps, cfg_value, schedule, use_zero_star) runs the loop eagerly; the
 * second records it as a HIP graph and every later call with the same
 * arguments (and the same internal buffers) replays that graph, reading the
 * current contents of x, cond and mu.  The steps' time rows (time_mlp and
 * delta_time_mlp, src/locdit.c:140-159) depend only on the steps' t: a solve
 * whose t are those of the model's previous time rows (every patch of an
 * utterance) reuses them.  Results are identical either way. */
#define VXM_CFM_SWAY 0      /* vcpm_cfm_sway_t_bf16 (src/cfm_solver.c:27-37) */
#define VXM_CFM_UNIFORM 1   /* t = bf16(1 - step / n_steps) */
int vxm_cfm_solve(vxm_locdit *m, float *x_dev, const float *cond_dev, int32_t P, int32_t Pc,
                  const float *mu_dev, int32_t n_steps, float cfg_value, int32_t schedule,
                  int32_t use_zero_star);

/* Block strategy of vxm_locdit_forward and vxm_cfm_solve (the VXM_DECODE_*
 * values).  The persistent kernel runs every block of an evaluation in one
 * launch; it supports hidden 1024, FFN 4096, 16 query heads of (16 kv x 64)
 * or (2 kv x 128), at most 48 rows in segments of at most 32, on 256 CUs.
 * AUTO takes it wherever it applies (it measured faster than block-by-block
 * launches at both layouts) and launches block by block otherwise; KERNELS
 * always launches block by block;
 * PERSISTENT fails with VXM_ERR_NOT_IMPLEMENTED where the kernel does not
 * apply.  No reference counterpart (ggml evaluates one graph per call). */
int vxm_locdit_set_block_mode(vxm_locdit *m, int mode);
/* Synchronises the context's stream and reports a device-side failure of the
 * persistent block kernel (a workgroup that timed out waiting for its inputs)
 * as VXM_ERR_BACKEND, then clears it.  Forward and solve calls are
 * asynchronous and cannot report such a failure themselves: call this after
 * the results of a solve are read.  A failed launch does not affect later
 * ones. */
int vxm_locdit_check(vxm_locdit *m);
/* Debug read-back of every block (as vxm_minicpm4_set_layer_dump): with a
 * non-null dump_dev each later evaluation writes the rows of both CFG branches
 * entering every block l to dump_dev + l * rows * hidden (rows = n_seg * (3 +
 * Pc + P)) and the last block's output, residual added, at l = n_layers: (n_layers
 * + 1) * rows * hidden floats.  A solve overwrites it at every step (the last
 * evaluation stays). */
int vxm_locdit_set_block_dump(vxm_locdit *m, float *dump_dev);

/* ---- LocEnc and the per-token LM update ----------------------------------
 * Mirrors vcpm_locenc_config (src/locenc.h:49-60); max_seq_len and
 * patch_size are unused there and left out. */
typedef struct vxm_locenc_config {
    int32_t hidden_size;
    int32_t n_layers;
    int32_t n_heads;
    int32_t n_kv_heads;
    int32_t intermediate_size;
    int32_t head_dim;
    int32_t feat_dim;         /* latent width of one patch position (in_proj input) */
    float   rms_norm_eps;
    int32_t rope_theta;       /* the reference passes 10000 (src/locenc.c:100-110) */
    /* head_dim/2 rope frequency factors (host), or NULL for the reference
     * rule (the LongRoPE short factors when head_dim == 128). */
    const float *rope_freq_factors;
} vxm_locenc_config;

/* vcpm_locenc_weights (src/locenc.h:67-73): GGUF Q8_0 rows of in_proj
 * [hidden][feat_dim] and of the blocks; F32 host copies of the vectors. */
typedef struct vxm_locenc_weights_q8_0 {
    const vxm_layer_weights_q8_0 *layers;
    const void  *in_proj;   const float *in_bias;     /* in_bias may be NULL   */
    const float *special_token;                       /* [hidden] or NULL      */
    const float *norm;                                /* [hidden] final RMSNorm */
} vxm_locenc_weights_q8_0;

typedef struct vxm_locenc vxm_locenc;

int vxm_locenc_create(vxm_ctx *ctx, const vxm_locenc_config *cfg, const vxm_locenc_weights_q8_0 *w,
                      vxm_locenc **out);
int vxm_locenc_free(vxm_locenc *m);

/* vcpm_locenc_forward (src/locenc.c:44-131) on x [P][feat_dim]: h = in_proj x
 * + bias (F32, no BF16), the special token prepended as row 0, n_layers
 * bidirectional rope blocks (positions 0..), final RMSNorm.  out is the
 * special token's row [hidden]; without a special token it is every row
 * [P][hidden]. */
int vxm_locenc_forward(vxm_locenc *m, const float *x_dev, int32_t P, float *out_dev);
/* Block strategy of vxm_locenc_forward, as vxm_locdit_set_block_mode (the
 * same persistent kernel; AUTO takes it wherever it applies), and
 * the report of its device-side failures, as vxm_locdit_check.  No reference
 * counterpart. */
int vxm_locenc_set_block_mode(vxm_locenc *m, int mode);
int vxm_locenc_check(vxm_locenc *m);
/* As vxm_locdit_set_block_dump for the P + 1 rows of the encoder. */
int vxm_locenc_set_block_dump(vxm_locenc *m, float *dump_dev);

/* The scalar quantizer core of the FSQ layer, vcpm_fsq_quantize
 * (src/fsq.c:16-29): y = round(tanh(x) * s) * (1/s) elementwise, round half
 * away from zero (ggml_round); quant_scale <= 0 copies x. */
int vxm_fsq_quantize(vxm_ctx *ctx, const float *x_dev, int64_t n, float quant_scale, float *y_dev);

/* Widths and FSQ scale of gen_lm_update (src/gen_step.c:712-927). */
typedef struct vxm_lm_update_config {
    int32_t lm_hidden;        /* TSLM hidden (audio embedding, FSQ output)    */
    int32_t enc_hidden;       /* LocEnc hidden                                */
    int32_t fsq_dim;          /* rows of fsq.in_proj                          */
    int32_t res_hidden;       /* RALM hidden                                  */
    float   fsq_quant_scale;  /* voxcpm.fsq_quant_scale, 9 by default (src/model_loader.c:60,152) */
} vxm_lm_update_config;

/* The projections around the two LMs (src/gen_init.c:325-348), GGUF Q8_0
 * rows and F32 biases (each bias may be NULL).  fsq_in == NULL means the
 * model has no FSQ layer: its output is the TSLM hidden unchanged
 * (src/gen_step.c:272). */
typedef struct vxm_lm_update_weights_q8_0 {
    const void *enc_to_lm;     const float *enc_to_lm_bias;   /* [lm_hidden][enc_hidden] */
    const void *fsq_in;        const float *fsq_in_bias;      /* [fsq_dim][lm_hidden]    */
    const void *fsq_out;       const float *fsq_out_bias;     /* [lm_hidden][fsq_dim]    */
    const void *fusion_concat;                                /* [res_hidden][2 lm_hidden] */
} vxm_lm_update_weights_q8_0;

typedef struct vxm_lm_update vxm_lm_update;

/* The update borrows enc, tslm and ralm (RALM = no_rope MiniCPM4); they must
 * outlive it. */
int vxm_lm_update_create(vxm_ctx *ctx, const vxm_lm_update_config *cfg, const vxm_lm_update_weights_q8_0 *w,
                         vxm_locenc *enc, vxm_minicpm4 *tslm, vxm_minicpm4 *ralm, vxm_lm_update **out);
int vxm_lm_update_free(vxm_lm_update *u);

/* gen_lm_update (src/gen_step.c:712-927) for the patch just generated,
 * prev_patch [P][feat_dim] (device), at sequence position pos:
 *   audio_embed = enc_to_lm(LocEnc(prev_patch)) + bias           [lm_hidden]
 *   base_hidden = TSLM(audio_embed), cache row pos               [lm_hidden]
 *   fsq         = fsq_out(FSQ(fsq_in(base_hidden) + b)) + b      [lm_hidden]
 *   ralm_hidden = RALM(fusion_concat([fsq ; audio_embed])), row pos [res_hidden]
 * The reference reads audio_embed / base_hidden / fsq back to the host
 * between the two LM graphs; here the whole chain is stream-ordered on the
 * device with no host synchronisation.  audio_embed_dev and fsq_dev may be
 * NULL; base_hidden_dev and ralm_hidden_dev receive the LM states. */
int vxm_lm_update_step(vxm_lm_update *u, vxm_kv_cache *tslm_kv, vxm_kv_cache *ralm_kv,
                       const float *prev_patch_dev, int32_t P, int32_t pos, float *audio_embed_dev,
                       float *base_hidden_dev, float *fsq_dev, float *ralm_hidden_dev);

/* gen_prompt_eval_range (src/gen_prompt.c:186-272) for n_tokens text tokens at
 * sequence positions [pos, pos + n_tokens), on the update's TSLM and RALM:
 *   base_hidden = TSLM(x), cache rows [pos, pos + n)                 [n][lm_hidden]
 *   ralm_hidden = RALM(fusion_concat([base_hidden ; 0])), same rows   [n][res_hidden]
 * The prompt carries no audio features, so the second half of every fusion
 * input row is zero (src/gen_prompt.c:206-217).  x_dev holds the n token
 * embeddings (vxm_embed_rows_q8_0) and receives base_hidden in place; the
 * last rows of the two outputs are the reference's lm_hidden_state and
 * residual_hidden_state (src/gen_prompt.c:247-270).  Stream-ordered, no host
 * synchronisation (the reference reads both outputs back after one graph). */
int vxm_prompt_prefill(vxm_lm_update *u, vxm_kv_cache *tslm_kv, vxm_kv_cache *ralm_kv, float *x_dev,
                       int32_t n_tokens, int32_t pos, float *ralm_hidden_dev);

/* The text embedding rows of gen_forward_text for a Q8_0 embed_tokens table
 * (src/gen_prompt.c:106-125): out[i] = dequantized row ids[i] of table (an id
 * outside [0, rows) reads row 0, src/gen_prompt.c:113-114).  ids_dev: n int32
 * on the device (the reference indexes token_ids[pos_start + i]: pass the
 * pointer at pos_start); out_dev: [n][cols] F32. */
int vxm_embed_rows_q8_0(vxm_ctx *ctx, const vxm_weight *table, const int32_t *ids_dev, int32_t n, float *out_dev);

/* ---- GGUF reader (host only) ----------------------------------------------
 * A read-only, memory-mapped GGUF v2/v3 file: tensor directory, key/value
 * metadata and tensor bytes in place.  Stands in for ggml's
 * gguf_init_from_file as vcpm_model_load uses it (src/model_loader.c:101-120)
 * for the tensors of this path; the tensor bytes of a Q8_0 tensor are exactly
 * the GGUF rows vxm_upload_q8_0 and the *_weights_q8_0 structs take. */
typedef struct vxm_gguf vxm_gguf;

/* ggml type ids of the tensors this path reads */
#define VXM_GGML_F32 0
#define VXM_GGML_F16 1
#define VXM_GGML_Q8_0 8
#define VXM_GGML_BF16 30

typedef struct vxm_gguf_tensor_info {
    const char *name;        /* valid while the file is open */
    int32_t     type;        /* ggml type id */
    int32_t     n_dims;
    int64_t     ne[4];       /* ne[0] = row length; unused dims are 1 */
    int64_t     n_elements;
    uint64_t    offset;      /* from the start of the data section */
    const void *data;        /* bytes in the mapping */
    uint64_t    nbytes;      /* 0 for a type whose size the reader does not know */
} vxm_gguf_tensor_info;

/* Opens and validates path (magic, version 2 or 3, every tensor inside the
 * file and aligned to general.alignment).  Errors: VXM_ERR_IO (unreadable),
 * VXM_ERR_MODEL_FORMAT (not a valid GGUF); err (may be NULL) gets the reason. */
int vxm_gguf_open(const char *path, vxm_gguf **out, char *err, size_t err_size);
int vxm_gguf_close(vxm_gguf *g);
const char *vxm_gguf_last_error(const vxm_gguf *g);
int32_t vxm_gguf_version(const vxm_gguf *g);
int64_t vxm_gguf_n_tensors(const vxm_gguf *g);
/* index of a tensor by name (vcpm_model_get_tensor), -1 if absent */
int64_t vxm_gguf_find_tensor(const vxm_gguf *g, const char *name);
int vxm_gguf_tensor(const vxm_gguf *g, int64_t idx, vxm_gguf_tensor_info *out);
/* Metadata with defaults, as get_key_i32 / get_key_f32 / get_key_str
 * (src/model_loader.c:20-41).  Integer keys of any width and bool keys read
 * as int; float keys also accept F64 and integers. */
int32_t vxm_gguf_get_i32(const vxm_gguf *g, const char *key, int32_t def);
float vxm_gguf_get_f32(const vxm_gguf *g, const char *key, float def);
const char *vxm_gguf_get_str(const vxm_gguf *g, const char *key, const char *def);
/* F32 copy of an F32 / F16 / BF16 / Q8_0 tensor of n elements, as
 * vcpm_model_ensure_f32 makes for norms, biases and special tokens
 * (src/model_loader.c:254-352): Q8_0 values are (float)qs * fp32(d). */
int vxm_gguf_tensor_f32(const vxm_gguf *g, int64_t idx, float *out, int64_t n);
/* The nine tensors of block `layer` named as fill_minicpm4_weights does
 * (src/gen_init.c:34-67): "<prefix>.<layer>.self_attn.q_proj.weight", ...
 * with prefix "base_lm.blk", "residual_lm.blk", "feat_encoder.blk" or
 * "feat_decoder.estimator.blk".  The seven projections (2-D Q8_0) point into
 * the mapping; the two norms are written as F32 to norms[2 * hidden].
 * q_dim = n_heads * head_dim, kv_dim = n_kv_heads * head_dim, ffn =
 * intermediate_size: every projection must have exactly the ne = [K, N] these
 * give (q [hidden, q_dim], k / v [hidden, kv_dim], o [q_dim, hidden], gate /
 * up [hidden, ffn], down [ffn, hidden]), else VXM_ERR_MODEL_FORMAT, so a file
 * whose shapes disagree with its config is never read past a tensor. */
int vxm_gguf_layer_q8_0(vxm_gguf *g, const char *prefix, int32_t layer, int64_t hidden, int64_t q_dim,
                        int64_t kv_dim, int64_t ffn, float *norms, vxm_layer_weights_q8_0 *out);
/* The TSLM (residual = 0) or RALM (residual = 1) config from the voxcpm.*
 * keys with vcpm_model_config_default's defaults and vcpm_model_load's
 * sanitisation (src/model_loader.c:52-97,139-219): eps below 1e-7 becomes
 * 1e-5, scale_depth is 0 unless voxcpm.use_mup.  VXM_ERR_UNSUPPORTED_ARCH
 * unless general.architecture is "voxcpm2". */
int vxm_gguf_minicpm4_config(vxm_gguf *g, int32_t residual, vxm_minicpm4_config *cfg);

/* ---- host helpers (no device work) --------------------------------------
 * GGUF Q8_0 quantization of F32 rows with the weight rule of
 * ggml_quantize_chunk (tools/quantize.c:292): d = amax/127 (fp16),
 * qs = roundf(x / d).  Writes rows * (k/32) 34-byte blocks. */
int vxm_host_quantize_q8_0(const float *x, int64_t rows, int64_t k, void *gguf_rows);
/* Seeded synthetic N(mean, std^2) data: SplitMix64 (as in the reference's
 * CFM noise, src/gen_step.c:409-431) with Box-Muller in double; element i is
 * stream element offset + i.  No reference counterpart: benchmark inputs. */
int vxm_host_randn(uint64_t seed, uint64_t offset, int64_t n, float mean, float std, float *out);
/* dit_sinusoidal_t_embed (src/locdit.c:163-188) of a scalar t: dim floats. */
int vxm_host_sinusoid_embed(float t, int32_t dim, float *out);
/* CFM time of a step: VXM_CFM_SWAY = vcpm_cfm_sway_t_bf16
 * (src/cfm_solver.c:27-37), VXM_CFM_UNIFORM = bf16(1 - step / n_steps). */
float vxm_host_cfm_t(int32_t step, int32_t n_steps, int32_t schedule);
/* vcpm_cfm_zero_star_steps (src/gen_step.c:50-54). */
int32_t vxm_host_cfm_zero_star_steps(int32_t n_steps);
/* The NEOX rope angles of ggml_rope_ext as vcpm_rope uses them
 * (src/minicpm4.c:165-223): for positions pos0 .. pos0+n_pos-1, head_dim/2
 * (cos, sin) pairs each, out[p * head_dim + 2i (+1)]; ff = head_dim/2
 * frequency factors or NULL.  The device kernels read this table. */
int vxm_host_rope_cache(float base, int32_t head_dim, const float *ff, int32_t pos0, int32_t n_pos,
                        float *out);

#ifdef __cplusplus
}
#endif
#endif /* VXM_Q8_H */
