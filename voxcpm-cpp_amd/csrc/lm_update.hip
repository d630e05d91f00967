// lm_update.hip -- the per-token LM update of the VoxCPM2 generation loop
// (gen_lm_update, src/gen_step.c:712-927) on gfx950: the LocEnc feature
// encoder (vcpm_locenc_forward, src/locenc.c:44-131), the audio embedding
// projection, the TSLM decode step, the FSQ layer (gen_fsq_hidden,
// src/gen_step.c:268-290 with vcpm_fsq_quantize, src/fsq.c:16-29), the
// fusion projection and the RALM decode step.
//
// The reference computes this as two graphs with the host reading the audio
// embedding, the TSLM hidden and the FSQ output in between.  Here every piece
// is a stream-ordered launch on device buffers: M = 1 projections take the
// Q8_0 GEMV, the two LM steps take vxm_minicpm4_forward (the persistent
// decode kernel where it applies), the encoder's P + 1 rows take the block
// kernels.  No host synchronisation.
#include <math.h>
#include <string.h>

#include <vector>

#include "vxm_model.h"

struct vxm_locenc {
    vxm_ctx *ctx = nullptr;
    vxm_locenc_config cfg{};
    vxm_block_dims dims;
    std::vector<vxm_block> blocks;
    vxm_weight *in_proj = nullptr;
    float *in_bias = nullptr, *special = nullptr, *norm = nullptr;
    vxm_workspace ws;
    void *buf = nullptr;   // seq [S][H], xh [P][H], aq/ad of x
    size_t buf_bytes = 0;
    float *seq = nullptr, *xh = nullptr;
    int8_t *aq = nullptr;
    uint16_t *ad = nullptr;
    int block_mode = VXM_DECODE_AUTO;   // blocks launch by launch, or all in one persistent launch
    // debug: each evaluation writes the rows entering every block and the last block's
    // output (residual added) here, [n_layers + 1][rows][H] (null: off)
    float *block_dump = nullptr;
    vxm_lpersist *lp = nullptr;
};

struct vxm_lm_update {
    vxm_ctx *ctx = nullptr;
    vxm_lm_update_config cfg{};
    vxm_locenc *enc = nullptr;
    vxm_minicpm4 *tslm = nullptr, *ralm = nullptr;
    vxm_weight *enc_to_lm = nullptr, *fsq_in = nullptr, *fsq_out = nullptr, *fusion = nullptr;
    float *enc_to_lm_bias = nullptr, *fsq_in_bias = nullptr, *fsq_out_bias = nullptr;
    float inv_scale = 0.0f;
    void *buf = nullptr;
    float *fe = nullptr;     // LocEnc output [enc_hidden]
    float *cat = nullptr;    // [fsq (lm_hidden) ; audio_embed (lm_hidden)]
    float *fh = nullptr;     // raw fsq.in_proj output [fsq_dim]
    int8_t *aq = nullptr;    // Q8_0 of the widest input (2 lm_hidden)
    uint16_t *ad = nullptr;
    // prompt prefill: [n][2 lm_hidden] fusion input and its Q8_0, grown on demand
    void *pbuf = nullptr;
    size_t pbytes = 0;
};

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------
// LocEnc sequence (src/locenc.c:55-85): row 0 the special token when there is
// one, then in_proj(x) + bias, all F32 (no BF16 here in the reference).
__global__ void k_locenc_assemble(float *__restrict__ seq, const float *__restrict__ special,
                                  const float *__restrict__ xh, const float *__restrict__ xb, int H) {
    const int row = blockIdx.x, off = special ? 1 : 0;
    float *dst = seq + (int64_t)row * H;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        float v;
        if (row < off) {
            v = special[i];
        } else {
            v = xh[(int64_t)(row - off) * H + i];
            if (xb) v = v + xb[i];
        }
        dst[i] = v;
    }
}

// y = x + b (ggml_add of a bias, F32); also into y2 when non-null.
__global__ void k_bias_add(const float *__restrict__ x, const float *__restrict__ b, float *__restrict__ y,
                           float *__restrict__ y2, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = x[i];
    if (b) v = v + b[i];
    y[i] = v;
    if (y2) y2[i] = v;
}

// FSQ core (src/fsq.c:16-29) after the in_proj bias (src/gen_step.c:273-276):
// v = x + b; y = roundf(tanhf(v) * s) * inv_s with inv_s = 1/s computed on the
// host in float (ggml_scale by 1.0f / quant_scale); s <= 0: y = v.
__global__ void k_fsq(const float *__restrict__ x, const float *__restrict__ b, float *__restrict__ y, int64_t n,
                      float s, float inv_s) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = x[i];
    if (b) v = v + b[i];
    if (s > 0.0f) v = roundf(tanhf(v) * s) * inv_s;
    y[i] = v;
}

// Prompt fusion input (src/gen_prompt.c:206-217): row i = [base_hidden[i] ;
// zeros] -- the prompt carries no audio features.
__global__ void k_prompt_fusion_in(const float *__restrict__ base, float *__restrict__ cat, int n, int H) {
    const int row = blockIdx.x;
    if (row >= n) return;
    const float *src = base + (int64_t)row * H;
    float *dst = cat + (int64_t)row * 2 * H;
    for (int i = threadIdx.x; i < 2 * H; i += blockDim.x) dst[i] = i < H ? src[i] : 0.0f;
}

// Q8_0 embedding rows (the Q8_0 branch of gen_forward_text, src/gen_prompt.c:
// 106-125): out[i][j] = (float)qs[j] * fp16(d[j/32]) of row ids[i]; an id outside
// [0, n_rows) takes row 0 (src/gen_prompt.c:113-114).
__global__ void k_embed_rows_q8_0(const int8_t *__restrict__ qs, const uint16_t *__restrict__ d,
                                  const int32_t *__restrict__ ids, int64_t n_rows, int64_t k,
                                  float *__restrict__ out) {
    const int i = blockIdx.x;
    int64_t r = ids[i];
    if (r < 0 || r >= n_rows) r = 0;
    const int8_t *q = qs + r * k;
    const uint16_t *dr = d + r * (k / 32);
    float *o = out + (int64_t)i * k;
    for (int64_t j = threadIdx.x; j < k; j += blockDim.x) o[j] = (float)q[j] * vxm_h2f(dr[j / 32]);
}

static unsigned grid_of(int64_t n) { return (unsigned)((n + 255) / 256); }

int vxm_upload_vec(vxm_ctx *ctx, const float *src, int64_t n, float **out) {
    *out = nullptr;
    if (!src) return VXM_OK;
    if (hipMalloc((void **)out, n * 4) != hipSuccess) {
        (void)hipGetLastError();
        *out = nullptr;
        return vxm_fail(ctx, VXM_ERR_OOM, "vector upload of %lld floats failed", (long long)n);
    }
    VXM_HIP(ctx, hipMemcpy(*out, src, n * 4, hipMemcpyHostToDevice));
    return VXM_OK;
}

// ---------------------------------------------------------------------------
// LocEnc
// ---------------------------------------------------------------------------
constexpr int kLocEncMaxRows = 4096;

static int locenc_bufs(vxm_locenc *m, int64_t S, int64_t P) {
    vxm_ctx *ctx = m->ctx;
    const int64_t H = m->dims.H, feat = m->cfg.feat_dim;
    const size_t parts[4] = {(size_t)(S * H * 4), (size_t)(P * H * 4), (size_t)(P * feat),
                             (size_t)(P * (feat / 32) * 2)};
    size_t total = 0;
    for (size_t p : parts) total += (p + 255) & ~(size_t)255;
    if (total > m->buf_bytes) {
        VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (m->buf) VXM_HIP(ctx, hipFree(m->buf));
        m->buf = nullptr;
        m->buf_bytes = 0;
        if (hipMalloc(&m->buf, total) != hipSuccess) {
            (void)hipGetLastError();
            return vxm_fail(ctx, VXM_ERR_OOM, "locenc: buffers of %zu bytes failed", total);
        }
        m->buf_bytes = total;
    }
    char *b = (char *)m->buf;
    void **dst[4] = {(void **)&m->seq, (void **)&m->xh, (void **)&m->aq, (void **)&m->ad};
    for (int i = 0; i < 4; i++) {
        *dst[i] = b;
        b += (parts[i] + 255) & ~(size_t)255;
    }
    return VXM_OK;
}

extern "C" int vxm_locenc_free(vxm_locenc *m) {
    if (!m) return VXM_ERR_INVALID_ARG;
    vxm_ctx *ctx = m->ctx;
    (void)hipStreamSynchronize(ctx->stream);
    for (auto &b : m->blocks) vxm_block_free(ctx, b);
    if (m->in_proj) vxm_weight_free(ctx, m->in_proj);
    for (float *p : {m->in_bias, m->special, m->norm})
        if (p) (void)hipFree(p);
    vxm_locdit_persistent_free(m->lp);
    vxm_rope_free(m->dims);
    vxm_ws_free(m->ws);
    if (m->buf) (void)hipFree(m->buf);
    delete m;
    return VXM_OK;
}

extern "C" int vxm_locenc_create(vxm_ctx *ctx, const vxm_locenc_config *cfg, const vxm_locenc_weights_q8_0 *w,
                                 vxm_locenc **out) {
    if (!ctx || !cfg || !w || !out) return VXM_ERR_INVALID_ARG;
    *out = nullptr;
    const vxm_locenc_config &c = *cfg;
    if (c.n_layers < 0 || c.hidden_size <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 ||
        c.intermediate_size <= 0 || c.n_heads % c.n_kv_heads || c.head_dim % 2 || c.hidden_size % 32 ||
        c.intermediate_size % 32 || (c.n_heads * c.head_dim) % 32 || c.head_dim > 256 || c.feat_dim <= 0 ||
        c.feat_dim % 32 || c.hidden_size > 8192)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "locenc config: unsupported sizes");
    if (!w->in_proj || !w->norm || (c.n_layers > 0 && !w->layers))
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "locenc weights: in_proj, norm or layers is NULL");
    vxm_locenc *m = new vxm_locenc();
    m->ctx = ctx;
    m->cfg = c;
    m->cfg.rope_freq_factors = nullptr;
    vxm_block_dims &d = m->dims;
    d.H = c.hidden_size;
    d.nh = c.n_heads;
    d.nkv = c.n_kv_heads;
    d.hd = c.head_dim;
    d.F = c.intermediate_size;
    d.eps = c.rms_norm_eps;
    d.no_rope = 0;          // rope on, positions from 0 (src/locenc.c:100-110)
    d.res_scale = 1.0f;     // no DeepNorm scale for the encoder (src/locenc.c:111)
    vxm_rope_setup(d, c.rope_theta, c.rope_freq_factors);
    int rc = VXM_OK;
    m->blocks.resize(c.n_layers);
    for (int l = 0; l < c.n_layers && rc == VXM_OK; l++) rc = vxm_block_upload(ctx, d, w->layers[l], m->blocks[l]);
    if (rc == VXM_OK) rc = vxm_upload_q8_0(ctx, w->in_proj, d.H, c.feat_dim, &m->in_proj);
    if (rc == VXM_OK) rc = vxm_upload_vec(ctx, w->in_bias, d.H, &m->in_bias);
    if (rc == VXM_OK) rc = vxm_upload_vec(ctx, w->special_token, d.H, &m->special);
    if (rc == VXM_OK) rc = vxm_upload_vec(ctx, w->norm, d.H, &m->norm);
    if (rc != VXM_OK) {
        vxm_locenc_free(m);
        return rc;
    }
    *out = m;
    return VXM_OK;
}

extern "C" int vxm_locenc_forward(vxm_locenc *m, const float *x_dev, int32_t P, float *out_dev) {
    if (!m) return VXM_ERR_INVALID_ARG;
    vxm_ctx *ctx = m->ctx;
    const int off = m->special ? 1 : 0;
    if (!x_dev || !out_dev || P <= 0 || (int64_t)P + off > kLocEncMaxRows)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "locenc: bad x / out / P = %d", P);
    const vxm_block_dims &d = m->dims;
    const int64_t H = d.H, S = (int64_t)P + off, qd = (int64_t)d.nh * d.hd, kvd = (int64_t)d.nkv * d.hd;
    const int var = ctx->quant_variant;
    int rc;
    if ((rc = vxm_ws_ensure(ctx, m->ws, S, H, qd, kvd, d.F, (int64_t)d.nkv * S * d.hd))) return rc;
    if ((rc = vxm_rope_ensure(ctx, m->dims, S))) return rc;
    if ((rc = locenc_bufs(m, S, P))) return rc;
    if ((rc = vxm_launch_quantize(ctx, x_dev, P, m->cfg.feat_dim, var, m->aq, m->ad))) return rc;
    if ((rc = vxm_launch_mul_mat(ctx, m->in_proj, m->aq, m->ad, P, m->xh))) return rc;
    hipLaunchKernelGGL(k_locenc_assemble, dim3((unsigned)S), dim3(256), 0, ctx->stream, m->seq, m->special, m->xh,
                       m->in_bias, (int)H);
    VXM_CHECK_LAUNCH(ctx);
    // bidirectional blocks over the S fresh rows, positions 0..S-1, no cache
    bool residual_added = false;   // the last block's residual already in seq (debug dump)
    const bool persistent = m->cfg.n_layers > 0 && vxm_locdit_persistent_pick(ctx, d, S, (int)S, m->block_mode);
    if (m->block_mode == VXM_DECODE_PERSISTENT && !persistent)
        return vxm_fail(ctx, VXM_ERR_NOT_IMPLEMENTED, "locenc: no persistent block kernel for this shape / device");
    if (persistent) {
        // all blocks in one launch; seq then holds the last block's output, residual included
        if ((rc = vxm_locdit_persistent_run(ctx, d, m->blocks, &m->lp, m->seq, S, (int)S, m->block_dump))) return rc;
    } else {
        const vxm_attn_site site{m->ws.lk, m->ws.lv, (int)S, (int64_t)d.nkv * S * d.hd, (int)S, 0, 0, 0};
        for (int l = 0; l < m->cfg.n_layers; l++) {
            const vxm_block &b = m->blocks[l];
            if ((rc = vxm_launch_rmsnorm(ctx, m->seq, l ? m->ws.dn_out : vxm_parts{}, 1.0f, b.g_in, S, H, d.eps,
                                         nullptr, m->ws.xq, m->ws.xd, var)))
                return rc;
            // the norm added the previous block's residual in place: seq holds block l's input
            if (m->block_dump)
                VXM_HIP(ctx, hipMemcpyAsync(m->block_dump + (size_t)l * S * H, m->seq, (size_t)S * H * sizeof(float),
                                            hipMemcpyDeviceToDevice, ctx->stream));
            if ((rc = vxm_block_run(ctx, d, b, m->ws, m->seq, S, site))) return rc;
        }
        if (m->block_dump && m->cfg.n_layers) {
            // debug: the last residual on its own (the final norm then adds none), and the rows out
            if ((rc = vxm_launch_residual(ctx, m->seq, m->ws.dn_out, 1.0f, S * H))) return rc;
            residual_added = true;
            VXM_HIP(ctx, hipMemcpyAsync(m->block_dump + (size_t)m->cfg.n_layers * S * H, m->seq,
                                        (size_t)S * H * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream));
        }
    }
    // last residual + final RMSNorm of the rows that are returned: the
    // special token's row (src/locenc.c:118-128), or every row
    const int64_t rows = off ? 1 : S;
    return vxm_launch_rmsnorm(ctx, m->seq, m->cfg.n_layers && !persistent && !residual_added ? m->ws.dn_out : vxm_parts{},
                              1.0f, m->norm,
                              rows, H, d.eps, out_dev, nullptr, nullptr, var);
}

extern "C" int vxm_locenc_set_block_dump(vxm_locenc *m, float *dump_dev) {
    if (!m) return VXM_ERR_INVALID_ARG;
    m->block_dump = dump_dev;
    return VXM_OK;
}

extern "C" int vxm_locenc_set_block_mode(vxm_locenc *m, int mode) {
    if (!m) return VXM_ERR_INVALID_ARG;
    if (mode < VXM_DECODE_AUTO || mode > VXM_DECODE_PERSISTENT)
        return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "unknown block mode %d", mode);
    m->block_mode = mode;
    return VXM_OK;
}

extern "C" int vxm_locenc_check(vxm_locenc *m) {
    if (!m) return VXM_ERR_INVALID_ARG;
    return vxm_locdit_persistent_check(m->ctx, m->lp);
}

// ---------------------------------------------------------------------------
// FSQ and the LM update
// ---------------------------------------------------------------------------
extern "C" int vxm_fsq_quantize(vxm_ctx *ctx, const float *x_dev, int64_t n, float quant_scale, float *y_dev) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (!x_dev || !y_dev || n < 0) return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "fsq_quantize: bad arguments");
    if (n == 0) return VXM_OK;
    const float inv = quant_scale > 0.0f ? 1.0f / quant_scale : 0.0f;
    hipLaunchKernelGGL(k_fsq, dim3(grid_of(n)), dim3(256), 0, ctx->stream, x_dev, (const float *)nullptr, y_dev, n,
                       quant_scale, inv);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

extern "C" int vxm_lm_update_free(vxm_lm_update *u) {
    if (!u) return VXM_ERR_INVALID_ARG;
    vxm_ctx *ctx = u->ctx;
    (void)hipStreamSynchronize(ctx->stream);
    for (vxm_weight *w : {u->enc_to_lm, u->fsq_in, u->fsq_out, u->fusion})
        if (w) vxm_weight_free(ctx, w);
    for (float *p : {u->enc_to_lm_bias, u->fsq_in_bias, u->fsq_out_bias})
        if (p) (void)hipFree(p);
    if (u->buf) (void)hipFree(u->buf);
    if (u->pbuf) (void)hipFree(u->pbuf);
    delete u;
    return VXM_OK;
}

extern "C" int vxm_lm_update_create(vxm_ctx *ctx, const vxm_lm_update_config *cfg,
                                    const vxm_lm_update_weights_q8_0 *w, vxm_locenc *enc, vxm_minicpm4 *tslm,
                                    vxm_minicpm4 *ralm, vxm_lm_update **out) {
    if (!ctx || !cfg || !w || !out) return VXM_ERR_INVALID_ARG;
    *out = nullptr;
    const vxm_lm_update_config &c = *cfg;
    if (!enc || !tslm || !ralm || enc->ctx != ctx || tslm->ctx != ctx || ralm->ctx != ctx)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "lm_update: encoder / TSLM / RALM missing or on another context");
    const bool fsq = w->fsq_in != nullptr;
    if (c.lm_hidden <= 0 || c.lm_hidden % 32 || c.enc_hidden <= 0 || c.enc_hidden % 32 || c.res_hidden <= 0 ||
        (fsq && (c.fsq_dim <= 0 || c.fsq_dim % 32)) || c.enc_hidden != enc->dims.H || c.lm_hidden != tslm->dims.H ||
        c.res_hidden != ralm->dims.H || enc->special == nullptr)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG,
                        "lm_update config: widths must be multiples of 32 and match the encoder (with a "
                        "special token), TSLM and RALM");
    if (!w->enc_to_lm || !w->fusion_concat || (fsq && !w->fsq_out))
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "lm_update weights: a projection is NULL");
    vxm_lm_update *u = new vxm_lm_update();
    u->ctx = ctx;
    u->cfg = c;
    u->enc = enc;
    u->tslm = tslm;
    u->ralm = ralm;
    u->inv_scale = c.fsq_quant_scale > 0.0f ? 1.0f / c.fsq_quant_scale : 0.0f;
    const int64_t L = c.lm_hidden, E = c.enc_hidden, Fq = fsq ? c.fsq_dim : 0;
    int rc = vxm_upload_q8_0(ctx, w->enc_to_lm, L, E, &u->enc_to_lm);
    if (rc == VXM_OK) rc = vxm_upload_vec(ctx, w->enc_to_lm_bias, L, &u->enc_to_lm_bias);
    if (rc == VXM_OK && fsq) rc = vxm_upload_q8_0(ctx, w->fsq_in, Fq, L, &u->fsq_in);
    if (rc == VXM_OK && fsq) rc = vxm_upload_vec(ctx, w->fsq_in_bias, Fq, &u->fsq_in_bias);
    if (rc == VXM_OK && fsq) rc = vxm_upload_q8_0(ctx, w->fsq_out, L, Fq, &u->fsq_out);
    if (rc == VXM_OK && fsq) rc = vxm_upload_vec(ctx, w->fsq_out_bias, L, &u->fsq_out_bias);
    if (rc == VXM_OK) rc = vxm_upload_q8_0(ctx, w->fusion_concat, c.res_hidden, 2 * L, &u->fusion);
    if (rc == VXM_OK) {
        const int64_t kq = std::max<int64_t>(std::max<int64_t>(2 * L, E), Fq);
        const size_t parts[5] = {(size_t)E * 4, (size_t)(2 * L) * 4, (size_t)std::max<int64_t>(Fq, 1) * 4,
                                 (size_t)kq, (size_t)(kq / 32) * 2};
        size_t total = 0;
        for (size_t p : parts) total += (p + 255) & ~(size_t)255;
        if (hipMalloc(&u->buf, total) != hipSuccess) {
            (void)hipGetLastError();
            u->buf = nullptr;
            rc = vxm_fail(ctx, VXM_ERR_OOM, "lm_update: buffers of %zu bytes failed", total);
        } else {
            char *b = (char *)u->buf;
            void **dst[5] = {(void **)&u->fe, (void **)&u->cat, (void **)&u->fh, (void **)&u->aq, (void **)&u->ad};
            for (int i = 0; i < 5; i++) {
                *dst[i] = b;
                b += (parts[i] + 255) & ~(size_t)255;
            }
        }
    }
    if (rc != VXM_OK) {
        vxm_lm_update_free(u);
        return rc;
    }
    *out = u;
    return VXM_OK;
}

extern "C" int vxm_lm_update_step(vxm_lm_update *u, vxm_kv_cache *tslm_kv, vxm_kv_cache *ralm_kv,
                                  const float *prev_patch_dev, int32_t P, int32_t pos, float *audio_embed_dev,
                                  float *base_hidden_dev, float *fsq_dev, float *ralm_hidden_dev) {
    if (!u) return VXM_ERR_INVALID_ARG;
    vxm_ctx *ctx = u->ctx;
    if (!prev_patch_dev || !base_hidden_dev || !ralm_hidden_dev || !tslm_kv || !ralm_kv || pos < 0)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "lm_update: bad patch / outputs / caches / pos");
    const int64_t L = u->cfg.lm_hidden, Fq = u->fsq_in ? u->cfg.fsq_dim : 0;
    const int var = ctx->quant_variant;
    float *fsq_part = u->cat, *audio_part = u->cat + L;
    int rc;
    // audio embedding (src/gen_step.c:208-266)
    if ((rc = vxm_locenc_forward(u->enc, prev_patch_dev, P, u->fe))) return rc;
    if ((rc = vxm_launch_quantize(ctx, u->fe, 1, u->cfg.enc_hidden, var, u->aq, u->ad))) return rc;
    if ((rc = vxm_launch_mul_mat(ctx, u->enc_to_lm, u->aq, u->ad, 1, audio_part))) return rc;
    hipLaunchKernelGGL(k_bias_add, dim3(grid_of(L)), dim3(256), 0, ctx->stream, audio_part, u->enc_to_lm_bias,
                       audio_part, base_hidden_dev, L);
    VXM_CHECK_LAUNCH(ctx);
    if (audio_embed_dev)
        VXM_HIP(ctx, hipMemcpyAsync(audio_embed_dev, audio_part, L * 4, hipMemcpyDeviceToDevice, ctx->stream));
    // TSLM step at pos, in place on base_hidden (src/gen_step.c:741-771)
    if ((rc = vxm_minicpm4_forward(u->tslm, tslm_kv, base_hidden_dev, 1, pos))) return rc;
    // FSQ (src/gen_step.c:268-290), or the hidden unchanged without one
    if (Fq > 0) {
        if ((rc = vxm_launch_quantize(ctx, base_hidden_dev, 1, L, var, u->aq, u->ad))) return rc;
        if ((rc = vxm_launch_mul_mat(ctx, u->fsq_in, u->aq, u->ad, 1, u->fh))) return rc;
        hipLaunchKernelGGL(k_fsq, dim3(grid_of(Fq)), dim3(256), 0, ctx->stream, u->fh, u->fsq_in_bias, u->fh, Fq,
                           u->cfg.fsq_quant_scale, u->inv_scale);
        VXM_CHECK_LAUNCH(ctx);
        if ((rc = vxm_launch_quantize(ctx, u->fh, 1, Fq, var, u->aq, u->ad))) return rc;
        if ((rc = vxm_launch_mul_mat(ctx, u->fsq_out, u->aq, u->ad, 1, fsq_part))) return rc;
        hipLaunchKernelGGL(k_bias_add, dim3(grid_of(L)), dim3(256), 0, ctx->stream, fsq_part, u->fsq_out_bias,
                           fsq_part, fsq_dev, L);
        VXM_CHECK_LAUNCH(ctx);
    } else {
        VXM_HIP(ctx, hipMemcpyAsync(fsq_part, base_hidden_dev, L * 4, hipMemcpyDeviceToDevice, ctx->stream));
        if (fsq_dev)
            VXM_HIP(ctx, hipMemcpyAsync(fsq_dev, base_hidden_dev, L * 4, hipMemcpyDeviceToDevice, ctx->stream));
    }
    // RALM input = fusion_concat_proj([fsq ; audio_embed]) (src/gen_step.c:870-899), then the RALM step
    if ((rc = vxm_launch_quantize(ctx, u->cat, 1, 2 * L, var, u->aq, u->ad))) return rc;
    if ((rc = vxm_launch_mul_mat(ctx, u->fusion, u->aq, u->ad, 1, ralm_hidden_dev))) return rc;
    return vxm_minicpm4_forward(u->ralm, ralm_kv, ralm_hidden_dev, 1, pos);
}

// ---------------------------------------------------------------------------
// prompt prefill and the embedding rows
// ---------------------------------------------------------------------------
extern "C" int vxm_embed_rows_q8_0(vxm_ctx *ctx, const vxm_weight *table, const int32_t *ids_dev, int32_t n,
                                   float *out_dev) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (!table || (n > 0 && (!ids_dev || !out_dev)) || n < 0)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "embed_rows: bad table / ids / out / n");
    if (n == 0) return VXM_OK;
    hipLaunchKernelGGL(k_embed_rows_q8_0, dim3((unsigned)n), dim3(256), 0, ctx->stream, table->qs, table->d, ids_dev,
                       table->n, table->k, out_dev);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

extern "C" int vxm_prompt_prefill(vxm_lm_update *u, vxm_kv_cache *tslm_kv, vxm_kv_cache *ralm_kv, float *x_dev,
                                  int32_t n_tokens, int32_t pos, float *ralm_hidden_dev) {
    if (!u) return VXM_ERR_INVALID_ARG;
    vxm_ctx *ctx = u->ctx;
    if (!x_dev || !ralm_hidden_dev || !tslm_kv || !ralm_kv || pos < 0 || n_tokens < 0)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "prompt_prefill: bad x / outputs / caches / pos / n_tokens");
    if (n_tokens == 0) return VXM_OK;
    const int64_t L = u->cfg.lm_hidden, n = n_tokens;
    const int var = ctx->quant_variant;
    int rc;
    // base LM over the n text tokens, in place (src/gen_prompt.c:197-200)
    if ((rc = vxm_minicpm4_forward(u->tslm, tslm_kv, x_dev, n, pos))) return rc;
    // RALM input = fusion_concat_proj([base_hidden ; 0]) (src/gen_prompt.c:204-217)
    const size_t cat_b = ((size_t)n * 2 * L * 4 + 255) & ~(size_t)255, q_b = ((size_t)n * 2 * L + 255) & ~(size_t)255,
                 d_b = (size_t)n * (2 * L / 32) * 2;
    if (u->pbytes < cat_b + q_b + d_b) {
        VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (u->pbuf) VXM_HIP(ctx, hipFree(u->pbuf));
        u->pbuf = nullptr;
        u->pbytes = 0;
        if (hipMalloc(&u->pbuf, cat_b + q_b + d_b) != hipSuccess) {
            (void)hipGetLastError();
            return vxm_fail(ctx, VXM_ERR_OOM, "prompt_prefill: %zu bytes of fusion buffers", cat_b + q_b + d_b);
        }
        u->pbytes = cat_b + q_b + d_b;
    }
    float *cat = (float *)u->pbuf;
    int8_t *cq = (int8_t *)((char *)u->pbuf + cat_b);
    uint16_t *cd = (uint16_t *)((char *)u->pbuf + cat_b + q_b);
    hipLaunchKernelGGL(k_prompt_fusion_in, dim3((unsigned)n), dim3(256), 0, ctx->stream, x_dev, cat, (int)n, (int)L);
    VXM_CHECK_LAUNCH(ctx);
    if ((rc = vxm_launch_quantize(ctx, cat, n, 2 * L, var, cq, cd))) return rc;
    if ((rc = vxm_launch_mul_mat(ctx, u->fusion, cq, cd, n, ralm_hidden_dev))) return rc;
    // RALM over the same positions (src/gen_prompt.c:219-223)
    return vxm_minicpm4_forward(u->ralm, ralm_kv, ralm_hidden_dev, n, pos);
}
