// minicpm4.hip -- the MiniCPM4 block / stack on gfx950 (vcpm_minicpm4_block
// and vcpm_minicpm4_forward, src/minicpm4.c:467-572) driven as a sequence of
// stream-ordered kernels, plus the f16 KV cache.
//
// Device layout of one block:
//   wqkv : Q8_0 [(n_heads + 2 n_kv) * head_dim][hidden]   q rows, then k, then v;
//          q and k rows pair-interleaved per head (dims i, i + hd/2 -> rows 2i, 2i+1)
//   wo   : Q8_0 [hidden][n_heads * head_dim]
//   wgu  : Q8_0 [2 * ffn][hidden]                          gate n at row 2n, up n at 2n+1
//   wd   : Q8_0 [hidden][ffn]
//   g_in, g_post : fp32 [hidden]
// Kernel sequence per layer (M tokens):
//   rms_norm(+residual of the previous layer) -> Q8_0 x
//   QKV matmul -> rope + BF16 + f16 KV append -> attention -> Q8_0
//   O matmul -> residual + post norm -> Q8_0
//   gate/up matmul -> SwiGLU + Q8_0 -> down matmul (residual folded into the
//   next layer's norm, or the final norm).
#include <math.h>

#include <atomic>
#include <vector>

#include "vxm_model.h"

// LongRoPE short factors of the VoxCPM2 lm_config (src/minicpm4.c:49-66):
// model constants, one per rotary pair, applied when head_dim == 128.
static const float kVoxcpm2RopeShortFactors[64] = {
    0.9977997200f,  1.0146582960f,  1.0349680405f,  1.0594292461f,  1.0888815017f,  1.1243301355f,
    1.1669771036f,  1.2182568067f,  1.2798772354f,  1.3538666752f,  1.4426259040f,  1.5489853360f,
    1.6762658237f,  1.8283407612f,  2.0096956086f,  2.2254789275f,  2.4815363797f,  2.7844159346f,
    3.1413289096f,  3.5600478448f,  4.0487193801f,  4.6155695421f,  5.2684819497f,  6.0144385919f,
    6.8588300492f,  7.8046682500f,  8.8517684937f,  9.9960050583f,  11.2287664413f, 12.5367574692f,
    13.9022579193f, 15.3038854599f, 16.7178382874f, 18.1194648743f, 19.4849643707f, 20.7929573059f,
    22.0257186890f, 23.1699542999f, 24.2170543671f, 25.1628932953f, 26.0072841644f, 26.7532405853f,
    27.4061527252f, 27.9730033875f, 28.4616756439f, 28.8803939819f, 29.2373065948f, 29.5401859283f,
    29.7962436676f, 30.0120277405f, 30.1933822632f, 30.3454570770f, 30.4727382660f, 30.5790977478f,
    30.6678562164f, 30.7418460846f, 30.8034667969f, 30.8547458649f, 30.8973922729f, 30.9328403473f,
    30.9622936249f, 30.9867553711f, 31.0070648193f, 31.0239238739f,
};

// ---------------------------------------------------------------------------
// workspace
// ---------------------------------------------------------------------------
int vxm_ws_ensure(vxm_ctx *ctx, vxm_workspace &ws, int64_t M, int64_t H, int64_t qd, int64_t kvd, int64_t F,
                  int64_t local_kv) {
    const int64_t kmax = std::max(std::max(H, qd), F);
    // small batches: the projections may arrive as K-split slices of the small-M GEMM
    const int pf = M <= VXM_SMALL_MAX_ROWS ? VXM_MAX_PARTS : 1;
    ws.max_parts = pf;
    struct Part { size_t bytes; void **dst; };
    std::vector<Part> parts = {
        {(size_t)(M * kmax), (void **)&ws.xq},
        {(size_t)(M * (kmax / 32) * 2), (void **)&ws.xd},
        {(size_t)(pf * M * (qd + 2 * kvd) * 4), (void **)&ws.qkv},
        {(size_t)(M * qd * 4), (void **)&ws.q},
        {(size_t)(M * qd * 4), (void **)&ws.att},
        {(size_t)(pf * M * H * 4), (void **)&ws.o},
        {(size_t)(pf * M * 2 * F * 4), (void **)&ws.gu},
        {(size_t)(pf * M * H * 4), (void **)&ws.dn},
        {(size_t)(local_kv * 2), (void **)&ws.lk},
        {(size_t)(local_kv * 2), (void **)&ws.lv},
    };
    size_t total = 0;
    for (auto &p : parts) total += (p.bytes + 255) & ~(size_t)255;
    if (total <= ws.bytes) {
        char *b = (char *)ws.base;
        for (auto &p : parts) { *p.dst = b; b += (p.bytes + 255) & ~(size_t)255; }
        return VXM_OK;
    }
    VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ws.base) VXM_HIP(ctx, hipFree(ws.base));
    ws.base = nullptr;
    ws.bytes = 0;
    if (hipMalloc(&ws.base, total) != hipSuccess) {
        (void)hipGetLastError();
        return vxm_fail(ctx, VXM_ERR_OOM, "workspace of %zu bytes failed", total);
    }
    ws.bytes = total;
    char *b = (char *)ws.base;
    for (auto &p : parts) { *p.dst = b; b += (p.bytes + 255) & ~(size_t)255; }
    return VXM_OK;
}

void vxm_ws_free(vxm_workspace &ws) {
    if (ws.base) (void)hipFree(ws.base);
    ws = vxm_workspace();
}

// ---------------------------------------------------------------------------
// block weights
// ---------------------------------------------------------------------------
// Fused QKV rows: for every q head and k head, dims (i, i + hd/2) become rows
// (2i, 2i + 1), so each NEOX rotary pair is produced by one wave; v rows keep
// their order.
static int upload_qkv(vxm_ctx *ctx, const void *q, const void *k, const void *v, int nh, int nkv, int hd,
                      int64_t K, vxm_weight **out) {
    const size_t rb = (size_t)(K / 32) * 34;
    const int64_t qd = (int64_t)nh * hd, kvd = (int64_t)nkv * hd;
    std::vector<uint8_t> buf(rb * (size_t)(qd + 2 * kvd));
    auto put = [&](int64_t dst, const void *src, int64_t row) {
        memcpy(buf.data() + rb * dst, (const uint8_t *)src + rb * row, rb);
    };
    for (int head = 0; head < nh + nkv; head++) {
        const void *src = head < nh ? q : k;
        const int64_t base = head < nh ? (int64_t)head * hd : (int64_t)(head - nh) * hd;
        for (int i = 0; i < hd / 2; i++) {
            put((int64_t)head * hd + 2 * i, src, base + i);
            put((int64_t)head * hd + 2 * i + 1, src, base + i + hd / 2);
        }
    }
    memcpy(buf.data() + rb * (qd + kvd), v, rb * kvd);
    return vxm_upload_q8_0(ctx, buf.data(), qd + 2 * kvd, K, out);
}

// Fused gate/up rows interleaved: row 2n = gate n, row 2n + 1 = up n.
static int upload_gate_up(vxm_ctx *ctx, const void *gate, const void *up, int64_t F, int64_t K, vxm_weight **out) {
    const size_t rb = (size_t)(K / 32) * 34;
    std::vector<uint8_t> buf(rb * (size_t)(2 * F));
    for (int64_t n = 0; n < F; n++) {
        memcpy(buf.data() + rb * (2 * n), (const uint8_t *)gate + rb * n, rb);
        memcpy(buf.data() + rb * (2 * n + 1), (const uint8_t *)up + rb * n, rb);
    }
    return vxm_upload_q8_0(ctx, buf.data(), 2 * F, K, out);
}

static int upload_f32(vxm_ctx *ctx, const float *src, int64_t n, float **out) {
    *out = nullptr;
    if (!src) return VXM_OK;
    if (hipMalloc((void **)out, n * 4) != hipSuccess) {
        (void)hipGetLastError();
        return vxm_fail(ctx, VXM_ERR_OOM, "gain upload failed");
    }
    VXM_HIP(ctx, hipMemcpy(*out, src, n * 4, hipMemcpyHostToDevice));
    return VXM_OK;
}

int vxm_block_upload(vxm_ctx *ctx, const vxm_block_dims &d, const vxm_layer_weights_q8_0 &w, vxm_block &b) {
    if (!w.q_proj || !w.k_proj || !w.v_proj || !w.o_proj || !w.gate_proj || !w.up_proj || !w.down_proj)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "layer weights: a projection is NULL");
    const int64_t qd = (int64_t)d.nh * d.hd, kvd = (int64_t)d.nkv * d.hd;
    int rc;
    (void)kvd;
    if ((rc = upload_qkv(ctx, w.q_proj, w.k_proj, w.v_proj, d.nh, d.nkv, d.hd, d.H, &b.wqkv))) return rc;
    if ((rc = vxm_upload_q8_0(ctx, w.o_proj, d.H, qd, &b.wo))) return rc;
    if ((rc = upload_gate_up(ctx, w.gate_proj, w.up_proj, d.F, d.H, &b.wgu))) return rc;
    if ((rc = vxm_upload_q8_0(ctx, w.down_proj, d.H, d.F, &b.wd))) return rc;
    if ((rc = upload_f32(ctx, w.input_layernorm, d.H, &b.g_in))) return rc;
    if ((rc = upload_f32(ctx, w.post_attention_layernorm, d.H, &b.g_post))) return rc;
    return VXM_OK;
}

void vxm_block_free(vxm_ctx *ctx, vxm_block &b) {
    vxm_weight_free(ctx, b.wqkv);
    vxm_weight_free(ctx, b.wo);
    vxm_weight_free(ctx, b.wgu);
    vxm_weight_free(ctx, b.wd);
    if (b.g_in) (void)hipFree(b.g_in);
    if (b.g_post) (void)hipFree(b.g_post);
    b = vxm_block();
}

void vxm_rope_setup(vxm_block_dims &d, int32_t theta, const float *ff_host) {
    d.rope_base = (float)theta;
    const float *src = ff_host ? ff_host : (d.hd == 128 ? kVoxcpm2RopeShortFactors : nullptr);
    d.ff_host.clear();
    if (src) d.ff_host.assign(src, src + d.hd / 2);
}

// Rope table rows [0, n_pos): grown to at least twice its size (or 1024 rows)
// when a call needs a position beyond it.  Growing synchronises the stream
// once; steady-state calls only read the table.
int vxm_rope_ensure(vxm_ctx *ctx, vxm_block_dims &d, int64_t n_pos) {
    if (n_pos <= d.rope_rows) return VXM_OK;
    if (n_pos > (1 << 24)) return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "rope: position %lld", (long long)n_pos);
    const int64_t rows = std::max<int64_t>(std::max<int64_t>(n_pos, 2 * (int64_t)d.rope_rows), 1024);
    const int64_t half = d.hd / 2;
    std::vector<float> host((size_t)(rows * half * 2));
    int rc = vxm_host_rope_cache(d.rope_base, d.hd, d.ff_host.empty() ? nullptr : d.ff_host.data(), 0,
                                 (int32_t)rows, host.data());
    if (rc) return vxm_fail(ctx, rc, "rope: table of %lld rows", (long long)rows);
    float2 *t = nullptr;
    if (hipMalloc((void **)&t, host.size() * 4) != hipSuccess) {
        (void)hipGetLastError();
        return vxm_fail(ctx, VXM_ERR_OOM, "rope: table of %lld rows", (long long)rows);
    }
    VXM_HIP(ctx, hipMemcpyAsync(t, host.data(), host.size() * 4, hipMemcpyHostToDevice, ctx->stream));
    VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (d.rope_cs) VXM_HIP(ctx, hipFree(d.rope_cs));
    d.rope_cs = t;
    d.rope_rows = (int)rows;
    return VXM_OK;
}

void vxm_rope_free(vxm_block_dims &d) {
    if (d.rope_cs) (void)hipFree(d.rope_cs);
    d.rope_cs = nullptr;
    d.rope_rows = 0;
}

// ---------------------------------------------------------------------------
// one block over M tokens (attention half and MLP half)
// ---------------------------------------------------------------------------
// x: [M][H] residual stream.  On entry xq/xd already hold Q8_0(rms_norm_in(x)).
// Leaves ws.dn = raw down projection; the caller folds it into x.
int vxm_block_run(vxm_ctx *ctx, const vxm_block_dims &d, const vxm_block &b, vxm_workspace &ws, float *x,
                  int64_t M, const vxm_attn_site &site) {
    const int64_t qd = (int64_t)d.nh * d.hd, kvd = (int64_t)d.nkv * d.hd;
    const int var = ctx->quant_variant;
    int rc, np;
    const bool local = !site.causal && site.cache_pos0 == 0 && site.S > 0 && M % site.S == 0 &&
                       vxm_attention_local_fits(site.S, d.hd);
    // many tokens: k_rope_kv's work in the QKV GEMM's epilogue where its plan allows
    bool fused_rope = false;
    if (!local) {
        const vxm_qkv_epi qe{ws.q, site.kc, site.vc, d.rope_cs, site.seg_stride, d.nh, d.nkv, (int)d.hd,
                             site.pos0, site.S, d.no_rope, site.cap, site.cache_pos0};
        fused_rope = vxm_launch_qkv_rope(ctx, b.wqkv, ws.xq, ws.xd, M, qe, d.rope_rows, &rc);
        if (rc) return rc;
    }
    if (!fused_rope && (rc = vxm_launch_mul_mat_parts(ctx, b.wqkv, ws.xq, ws.xd, M, ws.qkv, ws.max_parts, &np)))
        return rc;
    if (local) {
        // fresh K/V within each segment: RoPE, attention and the output's Q8_0 in one launch
        if ((rc = vxm_launch_attention_local(ctx, vxm_parts{ws.qkv, np, M * (qd + 2 * kvd)}, M, d.nh, d.nkv, d.hd,
                                             site.S, site.pos0, d.rope_cs, d.rope_rows, d.no_rope, ws.xq, ws.xd,
                                             var)))
            return rc;
    } else {
        if (!fused_rope &&
            (rc = vxm_launch_rope_kv(ctx, vxm_parts{ws.qkv, np, M * (qd + 2 * kvd)}, M, d.nh, d.nkv, d.hd,
                                     site.pos0, site.S, d.rope_cs, d.rope_rows, d.no_rope, ws.q, site.kc, site.vc,
                                     site.cap, site.seg_stride, site.cache_pos0)))
            return rc;
        // attention with the Q8_0 of its output rows (the O projection's input)
        if ((rc = vxm_launch_attention(ctx, ws.q, site.kc, site.vc, ws.att, M, d.nh, d.nkv, d.hd, site.cap,
                                       site.seg_stride, site.S, site.cache_pos0, site.causal, ws.xq, ws.xd, var)))
            return rc;
    }
    if ((rc = vxm_launch_mul_mat_parts(ctx, b.wo, ws.xq, ws.xd, M, ws.o, ws.max_parts, &np))) return rc;
    // x = bf16(x + scale*bf16(o)); post-attention norm -> Q8_0
    if ((rc = vxm_launch_rmsnorm(ctx, x, vxm_parts{ws.o, np, M * d.H}, d.res_scale, b.g_post, M, d.H, d.eps, nullptr,
                                 ws.xq, ws.xd, var)))
        return rc;
    // gate/up: the tiled GEMM applies SwiGLU and the Q8_0 in its epilogue when it takes the
    // product, writing the down projection's input into the (then unused) gate/up buffer,
    // apart from its own input
    int8_t *pq = ws.xq;
    uint16_t *pd = ws.xd;
    int8_t *fq = (int8_t *)ws.gu;
    uint16_t *fd = (uint16_t *)(fq + ((M * d.F + 255) & ~(int64_t)255));
    if (vxm_launch_gate_up_swiglu(ctx, b.wgu, ws.xq, ws.xd, M, fq, fd, var, &rc)) {
        if (rc) return rc;
        pq = fq;
        pd = fd;
    } else {
        if ((rc = vxm_launch_mul_mat_parts(ctx, b.wgu, ws.xq, ws.xd, M, ws.gu, ws.max_parts, &np))) return rc;
        if ((rc = vxm_launch_swiglu_quant(ctx, vxm_parts{ws.gu, np, M * 2 * d.F}, M, d.F, 2 * d.F, ws.xq, ws.xd,
                                          nullptr, var)))
            return rc;
    }
    if ((rc = vxm_launch_mul_mat_parts(ctx, b.wd, pq, pd, M, ws.dn, ws.max_parts, &np))) return rc;
    ws.dn_out = vxm_parts{ws.dn, np, M * d.H};
    return VXM_OK;
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" int vxm_rms_norm(vxm_ctx *ctx, const float *x_dev, const float *gain_dev, int64_t rows, int64_t n,
                            float eps, float *y_dev, int8_t *xq_dev, uint16_t *xd_dev) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (!x_dev || (!y_dev && !xq_dev) || (xq_dev && !xd_dev) || rows < 0)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "rms_norm: bad arguments");
    return vxm_launch_rmsnorm(ctx, (float *)x_dev, vxm_parts{}, 1.0f, gain_dev, rows, n, eps, y_dev, xq_dev, xd_dev,
                              ctx->quant_variant);
}

extern "C" int vxm_kv_cache_create(vxm_ctx *ctx, int32_t n_layers, int32_t n_kv_heads, int32_t head_dim,
                                   int32_t capacity, vxm_kv_cache **out) {
    if (!ctx || !out) return VXM_ERR_INVALID_ARG;
    *out = nullptr;
    if (n_layers <= 0 || n_kv_heads <= 0 || head_dim <= 0 || capacity <= 0)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "kv cache: sizes must be positive");
    static std::atomic<uint64_t> next_id{1};
    vxm_kv_cache *kv = new vxm_kv_cache();
    kv->ctx = ctx;
    kv->id = next_id.fetch_add(1);
    kv->n_layers = n_layers;
    kv->nkv = n_kv_heads;
    kv->hd = head_dim;
    kv->cap = capacity;
    kv->layer_elems = (int64_t)n_kv_heads * capacity * head_dim;
    const size_t bytes = (size_t)kv->layer_elems * 2 * 2 * n_layers;
    if (hipMalloc(&kv->base, bytes) != hipSuccess) {
        (void)hipGetLastError();
        delete kv;
        return vxm_fail(ctx, VXM_ERR_OOM, "kv cache of %zu bytes failed", bytes);
    }
    VXM_HIP(ctx, hipMemsetAsync(kv->base, 0, bytes, ctx->stream));
    VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    *out = kv;
    return VXM_OK;
}

extern "C" int vxm_kv_cache_free(vxm_kv_cache *kv) {
    if (!kv) return VXM_ERR_INVALID_ARG;
    (void)hipStreamSynchronize(kv->ctx->stream);
    if (kv->base) (void)hipFree(kv->base);
    delete kv;
    return VXM_OK;
}

extern "C" int vxm_kv_cache_reset(vxm_kv_cache *kv) {
    if (!kv) return VXM_ERR_INVALID_ARG;
    kv->n_used = 0;
    return VXM_OK;
}

extern "C" int vxm_kv_cache_set_used(vxm_kv_cache *kv, int32_t n_used) {
    if (!kv) return VXM_ERR_INVALID_ARG;
    if (n_used < 0 || n_used > kv->cap)
        return vxm_fail(kv->ctx, VXM_ERR_INVALID_ARG, "kv cache: n_used %d outside [0, %d]", n_used, kv->cap);
    kv->n_used = n_used;
    return VXM_OK;
}

extern "C" int32_t vxm_kv_cache_used(const vxm_kv_cache *kv) { return kv ? kv->n_used : -1; }

extern "C" int vxm_kv_cache_layer(vxm_kv_cache *kv, int32_t layer, uint16_t **k_dev, uint16_t **v_dev) {
    if (!kv || !k_dev || !v_dev) return VXM_ERR_INVALID_ARG;
    if (layer < 0 || layer >= kv->n_layers)
        return vxm_fail(kv->ctx, VXM_ERR_INVALID_ARG, "kv cache: layer %d out of range", layer);
    *k_dev = kv->k(layer);
    *v_dev = kv->v(layer);
    return VXM_OK;
}

extern "C" int vxm_minicpm4_create(vxm_ctx *ctx, const vxm_minicpm4_config *cfg, const vxm_layer_weights_q8_0 *layers,
                                   const float *final_norm, vxm_minicpm4 **out) {
    if (!ctx || !cfg || !layers || !out) return VXM_ERR_INVALID_ARG;
    *out = nullptr;
    const vxm_minicpm4_config &c = *cfg;
    if (c.n_layers <= 0 || c.hidden_size <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 ||
        c.intermediate_size <= 0 || c.n_heads % c.n_kv_heads || c.head_dim % 2 || c.hidden_size % 32 ||
        c.intermediate_size % 32 || (c.n_heads * c.head_dim) % 32 || c.head_dim > 256)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "minicpm4 config: unsupported sizes");
    vxm_minicpm4 *m = new vxm_minicpm4();
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
    d.no_rope = c.no_rope;
    d.res_scale = (c.scale_depth > 0.0f) ? c.scale_depth / sqrtf((float)c.n_layers) : 1.0f;
    vxm_rope_setup(d, c.rope_theta, c.rope_freq_factors);
    int rc = VXM_OK;
    m->blocks.resize(c.n_layers);
    for (int l = 0; l < c.n_layers && rc == VXM_OK; l++) rc = vxm_block_upload(ctx, d, layers[l], m->blocks[l]);
    if (rc == VXM_OK) rc = upload_f32(ctx, final_norm, d.H, &m->final_norm);
    if (rc != VXM_OK) {
        vxm_minicpm4_free(m);
        return rc;
    }
    *out = m;
    return VXM_OK;
}

extern "C" int vxm_minicpm4_free(vxm_minicpm4 *m) {
    if (!m) return VXM_ERR_INVALID_ARG;
    (void)hipStreamSynchronize(m->ctx->stream);
    for (auto &b : m->blocks) vxm_block_free(m->ctx, b);
    vxm_persistent_free(m);
    if (m->final_norm) (void)hipFree(m->final_norm);
    vxm_rope_free(m->dims);
    vxm_ws_free(m->ws);
    delete m;
    return VXM_OK;
}

extern "C" int vxm_minicpm4_check(vxm_minicpm4 *m) {
    if (!m) return VXM_ERR_INVALID_ARG;
    return vxm_persistent_check(m);
}

extern "C" int vxm_minicpm4_set_layer_dump(vxm_minicpm4 *m, float *dump_dev) {
    if (!m) return VXM_ERR_INVALID_ARG;
    m->layer_dump = dump_dev;
    return VXM_OK;
}

extern "C" int vxm_minicpm4_set_decode_epoch(vxm_minicpm4 *m, uint32_t epoch) {
    if (!m) return VXM_ERR_INVALID_ARG;
    return vxm_persistent_set_epoch(m, epoch);
}

extern "C" int vxm_minicpm4_decode_epoch(vxm_minicpm4 *m, uint32_t *epoch) {
    if (!m || !epoch) return VXM_ERR_INVALID_ARG;
    return vxm_persistent_get_epoch(m, epoch);
}

extern "C" int vxm_minicpm4_set_decode_mode(vxm_minicpm4 *m, int mode) {
    if (!m) return VXM_ERR_INVALID_ARG;
    if (mode < VXM_DECODE_AUTO || mode > VXM_DECODE_PERSISTENT)
        return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "unknown decode mode %d", mode);
    m->decode_mode = mode;
    return VXM_OK;
}

static int check_run(vxm_minicpm4 *m, vxm_kv_cache *kv, const float *x, int64_t M, int32_t pos, int causal) {
    if (!m) return VXM_ERR_INVALID_ARG;
    if (!x || M <= 0 || pos < 0) return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "minicpm4: bad x / n_tokens / pos");
    if (causal) {
        if (!kv) return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "minicpm4: causal run needs a kv cache");
        if (kv->n_layers < m->cfg.n_layers || kv->nkv != m->dims.nkv || kv->hd != m->dims.hd)
            return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "minicpm4: kv cache shape does not match the model");
        if ((int64_t)pos + M > kv->cap)
            return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "minicpm4: pos %d + %lld tokens exceeds capacity %d", pos,
                            (long long)M, kv->cap);
    }
    return m->dims.no_rope ? VXM_OK : vxm_rope_ensure(m->ctx, m->dims, (int64_t)pos + M);
}

extern "C" int vxm_minicpm4_block(vxm_minicpm4 *m, vxm_kv_cache *kv, int32_t layer, float *x_dev, int64_t n_tokens,
                                  int32_t pos, int no_causal) {
    int rc = check_run(m, kv, x_dev, n_tokens, pos, !no_causal);
    if (rc) return rc;
    if (layer < 0 || layer >= m->cfg.n_layers)
        return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "minicpm4: layer %d out of range", layer);
    vxm_ctx *ctx = m->ctx;
    const vxm_block_dims &d = m->dims;
    const int64_t qd = (int64_t)d.nh * d.hd, kvd = (int64_t)d.nkv * d.hd;
    const int64_t local = no_causal ? (int64_t)d.nkv * n_tokens * d.hd : 0;
    if ((rc = vxm_ws_ensure(ctx, m->ws, n_tokens, d.H, qd, kvd, d.F, local))) return rc;
    vxm_attn_site site;
    if (no_causal) {
        site = vxm_attn_site{m->ws.lk, m->ws.lv, (int)n_tokens, 0, (int)n_tokens, pos, 0, 0};
    } else {
        site = vxm_attn_site{kv->k(layer), kv->v(layer), kv->cap, 0, (int)n_tokens, pos, pos, 1};
    }
    const vxm_block &b = m->blocks[layer];
    if ((rc = vxm_launch_rmsnorm(ctx, x_dev, vxm_parts{}, 1.0f, b.g_in, n_tokens, d.H, d.eps, nullptr, m->ws.xq,
                                 m->ws.xd, ctx->quant_variant)))
        return rc;
    if ((rc = vxm_block_run(ctx, d, b, m->ws, x_dev, n_tokens, site))) return rc;
    return vxm_launch_residual(ctx, x_dev, m->ws.dn_out, d.res_scale, n_tokens * d.H);
}

extern "C" int vxm_minicpm4_forward(vxm_minicpm4 *m, vxm_kv_cache *kv, float *x_dev, int64_t n_tokens, int32_t pos) {
    int rc = check_run(m, kv, x_dev, n_tokens, pos, 1);
    if (rc) return rc;
    vxm_ctx *ctx = m->ctx;
    const vxm_block_dims &d = m->dims;
    const int64_t qd = (int64_t)d.nh * d.hd, kvd = (int64_t)d.nkv * d.hd;
    const int var = ctx->quant_variant;
    if (n_tokens == 1 && m->decode_mode != VXM_DECODE_KERNELS) {
        const bool ok = vxm_persistent_supported(m, kv) && var == VXM_QUANT_X86;
        if (ok) {
            if ((rc = vxm_persistent_decode(m, kv, x_dev, pos, m->layer_dump))) return rc;
            kv->n_used = pos + 1;
            return VXM_OK;
        }
        if (m->decode_mode == VXM_DECODE_PERSISTENT)
            return vxm_fail(ctx, VXM_ERR_NOT_IMPLEMENTED,
                            "persistent decode: no kernel for this shape / device / quantizer");
    }
    if ((rc = vxm_ws_ensure(ctx, m->ws, n_tokens, d.H, qd, kvd, d.F, 0))) return rc;
    for (int l = 0; l < m->cfg.n_layers; l++) {
        const vxm_block &b = m->blocks[l];
        // residual of the previous layer's MLP folded into this layer's input norm
        if ((rc = vxm_launch_rmsnorm(ctx, x_dev, l ? m->ws.dn_out : vxm_parts{}, d.res_scale, b.g_in, n_tokens, d.H, d.eps,
                                     nullptr, m->ws.xq, m->ws.xd, var)))
            return rc;
        // the norm added the previous layer's residual in place: x_dev is this layer's input
        if (m->layer_dump)
            VXM_HIP(ctx, hipMemcpyAsync(m->layer_dump + (size_t)l * n_tokens * d.H, x_dev,
                                        (size_t)n_tokens * d.H * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream));
        vxm_attn_site site{kv->k(l), kv->v(l), kv->cap, 0, (int)n_tokens, pos, pos, 1};
        if ((rc = vxm_block_run(ctx, d, b, m->ws, x_dev, n_tokens, site))) return rc;
    }
    // last residual + final norm (in place), or the residual alone
    if (m->layer_dump && m->cfg.n_layers > 0) {
        // debug: the residual alone first, so the last layer's output can be copied out
        if ((rc = vxm_launch_residual(ctx, x_dev, m->ws.dn_out, d.res_scale, n_tokens * d.H))) return rc;
        VXM_HIP(ctx, hipMemcpyAsync(m->layer_dump + (size_t)m->cfg.n_layers * n_tokens * d.H, x_dev,
                                    (size_t)n_tokens * d.H * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream));
        if (m->final_norm &&
            (rc = vxm_launch_rmsnorm(ctx, x_dev, vxm_parts{}, 1.0f, m->final_norm, n_tokens, d.H, d.eps, x_dev, nullptr,
                                     nullptr, var)))
            return rc;
    } else if (m->final_norm) {
        if ((rc = vxm_launch_rmsnorm(ctx, x_dev, m->ws.dn_out, d.res_scale, m->final_norm, n_tokens, d.H, d.eps, x_dev,
                                     nullptr, nullptr, var)))
            return rc;
    } else if ((rc = vxm_launch_residual(ctx, x_dev, m->ws.dn_out, d.res_scale, n_tokens * d.H))) {
        return rc;
    }
    kv->n_used = pos + (int32_t)n_tokens;
    return VXM_OK;
}
