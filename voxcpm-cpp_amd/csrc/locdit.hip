// locdit.hip -- the LocDiT velocity network (vcpm_locdit_forward,
// src/locdit.c:216-400) and the CFM Euler loop with CFG-Zero*
// (src/gen_step.c:583-649, src/cfm_solver.c:27-93) on gfx950.
//
// The reference builds one graph holding the conditional and the
// unconditional LocDiT forward and computes it once per Euler step, reading
// both velocities back to the host for CFG-Zero* and the Euler update.  Here
// the two branches are ONE batch: the sequences [mu(2), t(1), cond(Pc), x(P)]
// of both branches are stacked as 2 segments of S = 3 + Pc + P rows, so every
// Q8_0 projection reads its weights once for M = 2S rows (the MFMA GEMM),
// attention stays within a segment, and the update kernel blends and steps x
// on the device.  A whole solve is stream-ordered with no host sync.
//
// Per solve (independent of the step): the time embeddings of every step
// (host sinusoid, one upload), both time MLPs, cond_proj.  Per step:
// quantize x -> in_proj -> assemble both segments -> 12 blocks -> RMSNorm of
// the x rows -> out_proj -> bias + BF16 + CFG-Zero* + Euler (one workgroup).
#include <math.h>
#include <string.h>

#include <vector>

#include "vxm_model.h"

struct vxm_locdit {
    vxm_ctx *ctx = nullptr;
    vxm_locdit_config cfg{};
    vxm_block_dims dims;
    std::vector<vxm_block> blocks;
    vxm_weight *in_proj = nullptr, *cond_proj = nullptr, *out_proj = nullptr;
    vxm_weight *t_w1 = nullptr, *t_w2 = nullptr, *dt_w1 = nullptr, *dt_w2 = nullptr;
    float *in_bias = nullptr, *cond_bias = nullptr, *out_bias = nullptr, *norm = nullptr;
    float *t_b1 = nullptr, *t_b2 = nullptr, *dt_b1 = nullptr, *dt_b2 = nullptr;
    vxm_workspace ws;
    // per-call buffers (grown on demand)
    void *buf = nullptr;
    size_t buf_bytes = 0;
    float *seq = nullptr;      // [2S][H] residual stream of both segments
    float *ch = nullptr;       // [Pc][H] raw cond_proj(cond)
    float *emb = nullptr;      // [R][H] sinusoid rows: steps' t, then dt
    float *th = nullptr;       // [R][H] time MLP hidden / output
    float *tc = nullptr;       // [R][H] bf16(t_feat + dt_feat) per step
    float *vo = nullptr;       // raw out_proj [n_seg P][feat] as K-split slices
    int vo_parts = 1;          //   (slice z at vo + z n_seg P feat)
    int8_t *aq = nullptr;      // Q8_0 scratch of the small projections
    uint16_t *ad = nullptr;
    int8_t *xq8 = nullptr;     // Q8_0 of x [P][feat]: in_proj's input, written by the
    uint16_t *xd8 = nullptr;   //   Euler update for the next evaluation
    // tc holds the time rows of the last time_features call as long as the buffers
    // keep their carving: tf_key = (rows, quantizer, path, the bits of dt and of every
    // step's t) of that call (empty: nothing valid), carve = the carving's (S, P, Pc, R,
    // base)
    std::vector<uint32_t> tf_key;
    std::vector<int64_t> carve;
    // pinned staging of the host-computed embeddings, reused once its copy is done
    float *pin = nullptr;
    size_t pin_floats = 0;
    hipEvent_t pin_done = nullptr;
    // the Euler loop of vxm_cfm_solve as a HIP graph, valid for one set of
    // arguments and device buffers (cfm_key); built on the second call with a key
    hipGraphExec_t cfm_exec = nullptr;
    std::vector<uint64_t> cfm_key, cfm_last_eager;
    int block_mode = VXM_DECODE_AUTO;   // blocks launch by launch, or all in one persistent launch
    // debug: each evaluation writes the rows entering every block and the last block's
    // output (residual added) here, [n_layers + 1][rows][H] (null: off)
    float *block_dump = nullptr;
    vxm_lpersist *lp = nullptr;
};

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------
// h = bf16(silu(bf16(x + b))) (vcpm_time_mlp_forward's first layer,
// src/locdit.c:150-153), silu(v) = v / (1 + expf(-v)).
__global__ void k_bias_silu_bf16(const float *__restrict__ x, const float *__restrict__ b, float *__restrict__ y,
                                 int64_t rows, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * n) return;
    float v = x[i];
    if (b) v = v + b[i % n];
    v = vxm_bf16(v);
    y[i] = vxm_bf16(__fdiv_rn(v, 1.0f + expf(-v)));
}

// tc[r] = bf16(bf16(tt[r] + tb) + bf16(dd + db)) -- t_feat + dt_feat with the
// second-layer biases (src/locdit.c:155-158 and :288); dd is one row.
__global__ void k_time_combine(const float *__restrict__ tt, const float *__restrict__ tb,
                               const float *__restrict__ dd, const float *__restrict__ db, float *__restrict__ tc,
                               int64_t rows, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * n) return;
    const int64_t j = i % n;
    float a = tt[i], d = dd[j];
    if (tb) a = a + tb[j];
    if (db) d = d + db[j];
    tc[i] = vxm_bf16(vxm_bf16(a) + vxm_bf16(d));
}

// Both segments' sequences [mu(2), t(1), cond(Pc), x(P)] (src/locdit.c:296-317):
// segment g < n_mu takes mu, the others zero rows; cond and x rows are the
// raw projections plus bias, BF16 (src/locdit.c:232-252).  One workgroup per row.
// The rows of one evaluation's sequence (src/locdit.c:216-300): per segment
// mu (2 rows, or zeros), the time row, bf16(cond_proj + bias) of the cond
// rows, bf16(in_proj(x) + bias) of the x rows.  The x rows' in_proj is formed
// here from the Q8_0 of x (xq8 / xd8, K = feat) and the Q8_0 weight (wq / wd,
// rows of feat): per output the exact int32 block sums, each times
// d_w * d_x, added in block order -- the GEMV's terms (its lane tree adds
// the terms of K = 64, two blocks, in the same single addition).
__global__ void k_locdit_assemble(float *__restrict__ seq, const float *__restrict__ mu, int n_mu,
                                  const float *__restrict__ tc, const float *__restrict__ ch,
                                  const float *__restrict__ cb, const int8_t *__restrict__ xq8,
                                  const uint16_t *__restrict__ xd8, const int8_t *__restrict__ wq,
                                  const uint16_t *__restrict__ wd, const float *__restrict__ xb, int S, int Pc, int H,
                                  int feat) {
    const int row = blockIdx.x, g = row / S, r = row % S;
    float *dst = seq + (int64_t)row * H;
    if (r >= 3 + Pc) {
        const int xi = r - 3 - Pc, nb = feat / 32;
        const int8_t *xr = xq8 + (int64_t)xi * feat;
        const uint16_t *xs = xd8 + (int64_t)xi * nb;
        for (int i = threadIdx.x; i < H; i += blockDim.x) {
            const int8_t *wr = wq + (int64_t)i * feat;
            float acc = 0.0f;
            for (int b = 0; b < nb; b++) {
                int si = 0;
#pragma unroll
                for (int k = 0; k < 32; k += 16) {
                    const int4 wv = *(const int4 *)(wr + 32 * b + k), xv = *(const int4 *)(xr + 32 * b + k);
                    si = vxm_dot16(wv, xv, si);
                }
                const float t = (float)si * (vxm_h2f(wd[(int64_t)i * nb + b]) * vxm_h2f(xs[b]));
                acc = b ? acc + t : t;
            }
            float v = acc;
            if (xb) v = v + xb[i];
            dst[i] = vxm_bf16(v);
        }
        return;
    }
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        float v;
        if (r < 2) {
            v = (g < n_mu && mu) ? mu[r * H + i] : 0.0f;
        } else if (r == 2) {
            v = tc[i];
        } else {
            v = ch[(int64_t)(r - 3) * H + i];
            if (cb) v = v + cb[i];
            v = vxm_bf16(v);
        }
        dst[i] = v;
    }
}

// Velocities v = bf16(vo + out_bias) of the conditional rows [0, n) and,
// with CFG, the unconditional rows [n, 2n); CFG-Zero* (src/cfm_solver.c:65-93:
// st = bf16(bf16(sum bf16(p q)) / bf16(sum bf16(q q) + 1e-8)), sums in double
// in element order, v = bf16(ns + bf16(cfg * bf16(p - ns))), ns = bf16(q st));
// x = bf16(x + bf16(dt * v)) (src/gen_step.c:624-627).  One workgroup;
// dynamic LDS holds the 2n products (n <= kCfmMaxN).  vo is out_proj's K-split
// slices, added in slice order as they are read (the fix-up launch's sums).
// With xq8 the updated x also goes out as Q8_0 (the next evaluation's in_proj
// input; the activation rule of `variant`, 32 lanes per block).  Thread t holds
// elements t + 256 k in registers from its first loads (every slice, the bias
// and x requested at once) to its stores, so the serial sums are the only wait
// between them.
constexpr int kCfmMaxN = 2048;   // 2 x 2048 doubles = 32 KiB of LDS
constexpr int kCfmNPT = kCfmMaxN / 256;
__device__ __forceinline__ float parts_at(const vxm_parts &v, int64_t j) {
    float t[VXM_MAX_PARTS];
#pragma unroll
    for (int z = 0; z < VXM_MAX_PARTS; z++) t[z] = z < v.n ? v.p[z * v.stride + j] : 0.0f;
    float s = t[0];
#pragma unroll
    for (int z = 1; z < VXM_MAX_PARTS; z++)
        if (z < v.n) s = s + t[z];
    return s;
}

__global__ __launch_bounds__(256) void k_cfm_update(const vxm_parts vo, const float *__restrict__ ob,
                                                    int feat, int n, int use_cfg, float cfg_value, float dt,
                                                    float *__restrict__ x, float *__restrict__ v_out,
                                                    int8_t *__restrict__ xq8, uint16_t *__restrict__ xd8,
                                                    int variant) {
    extern __shared__ double prod[];   // [2][n]
    __shared__ float st_sh;
    const int t = threadIdx.x;
    float pv[kCfmNPT], qv[kCfmNPT], xv[kCfmNPT];
#pragma unroll
    for (int k = 0; k < kCfmNPT; k++) {
        const int j = t + 256 * k;
        if (j >= n) break;
        float p = parts_at(vo, j);
        if (ob) p = p + ob[j % feat];
        pv[k] = vxm_bf16(p);
        if (use_cfg) {
            float q = parts_at(vo, n + j);
            if (ob) q = q + ob[j % feat];
            qv[k] = vxm_bf16(q);
        }
        if (x) xv[k] = x[j];
    }
    if (use_cfg) {
#pragma unroll
        for (int k = 0; k < kCfmNPT; k++) {
            const int j = t + 256 * k;
            if (j >= n) break;
            prod[j] = (double)vxm_bf16(pv[k] * qv[k]);
            prod[n + j] = (double)vxm_bf16(qv[k] * qv[k]);
        }
        __syncthreads();
        if (t == 0) {
            // in element order; 16 elements' products read ahead of their additions (n % 32 == 0)
            double dot = 0.0, sq = 0.0;
            for (int j0 = 0; j0 < n; j0 += 16) {
                double a[16], b[16];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    a[i] = prod[j0 + i];
                    b[i] = prod[n + j0 + i];
                }
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    dot += a[i];
                    sq += b[i];
                }
            }
            const float dot_b = vxm_bf16((float)dot);
            const float norm_b = vxm_bf16((float)sq + 1.0e-8f);
            st_sh = vxm_bf16(__fdiv_rn(dot_b, norm_b));
        }
        __syncthreads();
    }
    const float st = use_cfg ? st_sh : 0.0f;
    const float cfg_b = vxm_bf16(cfg_value);
    // n % 32 == 0: the 32 lanes of a half wave hold one whole block of x
#pragma unroll
    for (int k = 0; k < kCfmNPT; k++) {
        const int j = t + 256 * k;
        if (j >= n) break;
        const float p = pv[k];
        float v = p;
        if (use_cfg) {
            const float q = qv[k];
            const float ns = vxm_bf16(q * st);
            const float gd = vxm_bf16(p - ns);
            const float gg = vxm_bf16(cfg_b * gd);
            v = vxm_bf16(ns + gg);
        }
        if (v_out) v_out[j] = v;
        if (x) {
            const float xn = vxm_bf16(xv[k] + vxm_bf16(dt * v));
            x[j] = xn;
            if (xq8) {
                // quantize_row_q8_0 of the block (k_quantize_q8_0's rule): d = amax / 127 as
                // fp16, q = round(x * id)
                float amax = fabsf(xn);
#pragma unroll
                for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
                const float d = __fdiv_rn(amax, 127.0f);
                float id;
                if (variant == VXM_QUANT_X86) id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
                else id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
                float q;
                if (variant == VXM_QUANT_X86) q = fminf(fmaxf(rintf(xn * id), -128.0f), 127.0f);
                else q = roundf(xn * id);
                xq8[j] = (int8_t)(int)q;
                if ((j & 31) == 0) xd8[j / 32] = vxm_f2h(d);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// host driver
// ---------------------------------------------------------------------------
static int upload_vec(vxm_ctx *ctx, const float *src, int64_t n, float **out) {
    *out = nullptr;
    if (!src) return VXM_OK;
    if (hipMalloc((void **)out, n * 4) != hipSuccess) {
        (void)hipGetLastError();
        return vxm_fail(ctx, VXM_ERR_OOM, "locdit: vector upload failed");
    }
    VXM_HIP(ctx, hipMemcpy(*out, src, n * 4, hipMemcpyHostToDevice));
    return VXM_OK;
}

static int ensure_bufs(vxm_locdit *m, int64_t S, int64_t P, int64_t Pc, int64_t R) {
    vxm_ctx *ctx = m->ctx;
    const int64_t H = m->dims.H, feat = m->cfg.feat_dim;
    const int64_t kq = std::max<int64_t>(std::max<int64_t>(H, feat), m->cfg.cond_dim);
    const int64_t arows = std::max<int64_t>(std::max<int64_t>(P, Pc), std::max<int64_t>(R, 2 * P));
    struct Part { size_t bytes; void **dst; };
    std::vector<Part> parts = {
        {(size_t)(2 * S * H * 4), (void **)&m->seq},
        {(size_t)(std::max<int64_t>(Pc, 1) * H * 4), (void **)&m->ch},
        {(size_t)(R * H * 4), (void **)&m->emb},      {(size_t)(R * H * 4), (void **)&m->th},
        {(size_t)(R * H * 4), (void **)&m->tc},
        {(size_t)(VXM_MAX_PARTS * 2 * P * feat * 4), (void **)&m->vo},
        {(size_t)(arows * kq), (void **)&m->aq},      {(size_t)(arows * (kq / 32) * 2), (void **)&m->ad},
        {(size_t)(P * feat), (void **)&m->xq8},       {(size_t)(P * (feat / 32) * 2), (void **)&m->xd8},
    };
    size_t total = 0;
    for (auto &p : parts) total += (p.bytes + 255) & ~(size_t)255;
    if (total > m->buf_bytes) {
        VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (m->buf) VXM_HIP(ctx, hipFree(m->buf));
        m->buf = nullptr;
        m->buf_bytes = 0;
        if (hipMalloc(&m->buf, total) != hipSuccess) {
            (void)hipGetLastError();
            return vxm_fail(ctx, VXM_ERR_OOM, "locdit: buffers of %zu bytes failed", total);
        }
        m->buf_bytes = total;
    }
    char *b = (char *)m->buf;
    for (auto &p : parts) { *p.dst = b; b += (p.bytes + 255) & ~(size_t)255; }
    // a new carving moves tc (and lays other buffers over its old rows)
    const std::vector<int64_t> cv = {S, P, Pc, R, (int64_t)(uintptr_t)m->buf};
    if (cv != m->carve) {
        m->tf_key.clear();
        m->carve = cv;
    }
    // staging for R embedding rows
    const size_t need = (size_t)(R * H);
    if (need > m->pin_floats) {
        if (m->pin) {
            VXM_HIP(ctx, hipEventSynchronize(m->pin_done));
            VXM_HIP(ctx, hipHostFree(m->pin));
            m->pin = nullptr;
            m->pin_floats = 0;
        }
        if (hipHostMalloc((void **)&m->pin, need * 4, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            return vxm_fail(ctx, VXM_ERR_OOM, "locdit: pinned staging failed");
        }
        m->pin_floats = need;
    }
    return VXM_OK;
}

static int elementwise_grid(int64_t n) { return (int)((n + 255) / 256); }

// Time conditioning of `rows` steps: emb rows [0, rows) hold the steps'
// t embeddings and row `rows` the dt embedding.  Leaves tc[rows][H].
static int time_features(vxm_locdit *m, const float *t_host, int rows, float dt) {
    vxm_ctx *ctx = m->ctx;
    const int64_t H = m->dims.H;
    const int var = ctx->quant_variant;
    // The time rows are a function of the steps' t and dt (the weights are the model's)
    // and of the context settings that pick the quantizer and the kernels: a solve with
    // the same schedule as the last one (every patch of an utterance) finds them in tc
    // already.  Under a caller's capture nothing runs now, so nothing is reused and
    // nothing is remembered.
    std::vector<uint32_t> key((size_t)rows + 4);
    key[0] = (uint32_t)rows;
    key[1] = (uint32_t)var;
    key[2] = (uint32_t)ctx->path;
    memcpy(&key[3], &dt, 4);
    if (rows > 0) memcpy(&key[4], t_host, (size_t)rows * 4);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    VXM_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cap));
    if (cap == hipStreamCaptureStatusNone && !m->tf_key.empty() && key == m->tf_key) return VXM_OK;
    m->tf_key.clear();
    // the pinned buffer may still feed the previous call's copy
    VXM_HIP(ctx, hipEventSynchronize(m->pin_done));
    for (int r = 0; r < rows; r++) {
        int rc = vxm_host_sinusoid_embed(t_host[r], (int32_t)H, m->pin + (int64_t)r * H);
        if (rc) return vxm_fail(ctx, rc, "locdit: sinusoid embedding of width %lld", (long long)H);
    }
    (void)vxm_host_sinusoid_embed(dt, (int32_t)H, m->pin + (int64_t)rows * H);
    VXM_HIP(ctx, hipMemcpyAsync(m->emb, m->pin, (size_t)(rows + 1) * H * 4, hipMemcpyHostToDevice, ctx->stream));
    VXM_HIP(ctx, hipEventRecord(m->pin_done, ctx->stream));
    int rc;
    // time_mlp over the t rows, delta_time_mlp over the dt row (src/locdit.c:140-159)
    float *dd = m->th + (int64_t)rows * H;
    if ((rc = vxm_launch_quantize(ctx, m->emb, rows + 1, H, var, m->aq, m->ad))) return rc;
    if ((rc = vxm_launch_mul_mat(ctx, m->t_w1, m->aq, m->ad, rows, m->th))) return rc;
    if ((rc = vxm_launch_mul_mat(ctx, m->dt_w1, m->aq + (int64_t)rows * H, m->ad + (int64_t)rows * (H / 32), 1,
                                 dd)))
        return rc;
    hipLaunchKernelGGL(k_bias_silu_bf16, dim3(elementwise_grid(rows * H)), dim3(256), 0, ctx->stream, m->th,
                       m->t_b1, m->th, (int64_t)rows, H);
    VXM_CHECK_LAUNCH(ctx);
    hipLaunchKernelGGL(k_bias_silu_bf16, dim3(elementwise_grid(H)), dim3(256), 0, ctx->stream, dd, m->dt_b1, dd,
                       (int64_t)1, H);
    VXM_CHECK_LAUNCH(ctx);
    if ((rc = vxm_launch_quantize(ctx, m->th, rows + 1, H, var, m->aq, m->ad))) return rc;
    if ((rc = vxm_launch_mul_mat(ctx, m->t_w2, m->aq, m->ad, rows, m->emb))) return rc;
    if ((rc = vxm_launch_mul_mat(ctx, m->dt_w2, m->aq + (int64_t)rows * H, m->ad + (int64_t)rows * (H / 32), 1,
                                 m->emb + (int64_t)rows * H)))
        return rc;
    hipLaunchKernelGGL(k_time_combine, dim3(elementwise_grid(rows * H)), dim3(256), 0, ctx->stream, m->emb,
                       m->t_b2, m->emb + (int64_t)rows * H, m->dt_b2, m->tc, (int64_t)rows, H);
    VXM_CHECK_LAUNCH(ctx);
    if (cap == hipStreamCaptureStatusNone) m->tf_key = std::move(key);
    return VXM_OK;
}

// One batched LocDiT evaluation of n_seg segments (segment 0 takes mu when
// n_mu = 1) for the time row tc_row; x [P][feat] on the device (its Q8_0
// already in xq8 / xd8 when x_quantized: the Euler update wrote it), ch already
// holds the raw cond projection.  Leaves vo = raw out_proj [n_seg * P][feat]
// as K-split slices (vo_parts).
static int dit_eval(vxm_locdit *m, const float *x, bool x_quantized, int P, int Pc, int n_seg, const float *mu,
                    int n_mu, const float *tc_row) {
    vxm_ctx *ctx = m->ctx;
    const vxm_block_dims &d = m->dims;
    const int64_t H = d.H, feat = m->cfg.feat_dim, S = 3 + Pc + P, M = n_seg * S;
    const int var = ctx->quant_variant;
    int rc;
    if (!x_quantized && (rc = vxm_launch_quantize(ctx, x, P, feat, var, m->xq8, m->xd8))) return rc;
    hipLaunchKernelGGL(k_locdit_assemble, dim3((unsigned)M), dim3(256), 0, ctx->stream, m->seq, mu, n_mu, tc_row,
                       m->ch, m->cond_bias, m->xq8, m->xd8, m->in_proj->qs, m->in_proj->d, m->in_bias, (int)S, Pc,
                       (int)H, (int)feat);
    VXM_CHECK_LAUNCH(ctx);
    // non-causal blocks, rope positions from 0 in each segment, fresh K/V per segment
    bool residual_added = false;   // the last block's residual already in seq (debug dump)
    const bool persistent = m->cfg.n_layers > 0 && vxm_locdit_persistent_pick(ctx, d, M, (int)S, m->block_mode);
    if (m->block_mode == VXM_DECODE_PERSISTENT && !persistent)
        return vxm_fail(ctx, VXM_ERR_NOT_IMPLEMENTED, "locdit: no persistent block kernel for this shape / device");
    // the final RMSNorm of the x rows fused into the single launch (needs the gain)
    const bool fin_fused = persistent && m->norm;
    if (persistent) {
        // all blocks in one launch; seq then holds the last block's output, residual included
        vxm_lfinal fin;
        if (fin_fused) {
            fin.g = m->norm;
            fin.r0 = 3 + Pc;
            fin.q = m->aq;
            fin.d = m->ad;
        }
        if ((rc = vxm_locdit_persistent_run(ctx, d, m->blocks, &m->lp, m->seq, M, (int)S, m->block_dump, fin)))
            return rc;
    } else {
        const vxm_attn_site site{m->ws.lk, m->ws.lv, (int)S, (int64_t)d.nkv * S * d.hd, (int)S, 0, 0, 0};
        for (int l = 0; l < m->cfg.n_layers; l++) {
            const vxm_block &b = m->blocks[l];
            if ((rc = vxm_launch_rmsnorm(ctx, m->seq, l ? m->ws.dn_out : vxm_parts{}, 1.0f, b.g_in, M, H, d.eps,
                                         nullptr, m->ws.xq, m->ws.xd, var)))
                return rc;
            // the norm added the previous block's residual in place: seq holds block l's input
            if (m->block_dump)
                VXM_HIP(ctx, hipMemcpyAsync(m->block_dump + (size_t)l * M * H, m->seq, (size_t)M * H * sizeof(float),
                                            hipMemcpyDeviceToDevice, ctx->stream));
            if ((rc = vxm_block_run(ctx, d, b, m->ws, m->seq, M, site))) return rc;
        }
        if (m->block_dump && m->cfg.n_layers) {
            // debug: the last residual on its own (the final norm then adds none), and the rows out
            if ((rc = vxm_launch_residual(ctx, m->seq, m->ws.dn_out, 1.0f, M * H))) return rc;
            residual_added = true;
            VXM_HIP(ctx, hipMemcpyAsync(m->block_dump + (size_t)m->cfg.n_layers * M * H, m->seq,
                                        (size_t)M * H * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream));
        }
    }
    // last residual + final RMSNorm of the x rows of each segment (src/locdit.c:373-390)
    // one launch over the P x rows of every segment (rows 3 + Pc .. S - 1 of each), unless
    // the single launch did it
    if (!fin_fused) {
        const int64_t r0 = 3 + Pc;
        const vxm_parts &dn = m->ws.dn_out;
        const vxm_parts delta =
            m->cfg.n_layers && !persistent && !residual_added ? vxm_parts{dn.p + r0 * H, dn.n, dn.stride} : vxm_parts{};
        if ((rc = vxm_launch_rmsnorm(ctx, m->seq + r0 * H, delta, 1.0f, m->norm, (int64_t)n_seg * P, H, d.eps,
                                     nullptr, m->aq, m->ad, var, P, (int)S)))
            return rc;
    }
    // the K-split slices stay separate: the Euler update adds them as it reads them
    return vxm_launch_mul_mat_parts(ctx, m->out_proj, m->aq, m->ad, (int64_t)n_seg * P, m->vo, VXM_MAX_PARTS,
                                    &m->vo_parts);
}

static int check_dims(vxm_locdit *m, const float *x, const float *cond, int32_t P, int32_t Pc) {
    if (!x || P <= 0 || Pc < 0 || (Pc > 0 && !cond))
        return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "locdit: bad x / cond / P / Pc");
    const int64_t S = 3 + (int64_t)Pc + P;
    if ((int64_t)P * m->cfg.feat_dim > kCfmMaxN)
        return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "locdit: P * feat_dim = %lld exceeds %d",
                        (long long)P * m->cfg.feat_dim, kCfmMaxN);
    if (S > 4096) return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "locdit: sequence of %lld rows", (long long)S);
    return VXM_OK;
}

static int prepare(vxm_locdit *m, const float *cond, int32_t P, int32_t Pc, int R, int n_seg) {
    vxm_ctx *ctx = m->ctx;
    const vxm_block_dims &d = m->dims;
    const int64_t S = 3 + (int64_t)Pc + P, qd = (int64_t)d.nh * d.hd, kvd = (int64_t)d.nkv * d.hd;
    int rc;
    if ((rc = vxm_ws_ensure(ctx, m->ws, n_seg * S, d.H, qd, kvd, d.F, (int64_t)n_seg * d.nkv * S * d.hd)))
        return rc;
    if ((rc = vxm_rope_ensure(ctx, m->dims, S))) return rc;
    if ((rc = ensure_bufs(m, S, P, Pc, R + 1))) return rc;
    if (Pc > 0) {
        if ((rc = vxm_launch_quantize(ctx, cond, Pc, m->cfg.cond_dim, ctx->quant_variant, m->aq, m->ad))) return rc;
        if ((rc = vxm_launch_mul_mat(ctx, m->cond_proj, m->aq, m->ad, Pc, m->ch))) return rc;
    }
    return VXM_OK;
}

// Everything a recorded Euler loop depends on: arguments, the device buffers
// its launches address, and the context settings that pick its kernels.
static std::vector<uint64_t> cfm_graph_key(vxm_locdit *m, const float *x, const float *cond, const float *mu,
                                           int P, int Pc, int n_steps, float cfg_value, int schedule, int zero_star) {
    vxm_ctx *ctx = m->ctx;
    uint32_t cfg_bits;
    memcpy(&cfg_bits, &cfg_value, 4);
    return {(uint64_t)(uintptr_t)x, (uint64_t)(uintptr_t)cond, (uint64_t)(uintptr_t)mu, (uint64_t)P, (uint64_t)Pc,
            (uint64_t)n_steps, cfg_bits, (uint64_t)schedule, (uint64_t)zero_star, (uint64_t)ctx->path,
            (uint64_t)ctx->quant_variant, (uint64_t)ctx->n_cu, (uint64_t)(uintptr_t)m->ws.base, m->ws.bytes,
            (uint64_t)(uintptr_t)m->buf, m->buf_bytes, (uint64_t)(uintptr_t)m->dims.rope_cs,
            (uint64_t)m->dims.rope_rows, (uint64_t)(uintptr_t)ctx->parts_buf, ctx->parts_bytes,
            (uint64_t)(uintptr_t)ctx->split_buf, ctx->split_bytes};
}

static void cfm_graph_drop(vxm_locdit *m) {
    if (m->cfm_exec) (void)hipGraphExecDestroy(m->cfm_exec);
    m->cfm_exec = nullptr;
    m->cfm_key.clear();
}

// x_q8: the updated x also goes out as Q8_0 (xq8 / xd8) for the next evaluation
static int cfm_update(vxm_locdit *m, int P, int n_seg, int use_cfg, float cfg_value, float dt, float *x,
                      float *v_out, bool x_q8) {
    vxm_ctx *ctx = m->ctx;
    const int feat = m->cfg.feat_dim, n = P * feat;
    const size_t lds = use_cfg ? (size_t)2 * n * sizeof(double) : 0;
    const vxm_parts vo{m->vo, m->vo_parts, (int64_t)n_seg * n};
    hipLaunchKernelGGL(k_cfm_update, dim3(1), dim3(256), lds, ctx->stream, vo, m->out_bias, feat, n, use_cfg,
                       cfg_value, dt, x, v_out, x_q8 ? m->xq8 : nullptr, x_q8 ? m->xd8 : nullptr,
                       ctx->quant_variant);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" int vxm_locdit_free(vxm_locdit *m) {
    if (!m) return VXM_ERR_INVALID_ARG;
    vxm_ctx *ctx = m->ctx;
    (void)hipStreamSynchronize(ctx->stream);
    for (auto &b : m->blocks) vxm_block_free(ctx, b);
    for (vxm_weight *w : {m->in_proj, m->cond_proj, m->out_proj, m->t_w1, m->t_w2, m->dt_w1, m->dt_w2})
        if (w) vxm_weight_free(ctx, w);
    for (float *p : {m->in_bias, m->cond_bias, m->out_bias, m->norm, m->t_b1, m->t_b2, m->dt_b1, m->dt_b2})
        if (p) (void)hipFree(p);
    cfm_graph_drop(m);
    vxm_locdit_persistent_free(m->lp);
    vxm_rope_free(m->dims);
    vxm_ws_free(m->ws);
    if (m->buf) (void)hipFree(m->buf);
    if (m->pin) (void)hipHostFree(m->pin);
    if (m->pin_done) (void)hipEventDestroy(m->pin_done);
    delete m;
    return VXM_OK;
}

extern "C" int vxm_locdit_create(vxm_ctx *ctx, const vxm_locdit_config *cfg, const vxm_locdit_weights_q8_0 *w,
                                 vxm_locdit **out) {
    if (!ctx || !cfg || !w || !out) return VXM_ERR_INVALID_ARG;
    *out = nullptr;
    const vxm_locdit_config &c = *cfg;
    if (c.n_layers < 0 || c.hidden_size <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 ||
        c.intermediate_size <= 0 || c.n_heads % c.n_kv_heads || c.head_dim % 2 || c.hidden_size % 32 ||
        c.intermediate_size % 32 || (c.n_heads * c.head_dim) % 32 || c.head_dim > 256 || c.feat_dim <= 0 ||
        c.feat_dim % 32 || c.cond_dim <= 0 || c.cond_dim % 32 || c.hidden_size > 8192)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "locdit config: unsupported sizes");
    if (!w->in_proj || !w->cond_proj || !w->out_proj || !w->t_w1 || !w->t_w2 || !w->dt_w1 || !w->dt_w2 ||
        (c.n_layers > 0 && !w->layers))
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "locdit weights: a projection is NULL");
    vxm_locdit *m = new vxm_locdit();
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
    d.no_rope = 0;          // rope stays on in the DiT blocks (src/locdit.c:336-339)
    d.res_scale = 1.0f;     // no DeepNorm scale (src/locdit.c:355)
    vxm_rope_setup(d, c.rope_theta, c.rope_freq_factors);
    int rc = VXM_OK;
    if (hipEventCreateWithFlags(&m->pin_done, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        rc = vxm_fail(ctx, VXM_ERR_BACKEND, "locdit: event creation failed");
    }
    m->blocks.resize(c.n_layers);
    for (int l = 0; l < c.n_layers && rc == VXM_OK; l++) rc = vxm_block_upload(ctx, d, w->layers[l], m->blocks[l]);
    const int64_t H = d.H;
    if (rc == VXM_OK) rc = vxm_upload_q8_0(ctx, w->in_proj, H, c.feat_dim, &m->in_proj);
    if (rc == VXM_OK) rc = vxm_upload_q8_0(ctx, w->cond_proj, H, c.cond_dim, &m->cond_proj);
    if (rc == VXM_OK) rc = vxm_upload_q8_0(ctx, w->out_proj, c.feat_dim, H, &m->out_proj);
    if (rc == VXM_OK) rc = vxm_upload_q8_0(ctx, w->t_w1, H, H, &m->t_w1);
    if (rc == VXM_OK) rc = vxm_upload_q8_0(ctx, w->t_w2, H, H, &m->t_w2);
    if (rc == VXM_OK) rc = vxm_upload_q8_0(ctx, w->dt_w1, H, H, &m->dt_w1);
    if (rc == VXM_OK) rc = vxm_upload_q8_0(ctx, w->dt_w2, H, H, &m->dt_w2);
    if (rc == VXM_OK) rc = upload_vec(ctx, w->in_bias, H, &m->in_bias);
    if (rc == VXM_OK) rc = upload_vec(ctx, w->cond_bias, H, &m->cond_bias);
    if (rc == VXM_OK) rc = upload_vec(ctx, w->out_bias, c.feat_dim, &m->out_bias);
    if (rc == VXM_OK) rc = upload_vec(ctx, w->norm, H, &m->norm);
    if (rc == VXM_OK) rc = upload_vec(ctx, w->t_b1, H, &m->t_b1);
    if (rc == VXM_OK) rc = upload_vec(ctx, w->t_b2, H, &m->t_b2);
    if (rc == VXM_OK) rc = upload_vec(ctx, w->dt_b1, H, &m->dt_b1);
    if (rc == VXM_OK) rc = upload_vec(ctx, w->dt_b2, H, &m->dt_b2);
    if (rc != VXM_OK) {
        vxm_locdit_free(m);
        return rc;
    }
    *out = m;
    return VXM_OK;
}

extern "C" int vxm_locdit_set_block_dump(vxm_locdit *m, float *dump_dev) {
    if (!m) return VXM_ERR_INVALID_ARG;
    m->block_dump = dump_dev;
    return VXM_OK;
}

extern "C" int vxm_locdit_set_block_mode(vxm_locdit *m, int mode) {
    if (!m) return VXM_ERR_INVALID_ARG;
    if (mode < VXM_DECODE_AUTO || mode > VXM_DECODE_PERSISTENT)
        return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "unknown block mode %d", mode);
    if (mode != m->block_mode) {
        // a recorded Euler loop holds the other path's launches
        (void)hipStreamSynchronize(m->ctx->stream);
        cfm_graph_drop(m);
        m->cfm_last_eager.clear();
        m->block_mode = mode;
    }
    return VXM_OK;
}

extern "C" int vxm_locdit_check(vxm_locdit *m) {
    if (!m) return VXM_ERR_INVALID_ARG;
    return vxm_locdit_persistent_check(m->ctx, m->lp);
}

extern "C" int vxm_locdit_forward(vxm_locdit *m, const float *x_dev, const float *cond_dev, int32_t P, int32_t Pc,
                                  float t, float dt, const float *mu_dev, float *out_dev) {
    if (!m) return VXM_ERR_INVALID_ARG;
    int rc = check_dims(m, x_dev, cond_dev, P, Pc);
    if (rc) return rc;
    if (!out_dev) return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "locdit: out is NULL");
    if ((rc = prepare(m, cond_dev, P, Pc, 1, 1))) return rc;
    if ((rc = time_features(m, &t, 1, dt))) return rc;
    if ((rc = dit_eval(m, x_dev, false, P, Pc, 1, mu_dev, mu_dev ? 1 : 0, m->tc))) return rc;
    // velocity = bf16(out_proj + bias), no CFG and no Euler step
    return cfm_update(m, P, 1, 0, 1.0f, 0.0f, nullptr, out_dev, false);
}

extern "C" int vxm_cfm_solve(vxm_locdit *m, float *x_dev, const float *cond_dev, int32_t P, int32_t Pc,
                             const float *mu_dev, int32_t n_steps, float cfg_value, int32_t schedule,
                             int32_t use_zero_star) {
    if (!m) return VXM_ERR_INVALID_ARG;
    int rc = check_dims(m, x_dev, cond_dev, P, Pc);
    if (rc) return rc;
    if (n_steps < 0 || n_steps > 1024 || (schedule != VXM_CFM_SWAY && schedule != VXM_CFM_UNIFORM))
        return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "cfm: n_steps %d / schedule %d", n_steps, schedule);
    if (n_steps == 0) return VXM_OK;
    const int use_cfg = (cfg_value != 1.0f && mu_dev != nullptr);   // src/gen_step.c:475
    const int n_seg = use_cfg ? 2 : 1;
    const int zs = use_zero_star ? vxm_host_cfm_zero_star_steps(n_steps) : 0;
    const int live = n_steps > zs ? n_steps - zs : 0;
    if (live == 0) return VXM_OK;
    std::vector<float> ts(live), dts(live);
    for (int k = 0; k < live; k++) {
        const int step = zs + k;
        const float t = vxm_host_cfm_t(step, n_steps, schedule);
        const float nt = vxm_host_cfm_t(step + 1, n_steps, schedule);
        ts[k] = t;
        // step_size = bf16(-(t - next_t)) (src/gen_step.c:598)
        const float dtv = -(t - nt);
        uint32_t u;
        memcpy(&u, &dtv, 4);
        u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
        memcpy(&dts[k], &u, 4);
    }
    if ((rc = prepare(m, cond_dev, P, Pc, live, n_seg))) return rc;
    if ((rc = time_features(m, ts.data(), live, 0.0f))) return rc;   // dt input is 0 (src/gen_step.c:601)
    const int64_t H = m->dims.H;
    // the whole loop in one launch of the single-launch blocks where it applies: the row
    // owners assemble each step's rows, one workgroup forms out_proj, CFG-Zero* and the
    // Euler step (the steps of k_locdit_assemble, k_rmsnorm and k_cfm_update)
    const int64_t S = 3 + (int64_t)Pc + P, M = n_seg * S;
    vxm_lsolve sv;
    sv.n_eval = live;
    sv.dts = dts.data();
    sv.tc = m->tc;
    sv.mu = mu_dev;
    sv.n_mu = 1;
    sv.ch = Pc ? m->ch : nullptr;
    sv.cb = m->cond_bias;
    sv.in_proj = m->in_proj;
    sv.in_b = m->in_bias;
    sv.out_proj = m->out_proj;
    sv.out_b = m->out_bias;
    sv.P = P;
    sv.Pc = Pc;
    sv.feat = m->cfg.feat_dim;
    sv.n_seg = n_seg;
    sv.use_cfg = use_cfg;
    sv.cfg = cfg_value;
    sv.x = x_dev;
    sv.xq0 = m->xq8;
    sv.xd0 = m->xd8;
    const bool fused = m->cfg.n_layers > 0 && m->norm && !m->block_dump &&
                       vxm_locdit_persistent_pick(m->ctx, m->dims, M, (int)S, m->block_mode) &&
                       vxm_locdit_persistent_solve_fits(m->ctx, m->dims, M, (int)S, sv);
    auto euler_loop = [&]() -> int {
        if (fused) {
            int r = vxm_launch_quantize(m->ctx, x_dev, P, m->cfg.feat_dim, m->ctx->quant_variant, m->xq8, m->xd8);
            if (r) return r;
            vxm_lfinal fin;
            fin.g = m->norm;
            fin.r0 = 3 + Pc;
            return vxm_locdit_persistent_run(m->ctx, m->dims, m->blocks, &m->lp, m->seq, M, (int)S, nullptr, fin, &sv);
        }
        for (int k = 0; k < live; k++) {
            // from the second step on, x's Q8_0 comes from the previous step's update
            int r = dit_eval(m, x_dev, k > 0, P, Pc, n_seg, mu_dev, 1, m->tc + (int64_t)k * H);
            if (r == VXM_OK) r = cfm_update(m, P, n_seg, use_cfg, cfg_value, dts[k], x_dev, nullptr, k + 1 < live);
            if (r) return r;
        }
        return VXM_OK;
    };
    // The loop is ~100 dependent launches per step: replay it as one HIP graph
    // when this call's key matches the recorded one; record it on the second
    // call with a key (the first, eager, call grows every buffer it needs, so
    // nothing allocates under capture).
    vxm_ctx *ctx = m->ctx;
    const std::vector<uint64_t> key = cfm_graph_key(m, x_dev, cond_dev, mu_dev, P, Pc, n_steps, cfg_value,
                                                    schedule, use_zero_star);
    if (m->cfm_exec && key == m->cfm_key) {
        VXM_HIP(ctx, hipGraphLaunch(m->cfm_exec, ctx->stream));
        return VXM_OK;
    }
    if (key != m->cfm_last_eager) {
        m->cfm_last_eager = key;
        return euler_loop();
    }
    cfm_graph_drop(m);
    VXM_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    rc = euler_loop();
    hipGraph_t graph = nullptr;
    const hipError_t ec = hipStreamEndCapture(ctx->stream, &graph);
    if (rc == VXM_OK && ec != hipSuccess)
        rc = vxm_fail(ctx, VXM_ERR_BACKEND, "cfm: graph capture failed: %s", hipGetErrorString(ec));
    if (rc == VXM_OK && hipGraphInstantiate(&m->cfm_exec, graph, nullptr, nullptr, 0) != hipSuccess) {
        m->cfm_exec = nullptr;
        rc = vxm_fail(ctx, VXM_ERR_BACKEND, "cfm: graph instantiation failed");
    }
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipGetLastError();
    if (rc) return rc;
    m->cfm_key = key;
    VXM_HIP(ctx, hipGraphLaunch(m->cfm_exec, ctx->stream));
    return VXM_OK;
}
