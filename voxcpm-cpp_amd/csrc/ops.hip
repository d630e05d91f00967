// ops.hip -- the non-matmul pieces of the MiniCPM4 block on gfx950:
// RMSNorm (+ residual, + Q8_0 activation quantization), NEOX RoPE with the
// f16 KV-cache append, softmax attention over the f16 cache, SwiGLU (+ Q8_0
// quantization).  Every rounding step follows the reference graph
// (src/minicpm4.c) as restated by the oracle; contraction is off, so each
// a*b+c below rounds twice like the reference's scalar code.
#include "vxm_ops.h"

// ---------------------------------------------------------------------------
// block-wide reductions (blockDim.x == 256)
// ---------------------------------------------------------------------------
__device__ __forceinline__ double block_sum_f64(double v, double *sh) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) t += sh[i];
    return t;
}

// The same for sums of squares in a tree order (each row of 16 lanes on DPP: xor 1,
// xor 2, half mirror, mirror; the wave's four rows read back as scalars).  Every lane
// of the block must be active.  The squares of BF16 values have 16 significant
// bits (of fp32 values, 24), so while a row's squares span less than about 2^26
// (values within 2^13; fp32 values within 2^9) every partial sum of up to 2^11 of
// them is exact in double and any order gives ggml's sequential double.  Beyond
// that the tree and the sequential order can round the double differently, and
// (float)(sum / n) can then differ by one ulp.
__device__ __forceinline__ double block_sum_exact_f64(double v, double *sh) {
    auto dpp = [](double x, auto ctrl) {
        const long long b = __double_as_longlong(x);
        const int lo = __builtin_amdgcn_update_dpp(0, (int)b, decltype(ctrl)::value, 0xF, 0xF, false);
        const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), decltype(ctrl)::value, 0xF, 0xF, false);
        return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
    };
    v = v + dpp(v, std::integral_constant<int, 0xB1>{});
    v = v + dpp(v, std::integral_constant<int, 0x4E>{});
    v = v + dpp(v, std::integral_constant<int, 0x141>{});
    v = v + dpp(v, std::integral_constant<int, 0x140>{});
    const long long b = __double_as_longlong(v);
    double w = 0.0;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)b, 16 * r);
        const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(b >> 32), 16 * r);
        w += __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
    }
    const int wv = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[wv] = w;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) t += sh[i];
    return t;
}

__device__ __forceinline__ float block_max_f32(float v, float *sh) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float t = sh[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) t = fmaxf(t, sh[i]);
    return t;
}

// ---------------------------------------------------------------------------
// [h = bf16(h + scale * bf16(delta))]; y = vcpm_rms_norm(h) (src/minicpm4.c:132-152):
// ggml_rms_norm (sum of fp32 squares in double, mean = (float)(sum/n),
// scale = 1/sqrtf(mean + eps)), BF16, * gain, BF16.  Outputs y (fp32, if
// non-null) and its Q8_0 quantization (xq/xd, if non-null).
// One workgroup per row: 128 threads for n <= 1024, else 256; n % 8 == 0 and
// n <= 8 * 256 * VXM_NORM_CHUNKS.
// ---------------------------------------------------------------------------
#define VXM_NORM_CHUNKS 4
__global__ __launch_bounds__(256) void k_rmsnorm(float *__restrict__ h, const vxm_parts delta, float res_scale,
                                                 const float *__restrict__ gain, int n, float eps,
                                                 float *__restrict__ y, int8_t *__restrict__ xq,
                                                 uint16_t *__restrict__ xd, int variant, int seg_rows,
                                                 int seg_stride) {
    __shared__ double shd[4];
    // output row `row`; its h / delta row: seg_rows rows of every seg_stride (the identity
    // when seg_rows == seg_stride)
    const int row = blockIdx.x;
    const int64_t hrow = (int64_t)(row / seg_rows) * seg_stride + row % seg_rows;
    float *hr = h + hrow * n;
    const float *dr = delta.p ? delta.p + hrow * n : nullptr;
    float v[VXM_NORM_CHUNKS][8];
    // the gain, fetched with the row (it is needed right after the reduction)
    float4 gl[VXM_NORM_CHUNKS][2];
#pragma unroll
    for (int c = 0; c < VXM_NORM_CHUNKS; c++) {
        const int base = (c * (int)blockDim.x + threadIdx.x) * 8;
        if (gain && base < n) {
            gl[c][0] = *(const float4 *)(gain + base);
            gl[c][1] = *(const float4 *)(gain + base + 4);
        } else {
            gl[c][0] = gl[c][1] = make_float4(1, 1, 1, 1);
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int c = 0; c < VXM_NORM_CHUNKS; c++) {
        const int base = (c * (int)blockDim.x + threadIdx.x) * 8;
        if (base < n) {
            float4 a = *(const float4 *)(hr + base), b = *(const float4 *)(hr + base + 4);
            v[c][0] = a.x; v[c][1] = a.y; v[c][2] = a.z; v[c][3] = a.w;
            v[c][4] = b.x; v[c][5] = b.y; v[c][6] = b.z; v[c][7] = b.w;
            if (dr) {
                // K-split slices: all loads in flight, then added in order
                float4 ps[VXM_MAX_PARTS], qs[VXM_MAX_PARTS];
#pragma unroll
                for (int z = 0; z < VXM_MAX_PARTS; z++)
                    if (z < delta.n) {
                        ps[z] = *(const float4 *)(dr + z * delta.stride + base);
                        qs[z] = *(const float4 *)(dr + z * delta.stride + base + 4);
                    }
                float4 p = ps[0], q = qs[0];
#pragma unroll
                for (int z = 1; z < VXM_MAX_PARTS; z++)
                    if (z < delta.n) {
                        p.x = p.x + ps[z].x; p.y = p.y + ps[z].y; p.z = p.z + ps[z].z; p.w = p.w + ps[z].w;
                        q.x = q.x + qs[z].x; q.y = q.y + qs[z].y; q.z = q.z + qs[z].z; q.w = q.w + qs[z].w;
                    }
                float dd[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    float o = vxm_bf16(dd[i]);
                    if (res_scale != 1.0f) o = o * res_scale;
                    v[c][i] = vxm_bf16(v[c][i] + o);
                }
                *(float4 *)(hr + base) = make_float4(v[c][0], v[c][1], v[c][2], v[c][3]);
                *(float4 *)(hr + base + 4) = make_float4(v[c][4], v[c][5], v[c][6], v[c][7]);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) ss += (double)(v[c][i] * v[c][i]);
        }
    }
    const double tot = block_sum_exact_f64(ss, shd);
    if (!y && !xq) return;
    const float mean = (float)(tot / (double)n);
    const float sc = __fdiv_rn(1.0f, __fsqrt_rn(mean + eps));
#pragma unroll
    for (int c = 0; c < VXM_NORM_CHUNKS; c++) {
        const int base = (c * (int)blockDim.x + threadIdx.x) * 8;
        if (base >= n) continue;   // whole 32-blocks live in 4 consecutive lanes: n % 32 == 0
        float o[8];
        const float4 g0 = gl[c][0], g1 = gl[c][1];
        const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float t = vxm_bf16(v[c][i] * sc);
            o[i] = gain ? vxm_bf16(t * g[i]) : t;
        }
        if (y) {
            float *yr = y + (int64_t)row * n + base;
            *(float4 *)yr = make_float4(o[0], o[1], o[2], o[3]);
            *(float4 *)(yr + 4) = make_float4(o[4], o[5], o[6], o[7]);
        }
        if (xq) {
            const int64_t e = (int64_t)row * n + base;
            quant_block_4lanes(o, variant, xq + e, xd + e / 32, (threadIdx.x & 3) == 0);
        }
    }
}

int vxm_launch_rmsnorm(vxm_ctx *ctx, float *h, vxm_parts delta, float res_scale, const float *gain,
                       int64_t rows, int64_t n, float eps, float *y, int8_t *xq, uint16_t *xd, int variant,
                       int seg_rows, int seg_stride) {
    if (rows <= 0) return VXM_OK;
    if (seg_rows <= 0) seg_rows = seg_stride = (int)rows;
    if (seg_stride < seg_rows) return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "rms_norm: segment stride below its rows");
    if (n % 32 != 0 || n > 8 * 256 * VXM_NORM_CHUNKS)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "rms_norm: n=%lld must be a multiple of 32 and <= %d",
                        (long long)n, 8 * 256 * VXM_NORM_CHUNKS);
    // rows of up to 1024 values fit 128 threads (8 values each): two waves reduce faster than four
    const unsigned threads = n <= 8 * 128 ? 128 : 256;
    hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(threads), 0, ctx->stream, h, delta, res_scale, gain,
                       (int)n, eps, y, xq, xd, variant, seg_rows, seg_stride);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

// ---------------------------------------------------------------------------
// Q/K/V post-processing of vcpm_attention (src/minicpm4.c:270-320): BF16 of
// the projections, NEOX RoPE (pair (i, i+hd/2) rotated by the angle of
// ggml_rope_ext, theta_i / ff_i with theta_0 = pos, theta_{i+1} = theta_i *
// theta_scale; BF16), K and V appended to the f16 cache.  cs holds the
// host-computed (cos, sin) of every (position, pair): [position][hd/2].  qkv: raw projections [M][qd + 2*kvd].
// Tokens come in segments of S (one per CFG branch); token t has position
// pos0 + t % S and segment t / S, whose cache starts at seg * seg_stride.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rope_kv(const vxm_parts qkv, int nh, int nkv, int hd,
                                                 int pos0, int S, const float2 *__restrict__ cs,
                                                 int no_rope, float *__restrict__ q_out, uint16_t *__restrict__ kc,
                                                 uint16_t *__restrict__ vc, int cap, int64_t seg_stride,
                                                 int cache_pos0) {
    const int t = blockIdx.x;
    const int seg = t / S, ti = t % S;
    const int pos = pos0 + ti;
    const int half = hd / 2;
    const int qd = nh * hd, kvd = nkv * hd;
    const float *row = qkv.p + (int64_t)t * (qd + 2 * kvd);
    // the projection: its K-split slices added in order
    auto at = [&](int i) {
        float v = row[i];
        for (int z = 1; z < qkv.n; z++) v = v + row[z * qkv.stride + i];
        return v;
    };
    uint16_t *kseg = kc + seg * seg_stride, *vseg = vc + seg * seg_stride;
    const int cpos = cache_pos0 + ti;
    // q and k pairs
    for (int idx = threadIdx.x; idx < (nh + nkv) * half; idx += blockDim.x) {
        const int head = idx / half, i = idx % half;
        const bool isq = head < nh;
        // q and k rows are stored pair-interleaved: head row 2i is dim i, 2i+1 is dim i + hd/2
        const int src = isq ? head * hd : qd + (head - nh) * hd;
        float x0 = vxm_bf16(at(src + 2 * i)), x1 = vxm_bf16(at(src + 2 * i + 1));
        float y0 = x0, y1 = x1;
        if (!no_rope) {
            const float2 r = cs[(int64_t)pos * half + i];
            const float c = r.x, s = r.y;
            y0 = vxm_bf16(x0 * c - x1 * s);
            y1 = vxm_bf16(x0 * s + x1 * c);
        }
        if (isq) {
            float *qo = q_out + (int64_t)t * qd + head * hd;
            qo[i] = y0;
            qo[i + half] = y1;
        } else {
            const int kh = head - nh;
            uint16_t *kd = kseg + ((int64_t)kh * cap + cpos) * hd;
            kd[i] = vxm_f2h(y0);
            kd[i + half] = vxm_f2h(y1);
        }
    }
    // v
    for (int idx = threadIdx.x; idx < kvd; idx += blockDim.x) {
        const int kh = idx / hd, dd = idx % hd;
        const float val = vxm_bf16(at(qd + kvd + idx));
        vseg[((int64_t)kh * cap + cpos) * hd + dd] = vxm_f2h(val);
    }
}

int vxm_launch_rope_kv(vxm_ctx *ctx, vxm_parts qkv, int64_t M, int nh, int nkv, int hd, int pos0, int S,
                       const float2 *cs, int cs_rows, int no_rope, float *q_out, uint16_t *kc,
                       uint16_t *vc, int cap, int64_t seg_stride, int cache_pos0) {
    if (M <= 0) return VXM_OK;
    if (!no_rope && (!cs || pos0 + std::min<int64_t>(M, S) > cs_rows))
        return vxm_fail(ctx, VXM_ERR_BACKEND, "rope: table holds %d positions, %lld needed", cs_rows,
                        (long long)(pos0 + std::min<int64_t>(M, S)));
    hipLaunchKernelGGL(k_rope_kv, dim3((unsigned)M), dim3(256), 0, ctx->stream, qkv, nh, nkv, hd, pos0, S,
                       cs, no_rope, q_out, kc, vc, cap, seg_stride, cache_pos0);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

// ---------------------------------------------------------------------------
// gqa_group_attn (src/minicpm4.c:232-248) for one (token, query head):
// s_j = (k_j . q) * (1/sqrt(hd)); p = softmax (sum in double, scaled by
// (float)(1/sum)); out = sum_j p_j v_j.  Query head h reads kv head
// h / (nh / nkv).  Causal: token t of a segment sees cache rows
// [0, kv_base + t]; non-causal: rows [0, S).  Scores live in LDS (kv_len <= cap).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_attention(const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                   const uint16_t *__restrict__ vc, float *__restrict__ out, int nh,
                                                   int nkv, int hd, int cap, int64_t seg_stride, int S,
                                                   int kv_base, int causal) {
    extern __shared__ float lds[];
    __shared__ float red[8];
    __shared__ double redd[4];
    const int h = blockIdx.x, t = blockIdx.y;
    const int seg = t / S, ti = t % S;
    const int kvh = h / (nh / nkv);
    const int kv_len = causal ? kv_base + ti + 1 : S;
    const uint16_t *kb = kc + seg * seg_stride + (int64_t)kvh * cap * hd;
    const uint16_t *vb = vc + seg * seg_stride + (int64_t)kvh * cap * hd;
    float *sq = lds;              // [hd]
    float *sc = lds + hd;         // [kv_len]
    float *part = sc + cap;       // [256]
    const float *qr = q + (int64_t)t * nh * hd + h * hd;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) sq[d] = qr[d];
    __syncthreads();
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn((float)hd));
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < kv_len; j += blockDim.x) {
        const uint16_t *kr = kb + (int64_t)j * hd;
        float s = 0.0f;
        for (int d = 0; d < hd; d++) s += vxm_h2f(kr[d]) * sq[d];
        s = s * scale;
        sc[j] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_max_f32(mx, red);
    double sum = 0.0;
    for (int j = threadIdx.x; j < kv_len; j += blockDim.x) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += (double)e;
    }
    sum = block_sum_f64(sum, redd);
    const float inv = (float)(1.0 / sum);
    for (int j = threadIdx.x; j < kv_len; j += blockDim.x) sc[j] = sc[j] * inv;
    __syncthreads();
    // out[d] = sum_j v[j][d] * p_j: thread (sl, d) sums a contiguous j-slice,
    // slices are added in order (hd <= 256, checked by the launcher).
    const int slices = blockDim.x / hd;
    const int d = threadIdx.x % hd, sl = threadIdx.x / hd;
    float acc = 0.0f;
    if (sl < slices) {
        const int jper = (kv_len + slices - 1) / slices;
        const int j0 = sl * jper, j1 = min(kv_len, j0 + jper);
        for (int j = j0; j < j1; j++) acc += vxm_h2f(vb[(int64_t)j * hd + d]) * sc[j];
    }
    part[threadIdx.x] = acc;
    __syncthreads();
    if (sl == 0) {
        float tot = 0.0f;
        for (int s2 = 0; s2 < slices; s2++) tot += part[s2 * hd + d];
        out[(int64_t)t * nh * hd + h * hd + d] = tot;
    }
}

// ---------------------------------------------------------------------------
// The same attention for many queries of one segment (prefill), on f16 MFMA
// (v_mfma_f32_32x32x16_f16: lane l supplies A[l%32][8(l/32)..+8] and
// B[8(l/32)..+8][l%32]; result register v of lane l is row 8(v/4) + 4(l/32)
// + v%4, column l%32).  One workgroup of 8 waves (2 per SIMD) per (query
// head, tile of AQ = 32 consecutive tokens).  Every phase is a chain of
// dependent loads and products, so the work is cut into as many independent
// chains as the waves:
//   scores  S = Q K^T * scale, the tile's 32-key blocks of [0, kv_end) split
//           into 8 contiguous runs, one per wave.  The queries are BF16 values
//           and the cache holds f16, both exact in f16, so every product is
//           exact and only the fp32 summation order differs from the
//           reference's.  A lane's B operands (16 bytes of a key row) come
//           straight from the cache; every load of a wave (Q, K and its V
//           rows) is issued at once;
//   softmax per query row over its own kv_len, on the scores in registers
//           (computed as S^T = K Q^T, so a lane holds 16 keys of one query per
//           block): max over the lane's keys, its partner lane's and the 8
//           waves', e = expf(s - max), sums in double the same way, p = e *
//           (float)(1 / sum), 0 past kv_len;
//   output  wave (kq, dh) = (w % 4, w / 4) forms the partial P V of key quarter
//           kq for dims [64 dh, 64 dh + 64): P enters the MFMA as f16 hi + lo
//           halves (two products, ~22 bits of p), V through the wave's own LDS
//           buffer, transposed as key-pair words; the four key quarters are
//           added in order at the end.
// The score buffer holds AKV keys: longer spans take k_attention_mfma_long.
// ---------------------------------------------------------------------------
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
constexpr int AQ = 32, AKV = 512, ATH = 512;

#ifdef VXM_ATTN_TRACE
// per-workgroup timestamps (s_memtime) of wave 0: [workgroup][entry, scores, softmax, P V, end]
__device__ uint64_t vxm_attn_trace[4096 * 8];
#define VXM_ATTN_TS(k)                                                                                        \
    do {                                                                                                      \
        if (tid == 0 && blockIdx.x * gridDim.y + blockIdx.y < 4096)                                           \
            vxm_attn_trace[(blockIdx.x * gridDim.y + blockIdx.y) * 8 + (k)] = __builtin_amdgcn_s_memtime(); \
    } while (0)
extern "C" int vxm_attn_trace_read(void *host, size_t bytes) {   // profiling builds only
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(vxm_attn_trace), bytes, 0, hipMemcpyDeviceToHost);
}
#else
#define VXM_ATTN_TS(k) \
    do {               \
    } while (0)
#endif

template <int HD>
__global__ __launch_bounds__(ATH) void k_attention_mfma(const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                        const uint16_t *__restrict__ vc, float *__restrict__ out,
                                                        int M, int nh, int nkv, int cap, int kv_base, int causal,
                                                        int8_t *__restrict__ xq, uint16_t *__restrict__ xd,
                                                        int variant) {
    constexpr int NW = ATH / 64;       // waves
    constexpr int SP = AKV + 4;        // fp32 P row pitch
    constexpr int KSTEPS = HD / 16;    // MFMA steps over the head dimension
    constexpr int HDH = HD / 2;        // dims of one output half
    constexpr int DT = HDH / 32;       // 32-dim output tiles per wave
    constexpr int VP = 32 + 8;         // f16 pitch of a wave's transposed V block (32 keys + pad)
    constexpr int VITEMS = 16 * (HDH / 8) / 64;   // (key pair, 8-dim chunk) items per lane and block
    constexpr int SB = AKV / 32 / NW;  // most score blocks of one wave
    constexpr int VB = AKV / 32 / 4;   // most P V blocks of one key quarter
    __shared__ __align__(16) float Sc[AQ * SP];
    __shared__ __align__(16) _Float16 Vt[NW][HDH * VP];
    __shared__ float smax[AQ][NW];
    __shared__ double ssum[AQ][NW];
    constexpr int QP = HD + 8;         // f16 pitch of the query tile (16-byte pad)
    __shared__ __align__(16) _Float16 Qh[AQ * QP];
    static_assert(NW == 8 && VITEMS >= 1 && 4 * AQ * HD <= AQ * SP, "8 waves; the key-quarter sums reuse P's buffer");
    const int h = blockIdx.x, t0 = blockIdx.y * AQ, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kvh = h / (nh / nkv);
    const uint16_t *kb = kc + (int64_t)kvh * cap * HD;
    const uint16_t *vb = vc + (int64_t)kvh * cap * HD;
    const int nq = min(AQ, M - t0);
    const int kv_end = causal ? kv_base + t0 + nq : M;
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn((float)HD));
    const int lr = lane & 31, lh = lane >> 5;
    const int nblk = (kv_end + 31) / 32;
    const int bw0 = nblk * wave / NW, nbw = nblk * (wave + 1) / NW - bw0;   // this wave's score blocks
    const int kq = wave & 3, dh = wave >> 2;
    const int bq0 = nblk * kq / 4, nbq = nblk * (kq + 1) / 4 - bq0;        // its P V blocks
    VXM_ATTN_TS(0);

    // loads in the order they are needed: the query tile (once per workgroup, 4 values
    // per thread and round, into LDS as f16) and the rows of the wave's score blocks'
    // keys (A operands: 16 bytes of key 32 b + lr's row per step); after the scores, the
    // V rows of its P V blocks (item (key pair p, dims 8c .. 8c+7 of its half), p = item
    // % 16 fastest).
    // Every load is unconditional (rows past the span, and blocks past a wave's share,
    // read the clamped last row, whose values are masked or multiplied by p = 0), so the
    // loads stay in one straight-line block and each product waits only for its own.
    constexpr int QL = AQ * HD / 4 / ATH;   // float4 query loads per thread
    float4 qf[QL];
#pragma unroll
    for (int u = 0; u < QL; u++) {
        const int i = (u * ATH + tid) * 4, r = i / HD, d = i % HD;
        qf[u] = *(const float4 *)(q + (int64_t)(t0 + min(r, nq - 1)) * nh * HD + h * HD + d);
    }
    uint4 kr[SB][KSTEPS];
#pragma unroll
    for (int i = 0; i < SB; i++) {
        const int key = min(32 * (bw0 + i) + lr, kv_end - 1);
#pragma unroll
        for (int kk = 0; kk < KSTEPS; kk++) kr[i][kk] = *(const uint4 *)(kb + (int64_t)key * HD + 16 * kk + 8 * lh);
    }
#pragma unroll
    for (int u = 0; u < QL; u++) {
        const int i = (u * ATH + tid) * 4, r = i / HD, d = i % HD;
        const bool qlive = r < nq;
        _Float16 *dst = Qh + r * QP + d;
        dst[0] = (_Float16)(qlive ? qf[u].x : 0.0f);
        dst[1] = (_Float16)(qlive ? qf[u].y : 0.0f);
        dst[2] = (_Float16)(qlive ? qf[u].z : 0.0f);
        dst[3] = (_Float16)(qlive ? qf[u].w : 0.0f);
    }
    __syncthreads();

    // pass 1: scores of this wave's blocks in registers, as S^T = K Q^T (the key rows are
    // the A operands, the queries the B operands): value v of block i in lane (lr, lh) is
    // query t0 + lr, key 32 (bw0 + i) + kr(v) with kr(v) = 8 (v / 4) + 4 lh + v % 4
    v8h qa[KSTEPS];   // B operands: query t0 + lr, dims 16 kk + 8 lh .. + 8
#pragma unroll
    for (int kk = 0; kk < KSTEPS; kk++) qa[kk] = *(const v8h *)(Qh + lr * QP + 16 * kk + 8 * lh);
    v16f sc[SB];
#pragma unroll
    for (int i = 0; i < SB; i++) {
        v16f c = v16f{};
#pragma unroll
        for (int kk = 0; kk < KSTEPS; kk++) {
            v8h av;
            __builtin_memcpy(&av, &kr[i][kk], 16);
            c = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, qa[kk], c, 0, 0, 0);
        }
#pragma unroll
        for (int v = 0; v < 16; v++) sc[i][v] = c[v] * scale;
    }
    // the V rows of the wave's P V blocks, in flight during the softmax
    const uint16_t *vbh = vb + HDH * dh;
    uint4 vr[VB][VITEMS][2];
#pragma unroll
    for (int i = 0; i < VB; i++)
#pragma unroll
        for (int u = 0; u < VITEMS; u++) {
            const int item = u * 64 + lane, r = 32 * (bq0 + i) + 2 * (item % 16), d = 8 * (item / 16);
#pragma unroll
            for (int e = 0; e < 2; e++)
                vr[i][u][e] = *(const uint4 *)(vbh + (int64_t)min(r + e, kv_end - 1) * HD + d);
        }
    VXM_ATTN_TS(1);
    // pass 2: softmax of query t0 + lr over its kv_len: max over the lane's keys, its
    // partner lane's (lr + 32: the other half of every block) and the 8 waves' (through
    // LDS); e = exp(s - max), the double sums the same way; p = e * (float)(1 / sum),
    // 0 past kv_len
    const int kvl = lr < nq ? (causal ? kv_base + t0 + lr + 1 : M) : 0;
    auto live = [&](int i, int v) { return i < nbw && 32 * (bw0 + i) + 8 * (v >> 2) + 4 * lh + (v & 3) < kvl; };
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < SB; i++)
#pragma unroll
        for (int v = 0; v < 16; v++)
            if (live(i, v)) m = fmaxf(m, sc[i][v]);
    m = fmaxf(m, __shfl_xor(m, 32));
    if (lh == 0) smax[lr][wave] = m;
    __syncthreads();
    m = smax[lr][0];
#pragma unroll
    for (int w = 1; w < NW; w++) m = fmaxf(m, smax[lr][w]);
    double sum = 0.0;
#pragma unroll
    for (int i = 0; i < SB; i++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const float e = live(i, v) ? expf(sc[i][v] - m) : 0.0f;
            sc[i][v] = e;
            sum += (double)e;
        }
    sum += __shfl_xor(sum, 32);
    if (lh == 0) ssum[lr][wave] = sum;
    __syncthreads();
    sum = ssum[lr][0];
#pragma unroll
    for (int w = 1; w < NW; w++) sum += ssum[lr][w];
    const float inv = kvl > 0 ? (float)(1.0 / sum) : 0.0f;
    // P rows in LDS: the lane's 4 runs of 4 consecutive keys per block
#pragma unroll
    for (int i = 0; i < SB; i++) {
        if (i >= nbw) break;
#pragma unroll
        for (int r4 = 0; r4 < 4; r4++)
            *(float4 *)(Sc + lr * SP + 32 * (bw0 + i) + 8 * r4 + 4 * lh) =
                make_float4(sc[i][4 * r4] * inv, sc[i][4 * r4 + 1] * inv, sc[i][4 * r4 + 2] * inv,
                            sc[i][4 * r4 + 3] * inv);
    }
    __syncthreads();
    VXM_ATTN_TS(2);
    // pass 3: partial O = P V of key quarter kq, dims [64 dh, 64 dh + 64); each block's V
    // goes to this wave's LDS buffer as key-pair words, dims as rows
    v16f o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) o[dt] = v16f{};
    _Float16 *vt = Vt[wave];
#pragma unroll
    for (int i = 0; i < VB; i++) {
        if (i >= nbq) break;
        const int b = bq0 + i;
#pragma unroll
        for (int u = 0; u < VITEMS; u++) {
            const int item = u * 64 + lane, r = 2 * (item % 16), d = 8 * (item / 16);
            const uint32_t a[4] = {vr[i][u][0].x, vr[i][u][0].y, vr[i][u][0].z, vr[i][u][0].w};
            const uint32_t bb[4] = {vr[i][u][1].x, vr[i][u][1].y, vr[i][u][1].z, vr[i][u][1].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                *(uint32_t *)(vt + (d + 2 * e) * VP + r) = (a[e] & 0xffffu) | (bb[e] << 16);
                *(uint32_t *)(vt + (d + 2 * e + 1) * VP + r) = (a[e] >> 16) | (bb[e] & 0xffff0000u);
            }
        }
        // the wave's own LDS writes are seen by its later reads (one wave, in order)
#pragma unroll
        for (int ks = 0; ks < 32; ks += 16) {
            const float *pr = Sc + lr * SP + 32 * b + ks + 8 * lh;
            const float4 p0 = *(const float4 *)pr, p1 = *(const float4 *)(pr + 4);
            const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
            v8h ahi, alo;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const _Float16 hi = (_Float16)pv[e];
                ahi[e] = hi;
                alo[e] = (_Float16)(pv[e] - (float)hi);
            }
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const v8h bv = *(const v8h *)(vt + (32 * dt + lr) * VP + ks + 8 * lh);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi, bv, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo, bv, o[dt], 0, 0, 0);
            }
        }
    }
    // the key quarters in order through LDS (P's buffer is free)
    __syncthreads();
    VXM_ATTN_TS(3);
    float *red = Sc;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int v = 0; v < 16; v++)
            red[(kq * AQ + 8 * (v >> 2) + 4 * lh + (v & 3)) * HD + HDH * dh + 32 * dt + lr] = o[dt][v];
    __syncthreads();
    if (xq) {
        // Q8_0 of the output rows (the O projection's input; the arithmetic of
        // k_quantize_q8_0): 8 values per lane, 4 lanes per 32-value block, the
        // blocks of a row never crossing a head
        for (int i = 8 * tid; i < AQ * HD; i += 8 * ATH) {
            const int qi = i / HD, d = i % HD;
            float v[8];
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                float4 s = *(const float4 *)(red + i + 4 * hf);
#pragma unroll
                for (int w = 1; w < 4; w++) {
                    const float4 t = *(const float4 *)(red + w * AQ * HD + i + 4 * hf);
                    s.x = s.x + t.x; s.y = s.y + t.y; s.z = s.z + t.z; s.w = s.w + t.w;
                }
                v[4 * hf] = s.x; v[4 * hf + 1] = s.y; v[4 * hf + 2] = s.z; v[4 * hf + 3] = s.w;
            }
            const int64_t o = (int64_t)(t0 + min(qi, nq - 1)) * nh * HD + h * HD + d;
            quant_block_4lanes(v, variant, xq + o, xd + o / 32, (tid & 3) == 0, qi < nq);
        }
    } else {
        for (int i = 4 * tid; i < AQ * HD; i += 4 * ATH) {
            const int qi = i / HD, d = i % HD;
            if (qi >= nq) continue;
            float4 s = *(const float4 *)(red + i);
#pragma unroll
            for (int w = 1; w < 4; w++) {
                const float4 t = *(const float4 *)(red + w * AQ * HD + i);
                s.x = s.x + t.x; s.y = s.y + t.y; s.z = s.z + t.z; s.w = s.w + t.w;
            }
            *(float4 *)(out + (int64_t)(t0 + qi) * nh * HD + h * HD + d) = s;
        }
    }
    VXM_ATTN_TS(4);
}

// Spans above AKV keys: the same tiles, lane layouts and score arithmetic in one
// pass over chunks of AKV keys with a running row max (every K and V row read
// once, every score formed once).  Per chunk: the chunk's row max m_c over all 8
// waves, m = max(m, m_c), the rescale a = exp(m_old - m) of the row's running
// P V sums and double exp sum, e = exp(s - m) into LDS and the P V products.  At
// the end the output is divided by the sum: o = (sum e v) * (float)(1 / sum e).
// Against the one-pass kernel only the rounding differs (each chunk's rescale,
// e instead of e / sum entering P V, and the summation orders).
template <int HD>
__global__ __launch_bounds__(ATH) void k_attention_mfma_long(const float *__restrict__ q,
                                                             const uint16_t *__restrict__ kc,
                                                             const uint16_t *__restrict__ vc, float *__restrict__ out,
                                                             int M, int nh, int nkv, int cap, int kv_base, int causal,
                                                             int8_t *__restrict__ xq, uint16_t *__restrict__ xd,
                                                             int variant) {
    constexpr int NW = ATH / 64;       // waves
    constexpr int SP = AKV + 4;        // fp32 P row pitch
    constexpr int KSTEPS = HD / 16;    // MFMA steps over the head dimension
    constexpr int HDH = HD / 2;        // dims of one output half
    constexpr int DT = HDH / 32;       // 32-dim output tiles per wave
    constexpr int VP = 32 + 8;         // f16 pitch of a wave's transposed V block
    constexpr int VITEMS = 16 * (HDH / 8) / 64;
    constexpr int CB = AKV / 32;       // key blocks per chunk
    constexpr int SB = CB / NW;        // most score blocks of one wave per chunk
    constexpr int VB = CB / 4;         // most P V blocks of one key quarter per chunk
    __shared__ __align__(16) float Sc[AQ * SP];
    __shared__ __align__(16) _Float16 Vt[NW][HDH * VP];
    __shared__ float smax[AQ][NW];
    __shared__ double ssum[AQ][NW];
    __shared__ float salpha[AQ], sinv[AQ];
    constexpr int QP = HD + 8;
    __shared__ __align__(16) _Float16 Qh[AQ * QP];
    static_assert(NW == 8 && VITEMS >= 1 && 4 * AQ * HD <= AQ * SP, "8 waves; the key-quarter sums reuse P's buffer");
    const int h = blockIdx.x, t0 = blockIdx.y * AQ, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kvh = h / (nh / nkv);
    const uint16_t *kb = kc + (int64_t)kvh * cap * HD;
    const uint16_t *vb = vc + (int64_t)kvh * cap * HD;
    const int nq = min(AQ, M - t0);
    const int kv_end = causal ? kv_base + t0 + nq : M;
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn((float)HD));
    const int lr = lane & 31, lh = lane >> 5;
    const int nblk = (kv_end + 31) / 32, nch = (nblk + CB - 1) / CB;
    const int kq = wave & 3, dh = wave >> 2;
    constexpr int QL = AQ * HD / 4 / ATH;
#pragma unroll
    for (int u = 0; u < QL; u++) {
        const int i = (u * ATH + tid) * 4, r = i / HD, d = i % HD;
        const float4 qf = *(const float4 *)(q + (int64_t)(t0 + min(r, nq - 1)) * nh * HD + h * HD + d);
        const bool qlive = r < nq;
        _Float16 *dst = Qh + r * QP + d;
        dst[0] = (_Float16)(qlive ? qf.x : 0.0f);
        dst[1] = (_Float16)(qlive ? qf.y : 0.0f);
        dst[2] = (_Float16)(qlive ? qf.z : 0.0f);
        dst[3] = (_Float16)(qlive ? qf.w : 0.0f);
    }
    __syncthreads();
    v8h qa[KSTEPS];
#pragma unroll
    for (int kk = 0; kk < KSTEPS; kk++) qa[kk] = *(const v8h *)(Qh + lr * QP + 16 * kk + 8 * lh);
    const int kvl = lr < nq ? (causal ? kv_base + t0 + lr + 1 : M) : 0;
    // the scores (S^T = K Q^T, scaled) of this wave's blocks of chunk c: block cb0 + i,
    // i < ncb; value v of lane (lr, lh) is query t0 + lr, key 32 b + 8 (v / 4) + 4 lh + v % 4
    auto scores = [&](int c, v16f (&sc)[SB], int &cb0, int &ncb) {
        const int nbc = min(CB, nblk - c * CB);
        cb0 = c * CB + nbc * wave / NW;
        ncb = c * CB + nbc * (wave + 1) / NW - cb0;
        uint4 kr[SB][KSTEPS];
#pragma unroll
        for (int i = 0; i < SB; i++) {
            const int key = min(32 * (cb0 + i) + lr, kv_end - 1);   // unconditional: clamped rows
#pragma unroll
            for (int kk = 0; kk < KSTEPS; kk++) kr[i][kk] = *(const uint4 *)(kb + (int64_t)key * HD + 16 * kk + 8 * lh);
        }
#pragma unroll
        for (int i = 0; i < SB; i++) {
            v16f acc = v16f{};
#pragma unroll
            for (int kk = 0; kk < KSTEPS; kk++) {
                v8h av;
                __builtin_memcpy(&av, &kr[i][kk], 16);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, qa[kk], acc, 0, 0, 0);
            }
#pragma unroll
            for (int v = 0; v < 16; v++) sc[i][v] = acc[v] * scale;
        }
    };
    auto live = [&](int i, int ncb, int b, int v) { return i < ncb && 32 * b + 8 * (v >> 2) + 4 * lh + (v & 3) < kvl; };
    v16f sc[SB];
    int cb0, ncb;
    float mrow = -INFINITY;   // running max of row lr (the same in every lane and wave)
    double lsum = 0.0;        // this lane's running double sum of e over its keys
    v16f o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) o[dt] = v16f{};
    _Float16 *vt = Vt[wave];
    const uint16_t *vbh = vb + HDH * dh;
    for (int c = 0; c < nch; c++) {
        const int nbc = min(CB, nblk - c * CB), cbase = c * CB;
        const int bq0 = cbase + nbc * kq / 4, nbq = cbase + nbc * (kq + 1) / 4 - bq0;
        // the V rows of the wave's P V blocks, in flight during the scores
        uint4 vr[VB][VITEMS][2];
#pragma unroll
        for (int i = 0; i < VB; i++)
#pragma unroll
            for (int u = 0; u < VITEMS; u++) {
                const int item = u * 64 + lane, r = 32 * (bq0 + i) + 2 * (item % 16), d = 8 * (item / 16);
#pragma unroll
                for (int e = 0; e < 2; e++)
                    vr[i][u][e] = *(const uint4 *)(vbh + (int64_t)min(r + e, kv_end - 1) * HD + d);
            }
        scores(c, sc, cb0, ncb);
        // the chunk's row max (the lane's, its partner's, the waves')
        float mc = -INFINITY;
#pragma unroll
        for (int i = 0; i < SB; i++)
#pragma unroll
            for (int v = 0; v < 16; v++)
                if (live(i, ncb, cb0 + i, v)) mc = fmaxf(mc, sc[i][v]);
        mc = fmaxf(mc, __shfl_xor(mc, 32));
        if (lh == 0) smax[lr][wave] = mc;
        __syncthreads();   // every wave's chunk max
        float mn = mrow;
#pragma unroll
        for (int w = 0; w < NW; w++) mn = fmaxf(mn, smax[lr][w]);
        // rescale of the row's sums so far (0 for the first live chunk, 1 while m holds;
        // a row with no live key yet keeps -inf and scale 1 over its zero sums)
        const float alpha = mn == -INFINITY ? 1.0f : expf(mrow - mn);
        mrow = mn;
        if (wave == 0 && lh == 0) salpha[lr] = alpha;
        lsum *= (double)alpha;
#pragma unroll
        for (int i = 0; i < SB; i++) {
            if (i >= ncb) break;
            float pv[16];
#pragma unroll
            for (int v = 0; v < 16; v++) {
                pv[v] = live(i, ncb, cb0 + i, v) ? expf(sc[i][v] - mn) : 0.0f;
                lsum += (double)pv[v];
            }
#pragma unroll
            for (int r4 = 0; r4 < 4; r4++)
                *(float4 *)(Sc + lr * SP + 32 * (cb0 + i - cbase) + 8 * r4 + 4 * lh) =
                    make_float4(pv[4 * r4], pv[4 * r4 + 1], pv[4 * r4 + 2], pv[4 * r4 + 3]);
        }
        __syncthreads();   // every wave's e rows of the chunk and the rows' rescales in LDS
        // the partial P V of earlier chunks, rescaled to the new max (row of value v of
        // the accumulators: 8 (v / 4) + 4 lh + v % 4)
        float al[16];
#pragma unroll
        for (int v = 0; v < 16; v++) al[v] = salpha[8 * (v >> 2) + 4 * lh + (v & 3)];
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int v = 0; v < 16; v++) o[dt][v] = o[dt][v] * al[v];
#pragma unroll
        for (int i = 0; i < VB; i++) {
            if (i >= nbq) break;
            const int b = bq0 + i;
#pragma unroll
            for (int u = 0; u < VITEMS; u++) {
                const int item = u * 64 + lane, r = 2 * (item % 16), d = 8 * (item / 16);
                const uint32_t a[4] = {vr[i][u][0].x, vr[i][u][0].y, vr[i][u][0].z, vr[i][u][0].w};
                const uint32_t bb[4] = {vr[i][u][1].x, vr[i][u][1].y, vr[i][u][1].z, vr[i][u][1].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    *(uint32_t *)(vt + (d + 2 * e) * VP + r) = (a[e] & 0xffffu) | (bb[e] << 16);
                    *(uint32_t *)(vt + (d + 2 * e + 1) * VP + r) = (a[e] >> 16) | (bb[e] & 0xffff0000u);
                }
            }
#pragma unroll
            for (int ks = 0; ks < 32; ks += 16) {
                const float *pr = Sc + lr * SP + 32 * (b - cbase) + ks + 8 * lh;
                const float4 p0 = *(const float4 *)pr, p1 = *(const float4 *)(pr + 4);
                const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
                v8h ahi, alo;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const _Float16 hi = (_Float16)pv[e];
                    ahi[e] = hi;
                    alo[e] = (_Float16)(pv[e] - (float)hi);
                }
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    const v8h bv = *(const v8h *)(vt + (32 * dt + lr) * VP + ks + 8 * lh);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi, bv, o[dt], 0, 0, 0);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo, bv, o[dt], 0, 0, 0);
                }
            }
        }
        __syncthreads();   // the chunk's e rows, maxima and rescales are read before the next chunk's
    }
    // the row's double sum (lanes, partner, waves) and its inverse for the output rows
    lsum += __shfl_xor(lsum, 32);
    if (lh == 0) ssum[lr][wave] = lsum;
    __syncthreads();
    if (wave == 0 && lh == 0) {
        double sum = ssum[lr][0];
#pragma unroll
        for (int w = 1; w < NW; w++) sum += ssum[lr][w];
        sinv[lr] = kvl > 0 ? (float)(1.0 / sum) : 0.0f;
    }
    // the key quarters in order through LDS (P's buffer is free)
    float *red = Sc;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int v = 0; v < 16; v++)
            red[(kq * AQ + 8 * (v >> 2) + 4 * lh + (v & 3)) * HD + HDH * dh + 32 * dt + lr] = o[dt][v];
    __syncthreads();
    if (xq) {
        for (int i = 8 * tid; i < AQ * HD; i += 8 * ATH) {
            const int qi = i / HD, d = i % HD;
            float v[8];
            const float inv = sinv[qi];
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                float4 s = *(const float4 *)(red + i + 4 * hf);
#pragma unroll
                for (int w = 1; w < 4; w++) {
                    const float4 t = *(const float4 *)(red + w * AQ * HD + i + 4 * hf);
                    s.x = s.x + t.x; s.y = s.y + t.y; s.z = s.z + t.z; s.w = s.w + t.w;
                }
                v[4 * hf] = s.x * inv; v[4 * hf + 1] = s.y * inv; v[4 * hf + 2] = s.z * inv; v[4 * hf + 3] = s.w * inv;
            }
            const int64_t o2 = (int64_t)(t0 + min(qi, nq - 1)) * nh * HD + h * HD + d;
            quant_block_4lanes(v, variant, xq + o2, xd + o2 / 32, (tid & 3) == 0, qi < nq);
        }
    } else {
        for (int i = 4 * tid; i < AQ * HD; i += 4 * ATH) {
            const int qi = i / HD, d = i % HD;
            if (qi >= nq) continue;
            float4 s = *(const float4 *)(red + i);
#pragma unroll
            for (int w = 1; w < 4; w++) {
                const float4 t = *(const float4 *)(red + w * AQ * HD + i);
                s.x = s.x + t.x; s.y = s.y + t.y; s.z = s.z + t.z; s.w = s.w + t.w;
            }
            const float inv = sinv[qi];
            s.x = s.x * inv; s.y = s.y * inv; s.z = s.z * inv; s.w = s.w * inv;
            *(float4 *)(out + (int64_t)(t0 + qi) * nh * HD + h * HD + d) = s;
        }
    }
}

int vxm_launch_attention(vxm_ctx *ctx, const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                         int64_t M, int nh, int nkv, int hd, int cap, int64_t seg_stride, int S, int kv_base,
                         int causal, int8_t *xq, uint16_t *xd, int variant) {
    if (M <= 0) return VXM_OK;
    if (hd > 256 || hd <= 0 || nkv <= 0 || nh % nkv)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "attention: head_dim %d / heads %d,%d unsupported", hd, nh, nkv);
    // many queries of a single segment whose key span fits the score buffer: the MFMA kernel
    const int64_t span = causal ? kv_base + M : M;
    if (S == M && M >= AQ && span <= cap && (hd == 128 || hd == 64)) {
        const dim3 grid(nh, (unsigned)((M + AQ - 1) / AQ));
        if (span <= AKV) {
            if (hd == 128)
                hipLaunchKernelGGL(k_attention_mfma<128>, grid, dim3(ATH), 0, ctx->stream, q, kc, vc, out, (int)M, nh,
                                   nkv, cap, kv_base, causal, xq, xd, variant);
            else
                hipLaunchKernelGGL(k_attention_mfma<64>, grid, dim3(ATH), 0, ctx->stream, q, kc, vc, out, (int)M, nh,
                                   nkv, cap, kv_base, causal, xq, xd, variant);
        } else if (hd == 128) {
            hipLaunchKernelGGL(k_attention_mfma_long<128>, grid, dim3(ATH), 0, ctx->stream, q, kc, vc, out, (int)M,
                               nh, nkv, cap, kv_base, causal, xq, xd, variant);
        } else {
            hipLaunchKernelGGL(k_attention_mfma_long<64>, grid, dim3(ATH), 0, ctx->stream, q, kc, vc, out, (int)M,
                               nh, nkv, cap, kv_base, causal, xq, xd, variant);
        }
        VXM_CHECK_LAUNCH(ctx);
        return VXM_OK;
    }
    const size_t lds = (size_t)(hd + cap + 256) * sizeof(float);
    if (lds > 160 * 1024)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "attention: capacity %d exceeds the LDS score buffer", cap);
    hipLaunchKernelGGL(k_attention, dim3(nh, (unsigned)M), dim3(256), lds, ctx->stream, q, kc, vc, out, nh, nkv,
                       hd, cap, seg_stride, S, kv_base, causal);
    VXM_CHECK_LAUNCH(ctx);
    return xq ? vxm_launch_quantize(ctx, out, M, (int64_t)nh * hd, variant, xq, xd) : VXM_OK;
}

// ---------------------------------------------------------------------------
// Non-causal attention within segments of S tokens at positions pos0 ..
// pos0+S-1 with fresh K/V (the LocDiT and LocEnc blocks): k_rope_kv, the
// f16 K/V rounding, k_attention and the Q8_0 quantization of the output in
// one launch, with the same rounding steps and summation orders as those
// kernels.  One workgroup (256 threads) per (query head, segment) keeps the
// segment's q of its head and k, v of its kv head in LDS; qkv may arrive as
// K-split slices.  Output: the Q8_0 rows of the attention output (xq, xd).
// ---------------------------------------------------------------------------
constexpr int kLocalMaxS = 64, kLocalMaxElems = 2048;   // S, and S * hd per operand
constexpr int kLocalRB = 4;                              // query rows per workgroup

bool vxm_attention_local_fits(int S, int hd) {
    return S >= 1 && S <= kLocalMaxS && (hd == 64 || hd == 128) && (int64_t)S * hd <= kLocalMaxElems;
}

template <int HD>
__global__ __launch_bounds__(256) void k_attention_local(const vxm_parts qkv, int nh, int nkv, int S, int pos0,
                                                         const float2 *__restrict__ cs, int no_rope,
                                                         int8_t *__restrict__ xq, uint16_t *__restrict__ xd,
                                                         int variant) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    constexpr int HALF = HD / 2, HP = HD + 4, RB = kLocalRB;
    const int h = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    const int q0 = blockIdx.z * RB, nq = min(RB, S - q0);   // this workgroup's query rows
    const int kvh = h / (nh / nkv);
    const int qd = nh * HD, kvd = nkv * HD, ld = qd + 2 * kvd;
    const int SP = S + 1;
    // raw k, v: [S][HD]; raw q (later the output): [RB][HD]; rotated k: [S][HD + 4],
    // rotated q: [RB][HD + 4] (the pad spreads the score loop's 16-byte row reads over
    // the banks); P: [RB][S + 1]; row max and 1/sum: [RB] each
    float *Kr = lds, *V = Kr + S * HD, *Qr = V + S * HD, *Kf = Qr + RB * HD, *Q = Kf + S * HP, *P = Q + RB * HP;
    float *mx = P + RB * SP, *inv = mx + RB;
    // 1. raw q (rows q0 .. q0+nq-1 of head h), k and v (all S rows of kv head kvh),
    //    K-split slices added in order; the loads of up to four slices are in flight together
    constexpr int kRopePer = ((kLocalMaxElems / HD + RB) * HALF + 255) / 256;
    float2 csr[kRopePer];
    {
        constexpr int kMaxPer = (3 * kLocalMaxElems / 4 + 255) / 256;   // float4s per thread
        constexpr int R4 = HD / 4;                                      // float4s per row
        const int nqf = nq * R4, total = nqf + 2 * S * R4;
        int64_t src[kMaxPer];
        float *dst[kMaxPer];
        float4 acc4[kMaxPer];
#pragma unroll
        for (int k = 0; k < kMaxPer; k++) {
            const int f = min(tid + 256 * k, total - 1);   // threads past the end reload the last element
            int row, col;
            if (f < nqf) {
                row = q0 + f / R4;
                col = h * HD;
                dst[k] = Qr + (f / R4) * HD;
            } else {
                const int e = f - nqf, part = e / (S * R4), rr = (e % (S * R4)) / R4;
                row = rr;
                col = part == 0 ? qd + kvh * HD : qd + kvd + kvh * HD;
                dst[k] = (part == 0 ? Kr : V) + rr * HD;
            }
            const int off = 4 * (f % R4);
            src[k] = (int64_t)(g * S + row) * ld + col + off;
            dst[k] += off;
            acc4[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        // the rope table entries of this thread's phase-2 items, fetched with the projections
        if (!no_rope) {
#pragma unroll
            for (int k = 0; k < kRopePer; k++) {
                const int idx = min(tid + 256 * k, (S + nq) * HALF - 1);
                const int rr = idx / HALF, i = idx % HALF;
                const int pos = pos0 + (rr < S ? rr : q0 + rr - S);
                csr[k] = cs[(int64_t)pos * HALF + i];
            }
        }
        for (int z0 = 0; z0 < qkv.n; z0 += 4) {
            float4 b[4][kMaxPer];
#pragma unroll
            for (int zz = 0; zz < 4; zz++)
#pragma unroll
                for (int k = 0; k < kMaxPer; k++)
                    if (z0 + zz < qkv.n) b[zz][k] = *(const float4 *)(qkv.p + (z0 + zz) * qkv.stride + src[k]);
#pragma unroll
            for (int zz = 0; zz < 4; zz++)
#pragma unroll
                for (int k = 0; k < kMaxPer; k++)
                    if (z0 + zz < qkv.n) {
                        if (z0 + zz == 0) {
                            acc4[k] = b[zz][k];
                        } else {
                            acc4[k].x = acc4[k].x + b[zz][k].x; acc4[k].y = acc4[k].y + b[zz][k].y;
                            acc4[k].z = acc4[k].z + b[zz][k].z; acc4[k].w = acc4[k].w + b[zz][k].w;
                        }
                    }
        }
#pragma unroll
        for (int k = 0; k < kMaxPer; k++)
            if (tid + 256 * k < total) *(float4 *)dst[k] = acc4[k];
    }
    __syncthreads();
    // 2. BF16 + RoPE of q and k (pair-interleaved rows: row 2i = dim i, 2i+1 = dim
    //    i + hd/2), the f16 cache rounding of k and v
#pragma unroll
    for (int k = 0; k < kRopePer; k++) {
        const int idx = tid + 256 * k;
        if (idx >= (S + nq) * HALF) break;
        const int rr = idx / HALF, i = idx % HALF;
        const bool isk = rr < S;
        const int lr = isk ? rr : rr - S;
        float c = 1.0f, sn = 0.0f;
        if (!no_rope) {
            c = csr[k].x;
            sn = csr[k].y;
        }
        const float *sp = (isk ? Kr : Qr) + lr * HD;
        const float x0 = vxm_bf16(sp[2 * i]), x1 = vxm_bf16(sp[2 * i + 1]);
        float y0 = x0, y1 = x1;
        if (!no_rope) {
            y0 = vxm_bf16(x0 * c - x1 * sn);
            y1 = vxm_bf16(x0 * sn + x1 * c);
        }
        if (isk) {
            y0 = vxm_h2f(vxm_f2h(y0));
            y1 = vxm_h2f(vxm_f2h(y1));
        }
        float *dp = (isk ? Kf : Q) + lr * HP;
        dp[i] = y0;
        dp[i + HALF] = y1;
    }
    for (int idx = tid; idx < S * HD; idx += 256) V[idx] = vxm_h2f(vxm_f2h(vxm_bf16(V[idx])));
    __syncthreads();
    // 3. scores s_ij = (k_j . q_i) * scale, d in order
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn((float)HD));
    for (int idx = tid; idx < nq * S; idx += 256) {
        const int i = idx / S, j = idx % S;
        const float4 *kr = (const float4 *)(Kf + j * HP), *qr = (const float4 *)(Q + i * HP);
        float sc = 0.0f;
#pragma unroll 8
        for (int d4 = 0; d4 < HD / 4; d4++) {
            const float4 a = kr[d4], b = qr[d4];
            sc += a.x * b.x;
            sc += a.y * b.y;
            sc += a.z * b.z;
            sc += a.w * b.w;
        }
        P[i * SP + j] = sc * scale;
    }
    __syncthreads();
    // 4. softmax: row max, exponentials, the row sum in double and (float)(1/sum); wave i
    //    takes query row i, lane j key j (S <= 64), so the max and the sum are wave
    //    reductions.  The double sum of at most 64 exponentials of one row is exact
    //    unless they span more than 2^29, so its order matches the serial sum's.
    static_assert(kLocalRB <= 4 && kLocalMaxS <= 64, "one wave per query row, one lane per key");
    {
        const int i = tid >> 6, j = tid & 63;
        if (i < nq) {
            // the wave reductions on DPP within rows of 16 lanes, the four rows read back
            // as scalars (no LDS round trip per step)
            const float sj = j < S ? P[i * SP + j] : -INFINITY;
            float m = sj;
            m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
            m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
            m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x141, 0xF, 0xF, false)));
            m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x140, 0xF, 0xF, false)));
            {
                float t = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0));
#pragma unroll
                for (int r = 1; r < 4; r++) t = fmaxf(t, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16 * r)));
                m = t;
            }
            const float e = j < S ? expf(sj - m) : 0.0f;
            if (j < S) P[i * SP + j] = e;
            double sum = (double)e;
            auto dpp_d = [](double x, auto ctrl) {
                const long long b = __double_as_longlong(x);
                const int lo = __builtin_amdgcn_update_dpp(0, (int)b, decltype(ctrl)::value, 0xF, 0xF, false);
                const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), decltype(ctrl)::value, 0xF, 0xF, false);
                return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
            };
            sum = sum + dpp_d(sum, std::integral_constant<int, 0xB1>{});
            sum = sum + dpp_d(sum, std::integral_constant<int, 0x4E>{});
            sum = sum + dpp_d(sum, std::integral_constant<int, 0x141>{});
            sum = sum + dpp_d(sum, std::integral_constant<int, 0x140>{});
            {
                const long long b = __double_as_longlong(sum);
                double t = 0.0;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)b, 16 * r);
                    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(b >> 32), 16 * r);
                    t += __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
                }
                sum = t;
            }
            if (j == 0) {
                mx[i] = m;
                inv[i] = (float)(1.0 / sum);
            }
        }
    }
    __syncthreads();
    // 5. out[i][d] = sum_j v[j][d] p_ij, p_ij = e_ij * inv_i, over the j-slices of
    //    k_attention (256 / hd of them, each summed in order, then added in order);
    //    thread (row group rg, dim d) owns rows rg, rg + R, ...; rows past nq read row
    //    nq - 1 with a zero weight, so the loop has no divergent reads
    {
        constexpr int R = 256 / HD, MAXR = (RB + R - 1) / R;
        const int d = tid % HD, rg = tid / HD;
        const int slices = 256 / HD, jper = (S + slices - 1) / slices;
        float tot[MAXR], acc[MAXR], iv[MAXR];
        int prow[MAXR];
#pragma unroll
        for (int k = 0; k < MAXR; k++) {
            tot[k] = 0.0f;
            iv[k] = rg + R * k < nq ? inv[rg + R * k] : 0.0f;
            prow[k] = min(rg + R * k, nq - 1) * SP;
        }
        for (int sl = 0; sl < slices; sl++) {
            const int j0 = sl * jper, j1 = min(S, j0 + jper);
#pragma unroll
            for (int k = 0; k < MAXR; k++) acc[k] = 0.0f;
#pragma unroll 4
            for (int j = j0; j < j1; j++) {
                const float v = V[j * HD + d];
#pragma unroll
                for (int k = 0; k < MAXR; k++) acc[k] += v * (P[prow[k] + j] * iv[k]);
            }
#pragma unroll
            for (int k = 0; k < MAXR; k++) tot[k] += acc[k];
        }
#pragma unroll
        for (int k = 0; k < MAXR; k++)
            if (rg + R * k < nq) Qr[(rg + R * k) * HD + d] = tot[k];
    }
    __syncthreads();
    // 6. Q8_0 of the output rows: thread (i, c) holds dims 8c .. 8c+7, four consecutive
    //    threads one 32-block (hd / 8 % 4 == 0: whole 4-lane groups stop together)
    constexpr int CPR = HD / 8;
    for (int idx = tid; idx < nq * CPR; idx += 256) {
        const int i = idx / CPR, c = idx % CPR;
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = Qr[i * HD + 8 * c + e];
        const int64_t el = (int64_t)(g * S + q0 + i) * qd + h * HD + 8 * c;
        quant_block_4lanes(o, variant, xq + el, xd + el / 32, (tid & 3) == 0);
    }
}

int vxm_launch_attention_local(vxm_ctx *ctx, vxm_parts qkv, int64_t M, int nh, int nkv, int hd, int S, int pos0,
                               const float2 *cs, int cs_rows, int no_rope, int8_t *xq, uint16_t *xd, int variant) {
    if (M <= 0) return VXM_OK;
    if (!vxm_attention_local_fits(S, hd) || M % S || nkv <= 0 || nh % nkv)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "local attention: S=%d hd=%d M=%lld unsupported", S, hd,
                        (long long)M);
    if (!no_rope && (!cs || pos0 + S > cs_rows))
        return vxm_fail(ctx, VXM_ERR_BACKEND, "rope: table holds %d positions, %d needed", cs_rows, pos0 + S);
    // query rows per workgroup: blocks of kLocalRB spread a segment's rows over several CUs
    // (each block re-derives the segment's k and v)
    const int RB = kLocalRB, QB = (S + RB - 1) / RB;
    const size_t lds = (size_t)(2 * S * hd + RB * hd + (S + RB) * (hd + 4) + RB * (S + 1) + 2 * RB) * sizeof(float);
    const dim3 grid(nh, (unsigned)(M / S), QB);
    if (hd == 64)
        hipLaunchKernelGGL(k_attention_local<64>, grid, dim3(256), lds, ctx->stream, qkv, nh, nkv, S, pos0, cs,
                           no_rope, xq, xd, variant);
    else
        hipLaunchKernelGGL(k_attention_local<128>, grid, dim3(256), lds, ctx->stream, qkv, nh, nkv, S, pos0, cs,
                           no_rope, xq, xd, variant);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

// ---------------------------------------------------------------------------
// vcpm_mlp activation (src/minicpm4.c:441-456): p = bf16(bf16(silu(bf16(g))) *
// bf16(u)), silu(x) = x / (1 + expf(-x)), then Q8_0 quantization of p.
// Row m of the fused gate/up projection holds 2F values interleaved: gate n at
// gu[m*ld + 2n], up n at gu[m*ld + 2n + 1].  8 outputs per thread.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_swiglu_quant(const vxm_parts gu, int64_t F, int64_t ld,
                                                      int64_t total, int8_t *__restrict__ xq,
                                                      uint16_t *__restrict__ xd, float *__restrict__ p_out,
                                                      int variant) {
    const int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (e >= total) return;   // total, F % 32 == 0: 4-lane groups are all live or all dead
    const int64_t m = e / F, j = e % F;
    const float *s = gu.p + m * ld + 2 * j;
    float gv[8], uv[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        // K-split slices: up to four loads in flight, added in order
        float4 a = *(const float4 *)(s + 4 * k);
        for (int z0 = 1; z0 < gu.n; z0 += 4) {
            float4 b[4];
#pragma unroll
            for (int zz = 0; zz < 4; zz++)
                if (z0 + zz < gu.n) b[zz] = *(const float4 *)(s + (z0 + zz) * gu.stride + 4 * k);
#pragma unroll
            for (int zz = 0; zz < 4; zz++)
                if (z0 + zz < gu.n) {
                    a.x = a.x + b[zz].x; a.y = a.y + b[zz].y; a.z = a.z + b[zz].z; a.w = a.w + b[zz].w;
                }
        }
        gv[2 * k] = a.x; uv[2 * k] = a.y; gv[2 * k + 1] = a.z; uv[2 * k + 1] = a.w;
    }
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float gb = vxm_bf16(gv[i]);
        const float s = vxm_bf16(__fdiv_rn(gb, 1.0f + expf(-gb)));
        p[i] = vxm_bf16(s * vxm_bf16(uv[i]));
    }
    if (p_out) {
        *(float4 *)(p_out + e) = make_float4(p[0], p[1], p[2], p[3]);
        *(float4 *)(p_out + e + 4) = make_float4(p[4], p[5], p[6], p[7]);
    }
    quant_block_4lanes(p, variant, xq + e, xd + e / 32, (threadIdx.x & 3) == 0);
}

int vxm_launch_swiglu_quant(vxm_ctx *ctx, vxm_parts gu, int64_t M, int64_t F, int64_t ld, int8_t *xq,
                            uint16_t *xd, float *p_out, int variant) {
    const int64_t total = M * F;
    if (total <= 0) return VXM_OK;
    if (F % 32) return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "swiglu: width %lld not a multiple of 32", (long long)F);
    const int64_t threads = total / 8;
    hipLaunchKernelGGL(k_swiglu_quant, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, ctx->stream, gu, F,
                       ld, total, xq, xd, p_out, variant);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

// ---------------------------------------------------------------------------
// h = bf16(h + scale * bf16(delta)) (the residual adds of
// vcpm_minicpm4_block, src/minicpm4.c:496-528), elementwise.
// ---------------------------------------------------------------------------
__global__ void k_residual(float *__restrict__ h, const vxm_parts delta, float scale, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float d = delta.p[i];
    for (int z = 1; z < delta.n; z++) d = d + delta.p[z * delta.stride + i];
    float o = vxm_bf16(d);
    if (scale != 1.0f) o = o * scale;
    h[i] = vxm_bf16(h[i] + o);
}

int vxm_launch_residual(vxm_ctx *ctx, float *h, vxm_parts delta, float scale, int64_t n) {
    if (n <= 0) return VXM_OK;
    hipLaunchKernelGGL(k_residual, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, h, delta, scale, n);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

// y = bf16(x + bias) per row (ggml_add of a repeated bias then BF16,
// src/locdit.c:190-210 and :118-121); bias may be null (BF16 only).
__global__ void k_bias_bf16(const float *__restrict__ x, const float *__restrict__ bias, float *__restrict__ y,
                            int64_t rows, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * n) return;
    float v = x[i];
    if (bias) v = v + bias[i % n];
    y[i] = vxm_bf16(v);
}

int vxm_launch_bias_bf16(vxm_ctx *ctx, const float *x, const float *bias, float *y, int64_t rows, int64_t n) {
    if (rows * n <= 0) return VXM_OK;
    hipLaunchKernelGGL(k_bias_bf16, dim3((unsigned)((rows * n + 255) / 256)), dim3(256), 0, ctx->stream, x, bias,
                       y, rows, n);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}
