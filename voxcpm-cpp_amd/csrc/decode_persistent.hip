// decode_persistent.hip -- one decode token through the whole MiniCPM4 stack
// (vcpm_minicpm4_forward with n_tokens = 1, src/minicpm4.c:536-572) in ONE
// cooperative launch of one workgroup per CU.
//
// Why: on MI355X a kernel boundary costs ~1.3-2.4 us and a cross-XCD signal
// ~1.5 us, against ~6.3 us of HBM streaming per layer; one launch per op
// (10 per layer) spends more time in boundaries than in streaming.
//
// Dataflow: each layer is five phases
//   A  rms_norm(x) -> Q8_0 -> QKV rows -> BF16 -> NEOX rope -> q, k, v
//   B  attention (+ f16 KV append), one workgroup per query head
//   C  O rows -> h1 = BF16(x + BF16(o))
//   D  rms_norm(h1) -> Q8_0 -> gate/up rows -> p = SwiGLU
//   E  Q8_0(p) -> down rows -> x' = BF16(h1 + BF16(d))
// and every phase publishes its outputs as 64-bit tagged words: a 32-bit tag
// (launch epoch, layer, phase) over 32 bits of payload -- two BF16 values
// (q/k/v, h1, p and x are all BF16-rounded by the reference graph) or one
// fp32 (the attention output).  Each word is one relaxed agent-scope atomic
// store.  A consumer polls the words it needs until every tag is the expected
// one, so data and synchronisation arrive together: one cross-XCD latency per
// phase and no grid barrier.  Every workgroup needs every element of its
// inputs, so the all-to-all dependency also protects the single-buffered
// channels against write-after-read.
//
// Waves: wave 0 of each workgroup only polls inputs (and stages the RMSNorm
// gains) into LDS; waves 1..3 own fixed weight rows of every matrix and keep
// them in registers.  The loads of the next phase's rows are issued right
// after the current phase's inputs arrive.  Vector-memory counters retire in
// order, so keeping polls and prefetches in different waves is what lets a
// poll complete while megabytes of weights are still in flight.
// The arithmetic per row is exactly that of the GEMV kernel (q8_matmul.hip):
// per-block int32 sums, then (float)sumi * (d_w * d_x).
#include "vxm_model.h"

typedef int v4i __attribute__((ext_vector_type(4)));

namespace {

constexpr int kWaves = 4;              // waves per workgroup: 1 poller + 3 compute
constexpr int kCW = kWaves - 1;
constexpr int kThreads = kWaves * 64;
constexpr int kSpin = 1 << 17;         // poll retries before giving up
// Every channel is written as kRep replicas; workgroup b polls replica
// b % kRep.  256 workgroups reading one copy concentrate the coherent loads
// on the few memory channels behind those lines; replicas spread them out.
constexpr int kRep = 16;
constexpr int kPad = 64;               // words between replicas

__host__ __device__ constexpr int rep_stride(int words) { return words + kPad; }

enum Phase { PH_X = 0, PH_QKV = 1, PH_ATT = 2, PH_H1 = 3, PH_P = 4 };

__device__ __forceinline__ uint32_t make_tag(uint32_t epoch, int layer, int phase) {
    return (epoch << 12) | ((uint32_t)layer << 3) | (uint32_t)phase;
}

// two BF16-valued floats (low 16 bits zero) in one 32-bit payload
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xffff0000u);
}

__device__ __forceinline__ void put_word(uint64_t *dst, uint32_t payload, uint32_t tag) {
    __hip_atomic_store(dst, ((uint64_t)tag << 32) | (uint64_t)payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t get_word(const uint64_t *src) {
    return __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int dot16(const v4i a, const v4i b) {
    int acc = __builtin_amdgcn_sdot4(a.x, b.x, 0, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

__device__ __forceinline__ float pair_sum(float v) {
#pragma unroll
    for (int m = 2; m <= 32; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

}  // namespace

struct vxm_player {
    const int8_t *qkv_qs, *o_qs, *gu_qs, *d_qs;
    const uint16_t *qkv_dg, *o_dg, *gu_dg, *d_dg;
    const float *g_in, *g_post;
    uint16_t *kc, *vc;
};

struct vxm_pparams {
    const vxm_player *layers;
    int n_layers;
    const float *final_norm;
    float *x;          // [H] input of layer 0 and output (after the final norm)
    // tagged channels, each kRep replicas of rep_stride(words) words
    uint64_t *xb;      // 2 x [H/2] layer inputs (BF16 pairs), by layer parity
    uint64_t *qkvb;    // [(QD + 2 KVD)/2] q, k (rope'd, pair-interleaved per head) and v (BF16 pairs)
    uint64_t *attb;    // [QD] attention output (fp32)
    uint64_t *h1b;     // [H/2] BF16 pairs
    uint64_t *pb;      // [F/2] BF16 pairs
    int *err;
    const float *ff;
    float theta_scale, eps, res_scale;
    int pos, cap, no_rope;
    uint32_t epoch;
};

namespace {

// LDS layout (dynamic): floats, then int8 quants (16-byte aligned).
template <int H, int QD, int F, int HD>
struct Lds {
    static constexpr int KMAX = (H > QD ? (H > F ? H : F) : (QD > F ? QD : F));
    static constexpr int XS = 0;                  // x of the layer            [H]
    static constexpr int H1 = XS + H;             // h1 / normed-x scratch     [H]
    static constexpr int GN = H1 + H;             // RMSNorm gain of the phase [H]
    static constexpr int XD = GN + H;             // activation block scales   [KMAX/32]
    static constexpr int CS = XD + KMAX / 32;     // rope cos/sin              [HD]
    static constexpr int AQ = CS + HD;            // attention q, k, v         [3 HD]
    static constexpr int RED = AQ + 3 * HD;       // reductions / partials     [2 kThreads]
    static constexpr int SC = RED + 2 * kThreads; // scores / staged vectors   [max(cap + 1, KMAX)]
    __host__ __device__ static int sc_len(int cap) { return cap + 1 > KMAX ? cap + 1 : KMAX; }
    __host__ __device__ static int xq_off(int cap) { return ((SC + sc_len(cap)) * 4 + 15) & ~15; }
    __host__ __device__ static int bytes(int cap) { return xq_off(cap) + KMAX; }
};

// Wave 0 polls n tagged words; word i at src(i); put(i, payload) stores the
// payload into LDS.  All loads of a round are issued before any is checked.
// Sets *bail on timeout or when another workgroup aborted.
template <int PER, typename Src, typename Put>
__device__ void poll_words(Src src, int n, uint32_t tag, Put put, int *err, int *bail) {
    const int lane = threadIdx.x & 63;
    uint64_t w[PER];
    bool done[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) done[k] = lane + k * 64 >= n;
    int it = 0;
    while (true) {
#pragma unroll
        for (int k = 0; k < PER; k++)
            if (!done[k]) w[k] = get_word(src(lane + k * 64));
        bool all = true;
#pragma unroll
        for (int k = 0; k < PER; k++) {
            if (!done[k]) {
                if ((uint32_t)(w[k] >> 32) == tag) {
                    put(lane + k * 64, (uint32_t)w[k]);
                    done[k] = true;
                } else {
                    all = false;
                }
            }
        }
        if (all) break;
        if (++it > kSpin || __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *bail = 1;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Wave 0: BF16-pair words -> dst floats (2 per word)
template <int PER>
__device__ void poll_pairs(const uint64_t *src, int nwords, uint32_t tag, float *dst, int *err, int *bail) {
    poll_words<PER>([src](int i) { return src + i; }, nwords, tag,
                    [dst](int i, uint32_t v) {
                        dst[2 * i] = __uint_as_float(v << 16);
                        dst[2 * i + 1] = __uint_as_float(v & 0xffff0000u);
                    },
                    err, bail);
}

// Wave 0: plain copy of n floats (gains) into LDS
__device__ void stage_f32(const float *src, int n, float *dst) {
    const int lane = threadIdx.x & 63;
    for (int i = lane * 4; i < n; i += 256) *(float4 *)(dst + i) = *(const float4 *)(src + i);
}

__device__ __forceinline__ double wg_sum_d(double v, float *red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    double *r = (double *)red;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) r[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < kWaves; i++) t += r[i];
    return t;
}

__device__ __forceinline__ float wg_max_f(float v, float *red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int i = 1; i < kWaves; i++) t = fmaxf(t, red[i]);
    return t;
}

// Q8_0 (x86 rule) of n values in LDS (n % 32 == 0): 8 values per thread, 4 threads per block.
__device__ void quantize_lds(const float *src, int n, int8_t *xq, float *xd) {
    for (int base = threadIdx.x * 8; base < n; base += kThreads * 8) {
        float v[8];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[i] = src[base + i];
            amax = fmaxf(amax, fabsf(v[i]));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        const float d = __fdiv_rn(amax, 127.0f);
        const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float q = fminf(fmaxf(rintf(v[i] * id), -128.0f), 127.0f);
            const uint32_t b = (uint32_t)(uint8_t)(int8_t)(int)q;
            if (i < 4) lo |= b << (8 * i);
            else hi |= b << (8 * (i - 4));
        }
        *(uint2 *)(xq + base) = make_uint2(lo, hi);
        if ((threadIdx.x & 3) == 0) xd[base / 32] = vxm_h2f(vxm_f2h(d));   // the fp16-rounded scale
    }
}

// vcpm_rms_norm of src (LDS) with gain (LDS): BF16(BF16(x*scale)*g) into dst (LDS).
__device__ void rmsnorm_lds(const float *src, const float *gain, int n, float eps, float *dst, float *red) {
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += kThreads) ss += (double)(src[i] * src[i]);
    const double tot = wg_sum_d(ss, red);
    const float mean = (float)(tot / (double)n);
    const float sc = __fdiv_rn(1.0f, __fsqrt_rn(mean + eps));
    for (int i = threadIdx.x; i < n; i += kThreads) dst[i] = vxm_bf16(vxm_bf16(src[i] * sc) * gain[i]);
    __syncthreads();
}

template <int NR, int C>
__device__ __forceinline__ void load_rows(const int8_t *qs, const uint16_t *dg, const int (&rows)[NR],
                                          v4i (&w)[NR][C], uint32_t (&d)[NR][C]) {
    const int lane = threadIdx.x & 63;
    const int pair = lane >> 1;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int8_t *p = qs + (int64_t)rows[r] * (C * 1024) + lane * 16;
#pragma unroll
        for (int c = 0; c < C; c++) w[r][c] = __builtin_nontemporal_load((const v4i *)(p + c * 1024));
        const uint16_t *q = dg + (int64_t)rows[r] * (C * 32) + pair * C;
#pragma unroll
        for (int c = 0; c < C; c++) d[r][c] = __builtin_nontemporal_load(q + c);
    }
}

template <int NR, int C>
__device__ __forceinline__ void dot_rows(const v4i (&w)[NR][C], const uint32_t (&d)[NR][C], const int8_t *xq,
                                         const float *xd, float (&out)[NR]) {
    const int lane = threadIdx.x & 63;
    const int pair = lane >> 1;
    v4i xv[C];
    float xs[C];
#pragma unroll
    for (int c = 0; c < C; c++) {
        xv[c] = *(const v4i *)(xq + c * 1024 + lane * 16);
        xs[c] = xd[c * 32 + pair];
    }
#pragma unroll
    for (int r = 0; r < NR; r++) {
        float a = 0.0f;
#pragma unroll
        for (int c = 0; c < C; c++) {
            int s = dot16(w[r][c], xv[c]);
            s += __shfl_xor(s, 1, 64);
            a += (float)s * (vxm_h2f((uint16_t)d[r][c]) * xs[c]);
        }
        out[r] = pair_sum(a);
    }
}

// Unit u of a phase owns rows [R*u, R*u + R); rows of invalid units are
// clamped to the last unit (loaded, never stored).
template <int U, int R>
__device__ __forceinline__ void unit_rows(int cw, int W, int n_units, int (&rows)[U * R], bool (&valid)[U],
                                          int (&unit)[U]) {
#pragma unroll
    for (int k = 0; k < U; k++) {
        const int u = cw + k * W;
        valid[k] = u < n_units;
        unit[k] = valid[k] ? u : n_units - 1;
#pragma unroll
        for (int r = 0; r < R; r++) rows[k * R + r] = unit[k] * R + r;
    }
}

__device__ __forceinline__ float swiglu(float g, float u) {
    const float gb = vxm_bf16(g);
    const float s = vxm_bf16(__fdiv_rn(gb, 1.0f + expf(-gb)));
    return vxm_bf16(s * vxm_bf16(u));
}


// The whole decode for one wave type.  POLLER = wave 0 of the workgroup
// (polls inputs, stages gains); otherwise a compute wave (owns weight rows).
// Both instantiations walk the same phase schedule and execute the same
// __syncthreads() sequence; keeping them separate functions keeps the polling
// registers and the weight registers out of each other's live ranges.
template <bool POLLER, int H, int NH, int NKV, int HD, int F, int G>
__device__ __forceinline__ void decode_run(const vxm_pparams &p, float *lds, int *bail) {
    constexpr int QD = NH * HD, KVD = NKV * HD, NQKV = QD + 2 * KVD;
    constexpr int W = G * kCW;                                   // compute waves in the grid
    constexpr int CH = H / 1024, CQ = QD / 1024, CF = F / 1024;
    constexpr int NA = NQKV / 2, NC = H / 2, ND = F / 2, NE = H / 2;   // output words per phase
    constexpr int UA = (NA + W - 1) / W, UC = (NC + W - 1) / W, UD = (ND + W - 1) / W, UE = (NE + W - 1) / W;
    constexpr int LPK = HD / 8, KPW = 64 / LPK;                  // attention: lanes per key, keys per wave
    constexpr int KB = 8;                                        // attention: key loads in flight per lane
    constexpr int SX = rep_stride(H / 2), SQ = rep_stride(NA), SAT = rep_stride(QD), SP = rep_stride(ND);
    const int rp = blockIdx.x % kRep;                            // replica this workgroup polls
    using L = Lds<H, QD, F, HD>;
    static_assert(H % 1024 == 0 && QD % 1024 == 0 && F % 1024 == 0, "K must be a multiple of 1024");
    static_assert(HD % 8 == 0 && HD <= 256 && 64 % LPK == 0, "head_dim");

    float *xs = lds + L::XS, *h1s = lds + L::H1, *gn = lds + L::GN, *xd = lds + L::XD, *cs = lds + L::CS;
    float *aq = lds + L::AQ, *red = lds + L::RED, *sc = lds + L::SC;
    int8_t *xq = (int8_t *)lds + L::xq_off(p.cap);

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int cw = blockIdx.x * kCW + (POLLER ? 0 : wave - 1);
    const int pos = p.pos;
    const uint32_t ep = p.epoch;

    // rope cos/sin of this token's position (ggml_rope_ext NEOX, iterative theta)
    for (int i = threadIdx.x; i < HD / 2; i += kThreads) {
        float theta = (float)pos;
        for (int k = 0; k < i; k++) theta = theta * p.theta_scale;
        const float th = p.ff ? __fdiv_rn(theta, p.ff[i]) : theta;
        cs[2 * i] = cosf(th);
        cs[2 * i + 1] = sinf(th);
    }

    // compute waves: fixed unit ownership and the weight registers
    int rA[2 * UA], rC[2 * UC], rD[4 * UD], rE[2 * UE];
    bool vA[UA], vC[UC], vD[UD], vE[UE];
    int uA[UA], uC[UC], uD[UD], uE[UE];
    v4i wA[POLLER ? 1 : 2 * UA][CH], wC[POLLER ? 1 : 2 * UC][CQ], wD[POLLER ? 1 : 4 * UD][CH],
        wE[POLLER ? 1 : 2 * UE][CF];
    uint32_t dA[POLLER ? 1 : 2 * UA][CH], dC[POLLER ? 1 : 2 * UC][CQ], dD[POLLER ? 1 : 4 * UD][CH],
        dE[POLLER ? 1 : 2 * UE][CF];
    if constexpr (!POLLER) {
        unit_rows<UA, 2>(cw, W, NA, rA, vA, uA);
        unit_rows<UC, 2>(cw, W, NC, rC, vC, uC);
        unit_rows<UD, 4>(cw, W, ND, rD, vD, uD);
        unit_rows<UE, 2>(cw, W, NE, rE, vE, uE);
        load_rows<2 * UA, CH>(p.layers[0].qkv_qs, p.layers[0].qkv_dg, rA, wA, dA);
    }

    for (int l = 0; l < p.n_layers; l++) {
        const vxm_player &Ly = p.layers[l];
        // ---------------- A: norm + QKV + rope ----------------
        if constexpr (POLLER) {
            stage_f32(Ly.g_in, H, gn);
            if (l == 0) {
                for (int i = lane * 4; i < H; i += 256) *(float4 *)(xs + i) = *(const float4 *)(p.x + i);
            } else {
                poll_pairs<(H / 2 + 63) / 64>(p.xb + ((l & 1) * kRep + rp) * SX, H / 2, make_tag(ep, l, PH_X), xs,
                                              p.err, bail);
            }
        }
        __syncthreads();
        if (*bail) return;
        if constexpr (!POLLER) load_rows<2 * UC, CQ>(Ly.o_qs, Ly.o_dg, rC, wC, dC);
        rmsnorm_lds(xs, gn, H, p.eps, h1s, red);
        quantize_lds(h1s, H, xq, xd);
        __syncthreads();
        if constexpr (!POLLER) {
            float out[2 * UA];
            dot_rows<2 * UA, CH>(wA, dA, xq, xd, out);
            if (lane < kRep) {
                const uint32_t tg = make_tag(ep, l, PH_QKV);
#pragma unroll
                for (int k = 0; k < UA; k++) {
                    if (!vA[k]) continue;
                    const int row = 2 * uA[k];
                    const float x0 = vxm_bf16(out[2 * k]), x1 = vxm_bf16(out[2 * k + 1]);
                    float y0 = x0, y1 = x1;
                    if (row < QD + KVD && !p.no_rope) {
                        const int i = (row % HD) / 2;
                        const float c = cs[2 * i], s = cs[2 * i + 1];
                        y0 = vxm_bf16(x0 * c - x1 * s);
                        y1 = vxm_bf16(x0 * s + x1 * c);
                    }
                    put_word(p.qkvb + lane * SQ + uA[k], pack_bf16x2(y0, y1), tg);
                }
            }
        }
        // ---------------- B: attention, workgroup h = query head h ----------------
        if (blockIdx.x < NH) {
            const int h = blockIdx.x, g = h / (NH / NKV);
            if constexpr (POLLER) {
                // q_h and k_g (pair-interleaved: word w = dims w, w + HD/2) and
                // v_g (natural pairs) -> aq[0..3HD) in natural order
                const uint64_t *qkvb = p.qkvb + rp * SQ;
                poll_words<(3 * HD / 2 + 63) / 64>(
                    [qkvb, h, g](int i) {
                        const int part = i / (HD / 2), w = i % (HD / 2);
                        return part == 0 ? qkvb + h * (HD / 2) + w
                                         : part == 1 ? qkvb + (QD + g * HD) / 2 + w : qkvb + (QD + KVD + g * HD) / 2 + w;
                    },
                    3 * HD / 2, make_tag(ep, l, PH_QKV),
                    [aq](int i, uint32_t v) {
                        const int part = i / (HD / 2), w = i % (HD / 2);
                        const float a = __uint_as_float(v << 16), b = __uint_as_float(v & 0xffff0000u);
                        float *dst = aq + part * HD;
                        if (part < 2) {
                            dst[w] = a;
                            dst[w + HD / 2] = b;
                        } else {
                            dst[2 * w] = a;
                            dst[2 * w + 1] = b;
                        }
                    },
                    p.err, bail);
            }
            __syncthreads();
            if (*bail) return;
            const float *qh = aq, *kcur = aq + HD, *vcur = aq + 2 * HD;
            const uint16_t *kb = Ly.kc + (int64_t)g * p.cap * HD;
            const uint16_t *vb = Ly.vc + (int64_t)g * p.cap * HD;
            // KV append: the first query head of each group writes the whole f16
            // rows of K and V at pos (one workgroup per row).
            if (h % (NH / NKV) == 0) {
                uint16_t *kw = Ly.kc + ((int64_t)g * p.cap + pos) * HD;
                uint16_t *vw = Ly.vc + ((int64_t)g * p.cap + pos) * HD;
                for (int d = threadIdx.x; d < HD; d += kThreads) {
                    kw[d] = vxm_f2h(kcur[d]);
                    vw[d] = vxm_f2h(vcur[d]);
                }
            }
            const int kv_len = pos + 1;
            const float scale = __fdiv_rn(1.0f, __fsqrt_rn((float)HD));
            const int sub = lane % LPK, kin = lane / LPK;
            float qv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) qv[i] = qh[sub * 8 + i];
            // batch jb covers keys jb + (k * kWaves + wave) * KPW + kin, k < KB
            constexpr int PERB = kWaves * KPW * KB;
            float mx = -INFINITY;
            for (int jb = 0; jb < kv_len; jb += PERB) {
                uint4 raw[KB];
#pragma unroll
                for (int k = 0; k < KB; k++) {
                    const int j = jb + (k * kWaves + wave) * KPW + kin;
                    raw[k] = j < pos ? *(const uint4 *)(kb + (int64_t)j * HD + sub * 8) : make_uint4(0, 0, 0, 0);
                }
#pragma unroll
                for (int k = 0; k < KB; k++) {
                    const int j = jb + (k * kWaves + wave) * KPW + kin;
                    float kv8[8];
                    if (j == pos) {
#pragma unroll
                        for (int i = 0; i < 8; i++) kv8[i] = vxm_h2f(vxm_f2h(kcur[sub * 8 + i]));
                    } else {
                        const uint32_t wv[4] = {raw[k].x, raw[k].y, raw[k].z, raw[k].w};
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            kv8[2 * i] = vxm_h2f((uint16_t)(wv[i] & 0xffffu));
                            kv8[2 * i + 1] = vxm_h2f((uint16_t)(wv[i] >> 16));
                        }
                    }
                    float part = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; i++) part += kv8[i] * qv[i];
#pragma unroll
                    for (int m = 1; m < LPK; m <<= 1) part += __shfl_xor(part, m, 64);
                    if (j < kv_len && sub == 0) {
                        const float s = part * scale;
                        sc[j] = s;
                        mx = fmaxf(mx, s);
                    }
                }
            }
            mx = wg_max_f(mx, red);
            double sum = 0.0;
            for (int j = threadIdx.x; j < kv_len; j += kThreads) {
                const float e = expf(sc[j] - mx);
                sc[j] = e;
                sum += (double)e;
            }
            sum = wg_sum_d(sum, red);
            const float inv = (float)(1.0 / sum);
            for (int j = threadIdx.x; j < kv_len; j += kThreads) sc[j] = sc[j] * inv;
            __syncthreads();
            // out[d] = sum_j p_j v_j[d]: lane (kin, sub) accumulates dims sub*8..+8 over its keys
            float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int jb = 0; jb < kv_len; jb += PERB) {
                uint4 raw[KB];
#pragma unroll
                for (int k = 0; k < KB; k++) {
                    const int j = jb + (k * kWaves + wave) * KPW + kin;
                    raw[k] = j < pos ? *(const uint4 *)(vb + (int64_t)j * HD + sub * 8) : make_uint4(0, 0, 0, 0);
                }
#pragma unroll
                for (int k = 0; k < KB; k++) {
                    const int j = jb + (k * kWaves + wave) * KPW + kin;
                    if (j >= kv_len) continue;
                    const float pj = sc[j];
                    if (j == pos) {
#pragma unroll
                        for (int i = 0; i < 8; i++) o[i] += vxm_h2f(vxm_f2h(vcur[sub * 8 + i])) * pj;
                    } else {
                        const uint32_t wv[4] = {raw[k].x, raw[k].y, raw[k].z, raw[k].w};
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            o[2 * i] += vxm_h2f((uint16_t)(wv[i] & 0xffffu)) * pj;
                            o[2 * i + 1] += vxm_h2f((uint16_t)(wv[i] >> 16)) * pj;
                        }
                    }
                }
            }
            // reduce over the KPW key lanes of the wave, then over waves (fixed order)
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int m = LPK; m < 64; m <<= 1) o[i] += __shfl_xor(o[i], m, 64);
            if (kin == 0) {
#pragma unroll
                for (int i = 0; i < 8; i++) red[wave * HD + sub * 8 + i] = o[i];
            }
            __syncthreads();
            const uint32_t tg = make_tag(ep, l, PH_ATT);
            for (int d = threadIdx.x; d < HD; d += kThreads) {
                float t = 0.0f;
#pragma unroll
                for (int w = 0; w < kWaves; w++) t += red[w * HD + d];
#pragma unroll
                for (int r = 0; r < kRep; r++) put_word(p.attb + r * SAT + h * HD + d, __float_as_uint(t), tg);
            }
            __syncthreads();
        }
        // ---------------- C: O rows + residual ----------------
        if constexpr (POLLER) {
            const uint64_t *attb = p.attb + rp * SAT;
            poll_words<(QD + 63) / 64>([attb](int i) { return attb + i; }, QD, make_tag(ep, l, PH_ATT),
                                       [sc](int i, uint32_t v) { sc[i] = __uint_as_float(v); }, p.err, bail);
        }
        __syncthreads();
        if (*bail) return;
        if constexpr (!POLLER) load_rows<4 * UD, CH>(Ly.gu_qs, Ly.gu_dg, rD, wD, dD);
        quantize_lds(sc, QD, xq, xd);
        __syncthreads();
        if constexpr (!POLLER) {
            float out[2 * UC];
            dot_rows<2 * UC, CQ>(wC, dC, xq, xd, out);
            if (lane < kRep) {
                const uint32_t tg = make_tag(ep, l, PH_H1);
#pragma unroll
                for (int k = 0; k < UC; k++) {
                    if (!vC[k]) continue;
                    const int r = 2 * uC[k];
                    float o0 = vxm_bf16(out[2 * k]), o1 = vxm_bf16(out[2 * k + 1]);
                    if (p.res_scale != 1.0f) { o0 = o0 * p.res_scale; o1 = o1 * p.res_scale; }
                    put_word(p.h1b + lane * SX + uC[k], pack_bf16x2(vxm_bf16(xs[r] + o0), vxm_bf16(xs[r + 1] + o1)),
                             tg);
                }
            }
        }
        // ---------------- D: post norm + gate/up + SwiGLU ----------------
        if constexpr (POLLER) {
            stage_f32(Ly.g_post, H, gn);
            poll_pairs<(H / 2 + 63) / 64>(p.h1b + rp * SX, H / 2, make_tag(ep, l, PH_H1), h1s, p.err, bail);
        }
        __syncthreads();
        if (*bail) return;
        if constexpr (!POLLER) load_rows<2 * UE, CF>(Ly.d_qs, Ly.d_dg, rE, wE, dE);
        rmsnorm_lds(h1s, gn, H, p.eps, sc, red);
        quantize_lds(sc, H, xq, xd);
        __syncthreads();
        if constexpr (!POLLER) {
            float out[4 * UD];
            dot_rows<4 * UD, CH>(wD, dD, xq, xd, out);
            if (lane < kRep) {
                const uint32_t tg = make_tag(ep, l, PH_P);
#pragma unroll
                for (int k = 0; k < UD; k++) {
                    if (!vD[k]) continue;
                    const float p0 = swiglu(out[4 * k], out[4 * k + 1]);
                    const float p1 = swiglu(out[4 * k + 2], out[4 * k + 3]);
                    put_word(p.pb + lane * SP + uD[k], pack_bf16x2(p0, p1), tg);
                }
            }
        }
        // ---------------- E: down rows + residual ----------------
        if constexpr (POLLER)
            poll_pairs<(F / 2 + 63) / 64>(p.pb + rp * SP, F / 2, make_tag(ep, l, PH_P), sc, p.err, bail);
        __syncthreads();
        if (*bail) return;
        if constexpr (!POLLER) {
            if (l + 1 < p.n_layers) load_rows<2 * UA, CH>(p.layers[l + 1].qkv_qs, p.layers[l + 1].qkv_dg, rA, wA, dA);
        }
        quantize_lds(sc, F, xq, xd);
        __syncthreads();
        if constexpr (!POLLER) {
            float out[2 * UE];
            dot_rows<2 * UE, CF>(wE, dE, xq, xd, out);
            if (lane < kRep) {
                const uint32_t tg = make_tag(ep, l + 1, PH_X);
#pragma unroll
                for (int k = 0; k < UE; k++) {
                    if (!vE[k]) continue;
                    const int r = 2 * uE[k];
                    float d0 = vxm_bf16(out[2 * k]), d1 = vxm_bf16(out[2 * k + 1]);
                    if (p.res_scale != 1.0f) { d0 = d0 * p.res_scale; d1 = d1 * p.res_scale; }
                    put_word(p.xb + (((l + 1) & 1) * kRep + lane) * SX + uE[k],
                             pack_bf16x2(vxm_bf16(h1s[r] + d0), vxm_bf16(h1s[r + 1] + d1)), tg);
                }
            }
        }
    }
    // ---------------- final norm (workgroup 0) ----------------
    if (blockIdx.x != 0) return;
    const int Lyr = p.n_layers;
    if constexpr (POLLER) {
        poll_pairs<(H / 2 + 63) / 64>(p.xb + ((Lyr & 1) * kRep + rp) * SX, H / 2, make_tag(ep, Lyr, PH_X), xs, p.err,
                                      bail);
        if (p.final_norm) stage_f32(p.final_norm, H, gn);
    }
    __syncthreads();
    if (*bail) return;
    if (p.final_norm) {
        rmsnorm_lds(xs, gn, H, p.eps, h1s, red);
        for (int i = threadIdx.x; i < H; i += kThreads) p.x[i] = h1s[i];
    } else {
        for (int i = threadIdx.x; i < H; i += kThreads) p.x[i] = xs[i];
    }
}

}  // namespace

template <int H, int NH, int NKV, int HD, int F, int G>
__global__ __launch_bounds__(kThreads, 1) void k_decode_persistent(vxm_pparams p) {
    extern __shared__ float lds[];
    __shared__ int bail;
    if (threadIdx.x == 0) bail = 0;
    // bail is read only after the first __syncthreads of decode_run
    if ((threadIdx.x >> 6) == 0) decode_run<true, H, NH, NKV, HD, F, G>(p, lds, &bail);
    else decode_run<false, H, NH, NKV, HD, F, G>(p, lds, &bail);
}


// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct vxm_persistent_state {
    void *base = nullptr;
    vxm_player *layers = nullptr;
    uint64_t *xb = nullptr, *qkvb = nullptr, *attb = nullptr, *h1b = nullptr, *pb = nullptr;
    int *err = nullptr;
    uint32_t epoch = 0;
    const vxm_kv_cache *kv = nullptr;   // cache whose pointers are in the layer table
};

template <int H, int NH, int NKV, int HD, int F, int G>
static int launch_decode(vxm_ctx *ctx, const vxm_pparams &prm) {
    using L = Lds<H, NH * HD, F, HD>;
    const int lds = L::bytes(prm.cap);
    auto kern = k_decode_persistent<H, NH, NKV, HD, F, G>;
    if (lds > 64 * 1024)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "persistent decode: kv capacity %d needs %d B of LDS", prm.cap, lds);
    void *args[] = {(void *)&prm};
    VXM_HIP(ctx, hipLaunchCooperativeKernel((const void *)kern, dim3(G), dim3(kThreads), args, (unsigned)lds,
                                            ctx->stream));
    return VXM_OK;
}

// Supported shapes: (hidden, heads, kv heads, head dim, ffn).
static bool persistent_shape(const vxm_block_dims &d, int n_cu) {
    if (n_cu != 256) return false;
    if (d.H == 2048 && d.nh == 16 && d.nkv == 2 && d.hd == 128 && d.F == 6144) return true;
    if (d.H == 1024 && d.nh == 8 && d.nkv == 2 && d.hd == 128 && d.F == 2048) return true;
    return false;
}

// Largest cache capacity whose attention scores fit the 64 KiB of LDS.
int vxm_persistent_max_cap(const vxm_block_dims &d) {
    int cap = 1 << 16;
    auto fits = [&](int c) {
        return d.H == 2048 ? Lds<2048, 2048, 6144, 128>::bytes(c) <= 64 * 1024
                           : Lds<1024, 1024, 2048, 128>::bytes(c) <= 64 * 1024;
    };
    while (cap > 0 && !fits(cap)) cap -= 64;
    return cap;
}

bool vxm_persistent_supported(const vxm_minicpm4 *m, const vxm_kv_cache *kv) {
    return persistent_shape(m->dims, m->ctx->n_cu) && kv->cap <= vxm_persistent_max_cap(m->dims);
}

void vxm_persistent_free(vxm_minicpm4 *m) {
    if (m->pstate) {
        if (m->pstate->base) (void)hipFree(m->pstate->base);
        delete m->pstate;
        m->pstate = nullptr;
    }
}

int vxm_persistent_decode(vxm_minicpm4 *m, vxm_kv_cache *kv, float *x, int32_t pos) {
    vxm_ctx *ctx = m->ctx;
    const vxm_block_dims &d = m->dims;
    if (!persistent_shape(d, ctx->n_cu))
        return vxm_fail(ctx, VXM_ERR_NOT_IMPLEMENTED, "persistent decode: no kernel for this shape");
    if (kv->cap > vxm_persistent_max_cap(d))
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "persistent decode: kv capacity %d above %d", kv->cap,
                        vxm_persistent_max_cap(d));
    if (m->cfg.n_layers >= 512) return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "persistent decode: at most 511 layers");
    const int L = m->cfg.n_layers;
    const int64_t qd = (int64_t)d.nh * d.hd, kvd = (int64_t)d.nkv * d.hd;
    if (!m->pstate) m->pstate = new vxm_persistent_state();
    vxm_persistent_state &s = *m->pstate;
    if (!s.base) {
        const size_t tab = ((size_t)L * sizeof(vxm_player) + 255) & ~(size_t)255;
        const int nx = rep_stride((int)d.H / 2), nq = rep_stride((int)(qd + 2 * kvd) / 2),
                  na = rep_stride((int)qd), np_ = rep_stride((int)d.F / 2);
        const size_t words = (size_t)kRep * (2 * nx + nq + na + nx + np_);
        const size_t total = tab + words * 8 + 256;
        if (hipMalloc(&s.base, total) != hipSuccess) {
            (void)hipGetLastError();
            return vxm_fail(ctx, VXM_ERR_OOM, "persistent decode buffers failed");
        }
        char *b = (char *)s.base;
        s.layers = (vxm_player *)b;
        b += tab;
        s.xb = (uint64_t *)b; b += (size_t)kRep * 2 * nx * 8;
        s.qkvb = (uint64_t *)b; b += (size_t)kRep * nq * 8;
        s.attb = (uint64_t *)b; b += (size_t)kRep * na * 8;
        s.h1b = (uint64_t *)b; b += (size_t)kRep * nx * 8;
        s.pb = (uint64_t *)b; b += (size_t)kRep * np_ * 8;
        s.err = (int *)b;
        // tags start as all-ones: never equal to a live (epoch >= 1) tag
        VXM_HIP(ctx, hipMemsetAsync((char *)s.base + tab, 0xff, words * 8, ctx->stream));
        VXM_HIP(ctx, hipMemsetAsync(s.err, 0, 4, ctx->stream));
        s.kv = nullptr;
    }
    if (s.kv != kv) {
        std::vector<vxm_player> tabh(L);
        for (int l = 0; l < L; l++) {
            const vxm_block &b = m->blocks[l];
            tabh[l] = vxm_player{b.wqkv->qs, b.wo->qs, b.wgu->qs, b.wd->qs, b.wqkv->dg, b.wo->dg, b.wgu->dg,
                                 b.wd->dg, b.g_in, b.g_post, kv->k(l), kv->v(l)};
        }
        VXM_HIP(ctx, hipMemcpyAsync(s.layers, tabh.data(), L * sizeof(vxm_player), hipMemcpyHostToDevice,
                                    ctx->stream));
        VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        s.kv = kv;
    }
    s.epoch = (s.epoch + 1) & 0xfffffu;
    if (s.epoch == 0) s.epoch = 1;
    vxm_pparams prm{};
    prm.layers = s.layers;
    prm.n_layers = L;
    prm.final_norm = m->final_norm;
    prm.x = x;
    prm.xb = s.xb;
    prm.qkvb = s.qkvb;
    prm.attb = s.attb;
    prm.h1b = s.h1b;
    prm.pb = s.pb;
    prm.err = s.err;
    prm.ff = d.ff;
    prm.theta_scale = d.theta_scale;
    prm.eps = d.eps;
    prm.res_scale = d.res_scale;
    prm.pos = pos;
    prm.cap = kv->cap;
    prm.no_rope = d.no_rope;
    prm.epoch = s.epoch;
    if (d.H == 2048) return launch_decode<2048, 16, 2, 128, 6144, 256>(ctx, prm);
    return launch_decode<1024, 8, 2, 128, 2048, 256>(ctx, prm);
}

int vxm_persistent_check(vxm_minicpm4 *m) {
    if (!m->pstate || !m->pstate->err) return VXM_OK;
    int e = 0;
    VXM_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    VXM_HIP(m->ctx, hipMemcpy(&e, m->pstate->err, 4, hipMemcpyDeviceToHost));
    if (e) {
        VXM_HIP(m->ctx, hipMemset(m->pstate->err, 0, 4));
        return vxm_fail(m->ctx, VXM_ERR_BACKEND, "persistent decode: a workgroup timed out waiting for data");
    }
    return VXM_OK;
}
