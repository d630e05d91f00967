// decode_persistent.hip -- one decode token through the whole MiniCPM4 stack
// (vcpm_minicpm4_forward with n_tokens = 1, src/minicpm4.c:536-572) in ONE
// launch of one 512-thread workgroup per CU, all resident at once.
//
// Why one launch: on MI355X a dependent kernel boundary costs ~2.7 us (1.6 us
// in a HIP graph) against ~6.3 us of HBM streaming per layer; one launch per
// op would spend more time in boundaries than in streaming.
//
// Dataflow.  Each layer is five phases
//   A  rms_norm(x) -> Q8_0 -> QKV rows -> BF16 -> NEOX rope -> q, k, v
//   B  attention (+ f16 KV append), one workgroup per query head
//   C  O rows -> h1 = BF16(x + BF16(o))
//   D  rms_norm(h1) -> Q8_0 -> gate/up rows -> p = SwiGLU
//   E  Q8_0(p) -> down rows -> x' = BF16(h1 + BF16(d))
// Every phase publishes its outputs as 64-bit tagged words: a 32-bit tag
// (launch epoch, layer, phase) over 32 bits of payload -- two BF16 values
// (q/k/v, h1, p and x are all BF16-rounded by the reference graph) or one
// fp32 (the attention output).  Each word is one relaxed agent-scope atomic
// store, so no fence (and no L2 writeback) is ever needed: a consumer reads
// the words it needs until every tag is the expected one.  Every workgroup
// needs every element of its inputs, so the all-to-all dependency also
// protects the single-buffered channels against write-after-read.
//
// Work split.  In every phase workgroup g owns a fixed, contiguous block of
// weight rows (10 QKV, 8 O, 48 gate/up, 8 down rows at the TSLM shape).  Its
// rows are cut into units of 2 KiB (64 blocks: 2048 quants + 64 scales); the
// seven compute waves take units round-robin, so every wave streams the same
// number of bytes (+-1 unit).  Lane l of a wave owns block l of its unit, so
// a unit's dot product is 8 sdot4 per lane and one wave sum.  The partials of
// a row are added in unit order from LDS.
//
// Weight streaming.  Wave 0 issues no weight loads; waves 1..7 stream
// weights with direct-to-LDS loads (global_load_lds_dwordx4) into a ring of
// RING unit slots per wave, with a fixed lookahead of P units: after
// consuming the unit at stream position j the wave issues the loads of
// position j + P (which may belong to the next phase or the next layer), so
// the weights of the next phase are in flight while a phase waits for its
// inputs.  The loads are inline asm with explicit vmcnt waits: the compiler
// neither tracks them (its wait insertion would drain the ring at every phase
// branch) nor holds their data in registers (nothing it can spill or move
// before the data lands).  Barriers fence LDS only (s_barrier with
// LDS-scoped fences), so they never drain the weight loads in flight.
//
// Latency budget.  A wave64 VALU instruction issues once per 4 cycles and a
// workgroup has two waves per SIMD, so the serial work between two phases is
// counted in instructions: reductions run on DPP (not ds_bpermute), BF16
// rounding on v_cvt_pk_bf16_f32, RMSNorm's sum of squares is formed by the
// reading wave while it unpacks the input, and the norm is fused with the
// Q8_0 quantization over all 512 threads.
//
// The arithmetic per row is that of the GEMV kernel (q8_matmul.hip): per-block
// int32 sums, then (float)sumi * (d_w * d_x); only the fp32 order of the
// block terms differs (lane tree within a chunk, chunks in order).
#include <stdio.h>
#include <stdlib.h>

#include <mutex>
#include <utility>

#include "vxm_model.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Phase timestamps for profiling builds (-DVXM_PERSISTENT_TRACE): slot k of
// layer l of this workgroup gets the 100 MHz real-time counter.  Compiled
// out of the library.
constexpr int kTraceSlots = 16;
#ifdef VXM_PERSISTENT_TRACE
#define VXM_TS(cond, k)                                                                              \
    do {                                                                                             \
        if ((cond) && p.trace)                                                                       \
            p.trace[(size_t)blockIdx.x * p.trace_stride + 2 + l * kTraceSlots + (k)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define VXM_TS(cond, k) do { } while (0)
#endif

namespace {

#ifndef VXM_WAVES
#define VXM_WAVES 8
#endif
constexpr int kWaves = VXM_WAVES;      // waves per workgroup: kNR readers + the compute waves
// Waves that read each exchanged input: x (phase A), the attention output
// (phase C), h1 (phase D) and p (phase E).  An exchange read is a round of
// agent-scope loads whose cost is their issue and their trip to the memory
// side, so spreading a round over more waves shortens it, even over compute
// waves whose own refill loads are still in flight (their loads retire in
// issue order).  Measured over the 28-layer decode (us per token), with 16
// channel replicas: x / att / h1 / p read by 2 / 2 / 1 / 4 waves 741-748; p by
// 1 wave 832; everything by wave 0 alone 863; 8 / 8 / 1 / 8 waves 722;
// 8 / 8 / 4 / 8 692; 8 / 8 / 8 / 8 694; 4 / 8 / 4 / 8 707; 8 / 4 / 4 / 8 698.
// With 4 replicas: 8 / 8 / 8 / 8 664; 8 / 8 / 4 / 8 667; 8 / 8 / 2 / 8 671;
// 4 / 8 / 4 / 8 676; 8 / 4 / 4 / 8 672; 8 / 8 / 4 / 4 680.
#ifndef VXM_X_READERS
#define VXM_X_READERS 8
#endif
#ifndef VXM_ATT_READERS
#define VXM_ATT_READERS 8
#endif
#ifndef VXM_P_READERS
#define VXM_P_READERS 8
#endif
#ifndef VXM_H1_READERS
#define VXM_H1_READERS 8
#endif
constexpr int kXReaders = VXM_X_READERS, kAttReaders = VXM_ATT_READERS, kPReaders = VXM_P_READERS;
constexpr int kH1Readers = VXM_H1_READERS;

// Waves 0 .. kNR-1 issue no weight loads (their exchange reads never wait behind
// a refill); the others stream weights through the ring and compute.
#ifndef VXM_NREADERS
#define VXM_NREADERS 1
#endif
constexpr int kNR = VXM_NREADERS;
// 1: the second part of phase D's ring refills is issued by the reader wave during
// phase E (ring_refill_readers); 0: by each compute wave before E's Q8_0 of p
#ifndef VXM_D2_READER
#define VXM_D2_READER 1
#endif
constexpr bool kD2Reader = VXM_D2_READER && VXM_NREADERS == 1;
constexpr int kCW = kWaves - kNR;
constexpr int kThreads = kWaves * 64;
constexpr int kG = 256;                // workgroups: one per CU
constexpr int kSpin = 1 << 17;         // poll rounds before giving up
#ifndef VXM_LOOK
#define VXM_LOOK 7
#endif
constexpr int kLook = VXM_LOOK;        // 2 KiB weight units in the LDS ring per compute wave
constexpr int kUnit = 2048;            // quant bytes per unit (64 blocks)
constexpr int kSlot = kUnit + 128;     // LDS bytes per ring slot: quants, then 64 fp16 scales
// Every channel is written as kRep replicas; workgroup b reads replica
// b % kRep, so the coherent loads of 256 workgroups spread over more lines.
// Each replica costs its producer one more agent-scope store per word:
// measured (us per token) 32 replicas 741, 16 693, 8 677, 4 667, 2 666, 1 672;
// with today's phases 8 replicas 568, 4 555.6, 2 550.6, 1 551.5.
#ifndef VXM_REPLICAS
#define VXM_REPLICAS 2
#endif
constexpr int kRep = VXM_REPLICAS;
constexpr int kPad = 64;               // words between replicas

__host__ __device__ constexpr int rep_stride(int words) { return words + kPad; }
__host__ __device__ constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ constexpr int cmax(int a, int b) { return a > b ? a : b; }

enum Phase { PH_X = 0, PH_QKV = 1, PH_ATT = 2, PH_H1 = 3, PH_P = 4, PH_ATTP = 5 };

// Long contexts split each head's keys over up to kAttSplitMax workgroups
// (chunks); every chunk publishes its softmax-normalised output with its
// score max m and exp sum l as kAttpWords tagged words (o[HD], m, l).
constexpr int kAttSplitMax = 16;
constexpr int kAttpWords = 132;

template <int H_, int NH_, int NKV_, int HD_, int F_>
struct Shape {
    static constexpr int H = H_, NH = NH_, NKV = NKV_, HD = HD_, F = F_;
    static constexpr int QD = NH * HD, KVD = NKV * HD, NQKV = QD + 2 * KVD;
    static constexpr int QPK = NH / NKV;
    // rows per workgroup per phase, 2 KiB units per row, units per workgroup
    static constexpr int RA = NQKV / kG, RC = H / kG, RD = 2 * F / kG, RE = H / kG;
    static constexpr int CA = H / kUnit, CC = QD / kUnit, CD = H / kUnit, CE = F / kUnit;
    static constexpr int UA = RA * CA, UC = RC * CC, UD = RD * CD, UE = RE * CE;
    // ring slots per compute wave: A, C, D, E units of one layer
    static constexpr int SA = cdiv(UA, kCW), SC = cdiv(UC, kCW), SD = cdiv(UD, kCW), SE = cdiv(UE, kCW);
    static constexpr int OA = 0, OC = SA, OD = SA + SC, OE = SA + SC + SD, NS = SA + SC + SD + SE;
    // lookahead: as many units as the widest phase gives one wave (SD for the
    // MLP), so a phase's whole share of weights is in flight while it waits
    // for its inputs
    static constexpr int P = kLook < NS ? kLook : NS;
    static_assert(P >= SD && P >= SE, "the lookahead covers a phase");
    // the ring has P slots: stream position q = l*NS + s lives in slot q % P,
    // and the unit issued when q is consumed (q + P) takes q's slot
    static constexpr int RING = P;
    static constexpr int RING_BYTES = kCW * RING * kSlot;
    static constexpr int UMAX = cmax(cmax(UA, UC), cmax(UD, UE));
    static constexpr int KMAX = cmax(cmax(H, QD), F);
    // att (QD fp32) / p (F BF16 values as F/2 pairs) / final norm (H fp32) /
    // attention scores (cap + 1 fp32, phase B only)
    static constexpr int BIG = cmax(cmax(QD, F / 2), H);
    static_assert(NQKV % kG == 0 && H % kG == 0 && (2 * F) % kG == 0, "rows must split over 256 workgroups");
    static_assert(RA % 2 == 0 && RC % 2 == 0 && RD % 4 == 0 && RE % 2 == 0, "rows per workgroup");
    static_assert(H % kUnit == 0 && QD % kUnit == 0 && F % kUnit == 0, "K must be a multiple of 2048");
    static_assert(H <= 4 * kThreads && (H & (H - 1)) == 0, "hidden: one norm pass, power of two");
    static_assert(HD == 128 && NH % NKV == 0, "heads: the attention maps one key to a row of 16 lanes");
    static_assert(NH <= kG && QPK * 8 <= kG && NH <= 64, "attention workgroups");
    static_assert(((NKV * kAttSplitMax - 1) / 8 * QPK + QPK - 1) * 8 + 7 < kG, "attention chunk workgroups");
    // LDS layout, in floats (the int8 quants go last, 16-byte aligned)
    static constexpr int L_XS = 0;                  // layer input x              [H]
    static constexpr int L_H1 = L_XS + H;           // h1                         [H]
    static constexpr int L_GN = L_H1 + H;           // RMSNorm gain of the phase  [H]
    static constexpr int L_BIG = L_GN + H;          // att / p / final norm / scores [BIG]
    static constexpr int L_XD = L_BIG + BIG;        // activation block scales    [KMAX/32]
    static constexpr int L_CS = L_XD + KMAX / 32;   // rope cos/sin               [HD]
    static constexpr int L_AQ = L_CS + HD;          // attention q, k, v          [3 HD]
    static constexpr int L_PART = L_AQ + 3 * HD;    // unit partials              [UMAX]
    static constexpr int L_RED = L_PART + UMAX;     // reductions / wave partials [kWaves * HD]
    static constexpr int L_END = L_RED + kWaves * HD;
    static constexpr int XQ_OFF = (L_END * 4 + 15) & ~15;          // int8 quants [KMAX]
    static constexpr int RING_OFF = XQ_OFF + KMAX;                   // 16-byte aligned
    static constexpr int BYTES = RING_OFF + RING_BYTES;
    // a chunk's scores fit BIG; the chunk-0 workgroup gathers every chunk's
    // (o, m, l) in the same space
    static constexpr int MAX_CAP = kAttSplitMax * BIG - 1;
    static_assert(kAttSplitMax * (HD + 2) <= BIG && HD + 2 <= kAttpWords, "chunk partials fit the score space");
};

// workgroup that runs the attention of query head h: the heads of one kv
// group land on workgroups of one XCD (dispatch is round-robin over the 8
// XCDs), so the group's K/V rows are shared through that XCD's L2.
template <class S>
__device__ __forceinline__ int attn_wg(int h) { return (h % S::QPK) * 8 + h / S::QPK; }

// Workgroup of chunk c of query head h: (kv group g, chunk c) is combination
// k = c * NKV + g, whose QPK heads share one XCD (x = k % 8) and so read the
// chunk's K/V rows through one L2; chunk 0 is attn_wg(h).  Injective over
// h < NH, c < kAttSplitMax: workgroup (sb * QPK + h % QPK) * 8 + x with
// sb = k / 8.
template <class S>
__device__ __forceinline__ int attn_wg_chunk(int h, int c) {
    const int k = c * S::NKV + h / S::QPK;
    return ((k / 8) * S::QPK + h % S::QPK) * 8 + k % 8;
}

__device__ __forceinline__ uint32_t make_tag(uint32_t epoch, int layer, int phase) {
    return (epoch << 12) | ((uint32_t)layer << 3) | (uint32_t)phase;
}

// F32 -> BF16 (round to nearest even) -> F32 on v_cvt_pk_bf16_f32; the same
// rounding as minicpm_bf16_round (src/minicpm4.c:39-42) for every non-NaN.
__device__ __forceinline__ float bf16r(float f) { return (float)(__bf16)f; }

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

// Workgroup barrier that orders LDS only.  Global traffic between waves of a
// workgroup goes through the agent-scope tagged words, so the barrier never
// has to wait for the weight loads in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ int dot16(const v4i a, const v4i b) {
    int acc = __builtin_amdgcn_sdot4(a.x, b.x, 0, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

// ---- cross-lane reductions on DPP (VALU data sharing, a few cycles per step;
// __shfl_xor goes through ds_bpermute at LDS latency) ----------------------
// dpp control codes (GFX9): quad_perm, row_shr:n = 0x110 + n,
// row_half_mirror = 0x141, row_bcast:15 = 0x142, row_bcast:31 = 0x143
constexpr int kDppXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppMirror8 = 0x141;

template <int CTRL, int RM = 0xF>
__device__ __forceinline__ int dpp_i(int v) {   // lanes with no source (or outside RM) read 0
    return __builtin_amdgcn_update_dpp(0, v, CTRL, RM, 0xF, false);
}
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL, RM>(__float_as_int(v)));
}
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ float dpp_keep_f(float v) {   // lanes with no source keep v
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, RM, 0xF, false));
}
template <int CTRL, int RM = 0xF>
__device__ __forceinline__ double dpp_d(double v) {
    const int lo = dpp_i<CTRL, RM>(__double2loint(v)), hi = dpp_i<CTRL, RM>(__double2hiint(v));
    return __hiloint2double(hi, lo);
}

// inclusive prefix sums within rows of 16, then across rows: lane 63 holds
// the wave total (lane 15 + 16r holds the total of rows 0..r)
__device__ __forceinline__ float wave_sum_63(float v) {
    v += dpp_f<0x111>(v);
    v += dpp_f<0x112>(v);
    v += dpp_f<0x114>(v);
    v += dpp_f<0x118>(v);
    v += dpp_f<0x142, 0xA>(v);
    v += dpp_f<0x143, 0xC>(v);
    return v;
}
// Two independent wave_sum_63 chains interleaved, so each DPP step of one
// hides the latency of the other's.
__device__ __forceinline__ void wave_sum_63_x2(float &a, float &b) {
    a += dpp_f<0x111>(a); b += dpp_f<0x111>(b);
    a += dpp_f<0x112>(a); b += dpp_f<0x112>(b);
    a += dpp_f<0x114>(a); b += dpp_f<0x114>(b);
    a += dpp_f<0x118>(a); b += dpp_f<0x118>(b);
    a += dpp_f<0x142, 0xA>(a); b += dpp_f<0x142, 0xA>(b);
    a += dpp_f<0x143, 0xC>(a); b += dpp_f<0x143, 0xC>(b);
}
__device__ __forceinline__ double wave_sum_63_d(double v) {
    v += dpp_d<0x111>(v);
    v += dpp_d<0x112>(v);
    v += dpp_d<0x114>(v);
    v += dpp_d<0x118>(v);
    v += dpp_d<0x142, 0xA>(v);
    v += dpp_d<0x143, 0xC>(v);
    return v;
}
__device__ __forceinline__ float wave_max_63(float v) {
    v = fmaxf(v, dpp_keep_f<0x111>(v));
    v = fmaxf(v, dpp_keep_f<0x112>(v));
    v = fmaxf(v, dpp_keep_f<0x114>(v));
    v = fmaxf(v, dpp_keep_f<0x118>(v));
    v = fmaxf(v, dpp_keep_f<0x142, 0xA>(v));
    v = fmaxf(v, dpp_keep_f<0x143, 0xC>(v));
    return v;
}
// sum over each row of 16 lanes, valid in lane 15 of the row
__device__ __forceinline__ float row16_sum_15(float v) {
    v += dpp_f<0x111>(v);
    v += dpp_f<0x112>(v);
    v += dpp_f<0x114>(v);
    v += dpp_f<0x118>(v);
    return v;
}
// max over each aligned group of 8 lanes, valid in all 8
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    v = fmaxf(v, dpp_f<kDppMirror8>(v));
    return v;
}

__device__ __forceinline__ float swiglu(float g, float u) {
    const float gb = bf16r(g);
    const float s = bf16r(__fdiv_rn(gb, 1.0f + expf(-gb)));
    return bf16r(s * bf16r(u));
}

// A zero the compiler cannot see through: address arithmetic that uses it is
// recomputed where it is needed instead of being hoisted out of the layer
// loop, which would keep ~100 loop-invariant offsets live in registers.
__device__ __forceinline__ int opaque_zero() {
    int z = 0;
    asm volatile("" : "+s"(z));
    return z;
}
__device__ __forceinline__ int opaque_v(int x) {   // per-lane value, recomputed at each use
    asm volatile("" : "+v"(x));
    return x;
}
// threadIdx.x through an opaque copy: the index arithmetic of a helper that
// runs inside the layer loop stays there instead of being hoisted (with long
// live ranges) into the kernel prologue.
__device__ __forceinline__ int tid_now() { return opaque_v((int)threadIdx.x); }

}  // namespace

struct vxm_player {
    const int8_t *qkv_qs, *o_qs, *gu_qs, *d_qs;
    const uint16_t *qkv_d, *o_d, *gu_d, *d_d;   // natural scale layout [rows][k/32]
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
    uint64_t *qkvb;    // [NQKV/2] q, k (rope'd, pair-interleaved per head) and v (BF16 pairs)
    uint64_t *attb;    // Q8_0 attention output: [NH][HD/4] quant words, then [NH][HD/32] scales (room for QD words)
    uint64_t *h1b;     // [H/2] BF16 pairs
    uint64_t *pb;      // [F/2] BF16 pairs
    uint64_t *attp;    // [NH][kAttSplitMax][kAttpWords] chunk partials (fp32), long contexts only
    int att_split;     // key chunks per head (1: one workgroup per head)
    const int8_t *dummy_q;     // 2 KiB of zeros: loads of units a wave does not own
    const uint16_t *dummy_d;   // 64 zero scales
    // [0] live: set by a workgroup that gave up waiting, polled by the others,
    // cleared at the end of the launch by its last workgroup; [1] sticky: also
    // set, read and cleared by vxm_minicpm4_check
    int *err;
    // [0] launch epoch (read by every workgroup at start, advanced by the last
    // workgroup to finish), [1] workgroups finished in this launch
    uint32_t *state;
    uint64_t n_chan;   // words of the channels xb .. attp (contiguous), reset when the epoch wraps
    // debug: [n_layers + 1][H] -- the input of every layer and the last layer's
    // output before the final norm (written by workgroup 0), or null
    float *dump;
    const float2 *rope_cs;   // (cos, sin) table [position][HD/2]
    float eps, res_scale;
    int pos, cap, no_rope;
#ifdef VXM_PERSISTENT_TRACE
    uint64_t *trace;
    int trace_stride;
#endif
};

namespace {

// The layer table through the constant address space: the compiler then
// reads it with scalar loads (counted by lgkmcnt).  A vector load of a
// pointer would be counted by vmcnt, which retires in order, so waiting for
// it would also wait for every weight load in flight.
typedef const __attribute__((address_space(4))) vxm_player *vxm_ptab;
__device__ __forceinline__ vxm_ptab layer_tab(const vxm_pparams &p) { return (vxm_ptab)p.layers; }
// Entry l of the layer table through a uniform address.  Under register
// pressure the compiler may keep l or the table base in VGPRs; the entry's
// fields would then be fetched with vector loads, whose in-order completion
// (vmcnt) would make every fetch wait for the whole weight ring.  Read-first-
// lane makes the address scalar, so the fields are scalar (lgkmcnt) loads.
__device__ __forceinline__ vxm_ptab layer_at(const vxm_pparams &p, int l) {
    const uint64_t a = (uint64_t)(uintptr_t)(layer_tab(p) + l);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return (vxm_ptab)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ bool give_up(const vxm_pparams &p, int &it, int *bail) {
    // the error word (another workgroup gave up) is polled every 32nd round:
    // each read of it is one more round trip to the memory side (631 -> 628 us
    // per token)
    if (++it > kSpin || ((it & 31) == 0 && __hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
        __hip_atomic_store(p.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p.err + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *bail = 1;
        return true;
    }
    return false;
}

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// A channel replica as a buffer resource; 16-byte loads through it carry the sc1
// bit (aux 16), so, like agent-scope atomic loads, they bypass the non-coherent
// caches.  Each 8-byte half of a load is one word written by one 64-bit atomic
// store, so each half is whole; the two halves are checked separately.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t chan_rsrc(const uint64_t *base, int words) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, words * 8, 0x00020000);
}
__device__ __forceinline__ v4u load_pair(__amdgpu_buffer_rsrc_t rs, int pair) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, pair * 16, 0, 16);
}

// One reading wave: the np word pairs src[2i], src[2i + 1] (i < np; lane l owns
// pairs l + 64k, all loads of a round in flight, 16 bytes each) into LDS:
// PAIRS unpacks the four BF16 values of a pair to dst[4i .. 4i + 3], RAW stores
// the two BF16 pairs as they are, otherwise two fp32 to dst[2i], dst[2i + 1].
// Pairs not yet carrying `tag` in both words are read again next round.
// Returns this lane's sum of the squares of its values in double (each square
// exact for BF16-valued inputs).
template <int NPP, bool PAIRS, bool RAW = false>
__device__ double read_words(const vxm_pparams &p, const uint64_t *src, int np, uint32_t tag, float *dst, int *bail) {
    static_assert(NPP <= 32, "pairs per lane");
    const int lane = tid_now() & 63;
    const __amdgpu_buffer_rsrc_t rs = chan_rsrc(src, 2 * np);
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < NPP; k++)
        if (lane + 64 * k < np) pending |= 1u << k;
    double ss = 0.0;
    int it = 0;
    while (true) {
        v4u w[NPP];
#pragma unroll
        for (int k = 0; k < NPP; k++)
            if (pending & (1u << k)) w[k] = load_pair(rs, lane + 64 * k);
#pragma unroll
        for (int k = 0; k < NPP; k++) {
            if ((pending & (1u << k)) && w[k].y == tag && w[k].w == tag) {
                const int i = lane + 64 * k;
                if (RAW) {
                    *(uint2 *)(dst + 2 * i) = make_uint2(w[k].x, w[k].z);   // the BF16 pairs as they are
                } else if (PAIRS) {
                    const float a0 = __uint_as_float(w[k].x << 16), b0 = __uint_as_float(w[k].x & 0xffff0000u);
                    const float a1 = __uint_as_float(w[k].z << 16), b1 = __uint_as_float(w[k].z & 0xffff0000u);
                    *(float4 *)(dst + 4 * i) = make_float4(a0, b0, a1, b1);
                    ss += ((double)(a0 * a0) + (double)(b0 * b0)) + ((double)(a1 * a1) + (double)(b1 * b1));
                } else {
                    *(float2 *)(dst + 2 * i) = make_float2(__uint_as_float(w[k].x), __uint_as_float(w[k].z));
                }
                pending &= ~(1u << k);
            }
        }
        if (__all(pending == 0)) break;
        if (give_up(p, it, bail)) break;
        __builtin_amdgcn_s_sleep(1);
    }
    return ss;
}

// Word pairs [p0, p0 + np) of a Q8_0 channel (16-byte loads): words below nq
// (even) hold four quants each (stored to xq as they are), the words from nq on
// one block scale each (to xd[i - nq]).  Polls until every word carries tag.
template <int NPP>
__device__ void read_q8_words(const vxm_pparams &p, const uint64_t *src, int p0, int np, int nq, uint32_t tag,
                              int8_t *xq, float *xd, int *bail) {
    static_assert(NPP <= 32, "pairs per lane");
    const int lane = tid_now() & 63;
    const __amdgpu_buffer_rsrc_t rs = chan_rsrc(src, 2 * (p0 + np));
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < NPP; k++)
        if (lane + 64 * k < np) pending |= 1u << k;
    int it = 0;
    while (true) {
        v4u w[NPP];
#pragma unroll
        for (int k = 0; k < NPP; k++)
            if (pending & (1u << k)) w[k] = load_pair(rs, p0 + lane + 64 * k);
#pragma unroll
        for (int k = 0; k < NPP; k++) {
            if ((pending & (1u << k)) && w[k].y == tag && w[k].w == tag) {
                const int i = 2 * (p0 + lane + 64 * k);
                if (i < nq) *(uint2 *)(xq + 4 * i) = make_uint2(w[k].x, w[k].z);
                else *(float2 *)(xd + i - nq) = make_float2(__uint_as_float(w[k].x), __uint_as_float(w[k].z));
                pending &= ~(1u << k);
            }
        }
        if (__all(pending == 0)) break;
        if (give_up(p, it, bail)) break;
        __builtin_amdgcn_s_sleep(1);
    }
}

// Wave 0: wait until the first word of each of the n producers (word i * stride)
// carries tag.  Used where the wait is long (the attention output), so that
// 240 waiting workgroups read 16 words per round instead of 2048.
__device__ void wait_sentinels(const vxm_pparams &p, const uint64_t *src, int n, int stride, uint32_t tag,
                               int *bail) {
    const int lane = tid_now() & 63;
    bool done = lane >= n;
    int it = 0;
    while (true) {
        if (!done) done = (uint32_t)(get_word(src + lane * stride) >> 32) == tag;
        if (__all(done)) return;
        if (give_up(p, it, bail)) return;
        __builtin_amdgcn_s_sleep(2);
    }
}

// Wave 0: plain copy of n floats (gains) into LDS, n % 256 == 0
__device__ __forceinline__ void stage_f32(const float *src, int n, float *dst) {
    const int lane = tid_now() & 63;
    for (int i = lane * 4; i < n; i += 256) *(float4 *)(dst + i) = *(const float4 *)(src + i);
}

__device__ __forceinline__ double wg_sum_d(double v, float *red) {
    v = wave_sum_63_d(v);
    double *r = (double *)red;
    lds_barrier();
    if ((tid_now() & 63) == 63) r[tid_now() >> 6] = v;
    lds_barrier();
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < kWaves; i++) t += r[i];
    return t;
}

__device__ __forceinline__ float wg_max_f(float v, float *red) {
    v = wave_max_63(v);
    lds_barrier();
    if ((tid_now() & 63) == 63) red[tid_now() >> 6] = v;
    lds_barrier();
    float t = red[0];
#pragma unroll
    for (int i = 1; i < kWaves; i++) t = fmaxf(t, red[i]);
    return t;
}

// Q8_0 (x86 rule: id = 127/amax, round half even) of 4 values held by each
// lane of an aligned group of 8 lanes (one 32-value block); writes the four
// quants and, from the group's first lane, the fp16-rounded block scale.
// The same in registers: the four quants packed low byte first, and the block
// scale as the consumer uses it (fp16-rounded, as float).
__device__ __forceinline__ void quant4_reg(const float v[4], uint32_t &w, float &dsc) {
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = max8(amax);
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    w = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float q = fminf(fmaxf(rintf(v[i] * id), -128.0f), 127.0f);
        w |= (uint32_t)(uint8_t)(int8_t)(int)q << (8 * i);
    }
    dsc = vxm_h2f(vxm_f2h(d));
}

__device__ __forceinline__ void quant4(const float v[4], int8_t *xq4, float *xd1, bool first) {
    uint32_t w;
    float dsc;
    quant4_reg(v, w, dsc);
    *(uint32_t *)xq4 = w;
    if (first) *xd1 = dsc;
}

// Q8_0 of n BF16 values stored as pairs (low half first) in LDS.  Two lanes
// (an even lane and the next) take one 32-value block, 16 values each, in a
// single pass for n <= 32 kThreads: the block max is one DPP step and the two
// divisions of the scale are issued once per 16 values instead of once per 4
// (the activation of the down projection: 1.76 -> 0.3 us per layer).  The
// arithmetic per value is quant4_reg's.
__device__ void quantize_lds_bf16x2(const uint32_t *src, int n, int8_t *xq, float *xd) {
    const int t = tid_now();
    for (int base = t * 16; base < n; base += kThreads * 16) {
        const uint4 a = *(const uint4 *)(src + base / 2), b = *(const uint4 *)(src + base / 2 + 4);
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float v[16];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
            amax = fmaxf(amax, fmaxf(fabsf(v[2 * i]), fabsf(v[2 * i + 1])));
        }
        amax = fmaxf(amax, dpp_f<kDppXor1>(amax));   // the other half of the block
        const float d = __fdiv_rn(amax, 127.0f);
        const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
        uint32_t q4[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            q4[j] = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float q = fminf(fmaxf(rintf(v[4 * j + i] * id), -128.0f), 127.0f);
                q4[j] |= (uint32_t)(uint8_t)(int8_t)(int)q << (8 * i);
            }
        }
        *(uint4 *)(xq + base) = make_uint4(q4[0], q4[1], q4[2], q4[3]);
        if ((t & 1) == 0) xd[base / 32] = vxm_h2f(vxm_f2h(d));
    }
}

// vcpm_rms_norm (src/minicpm4.c:132-152) fused with the Q8_0 of its output:
// y = BF16(BF16(x * sc) * g), sc = 1 / sqrt(sum(x^2) / n + eps), 4 values per
// thread, n <= 4 * kThreads.  sumsq is the double sum of squares, formed in a
// tree order by the reading waves: equal to ggml's sequential double while the
// squares span less than about 2^26 (every partial sum exact), else possibly one
// rounding apart.
template <int N>
__device__ __forceinline__ void norm_quant(const float *x, const float *g, double sumsq, float eps, int8_t *xq,
                                           float *xd) {
    const float mean = (float)(sumsq * (1.0 / (double)N));   // N is a power of two: exact
    const float sc = __fdiv_rn(1.0f, __fsqrt_rn(mean + eps));
    const int base = tid_now() * 4;
    if (base < N) {
        const float4 a = *(const float4 *)(x + base), b = *(const float4 *)(g + base);
        const float v[4] = {bf16r(bf16r(a.x * sc) * b.x), bf16r(bf16r(a.y * sc) * b.y),
                            bf16r(bf16r(a.z * sc) * b.z), bf16r(bf16r(a.w * sc) * b.w)};
        quant4(v, xq + base, xd + base / 32, (tid_now() & 7) == 0);
    }
}

// vcpm_rms_norm of src (LDS) with gain (LDS) into dst (LDS), all threads.
__device__ void rmsnorm_lds(const float *src, const float *gain, int n, float eps, float *dst, float *red) {
    double ss = 0.0;
    for (int i = tid_now(); i < n; i += kThreads) ss += (double)(src[i] * src[i]);
    const double tot = wg_sum_d(ss, red);
    const float mean = (float)(tot / (double)n);
    const float sc = __fdiv_rn(1.0f, __fsqrt_rn(mean + eps));
    for (int i = tid_now(); i < n; i += kThreads) dst[i] = bf16r(bf16r(src[i] * sc) * gain[i]);
}

// ---- the weight ring ---------------------------------------------------------
// Slot s of a compute wave's per-layer schedule belongs to phase ph(s) and is
// its k-th unit: workgroup-local unit u = ci + 7k (ci = compute wave index).
template <class S, int s>
struct Slot {
    static constexpr int ph = s < S::OC ? 0 : s < S::OD ? 1 : s < S::OE ? 2 : 3;
    static constexpr int k = s - (ph == 0 ? S::OA : ph == 1 ? S::OC : ph == 2 ? S::OD : S::OE);
    static constexpr int U = ph == 0 ? S::UA : ph == 1 ? S::UC : ph == 2 ? S::UD : S::UE;
    static constexpr int C = ph == 0 ? S::CA : ph == 1 ? S::CC : ph == 2 ? S::CD : S::CE;
    static constexpr int R = ph == 0 ? S::RA : ph == 1 ? S::RC : ph == 2 ? S::RD : S::RE;
};

// The ring's loads: direct-to-LDS DMA issued as inline asm.  Lane l of
// global_load_lds_dwordx4 writes its 16 bytes at M0 + 16 l.  The loads are
// non-temporal (nt): each weight byte is read once per token, and keeping it
// out of the caches leaves them to the exchanged words: 635 -> 631 us per
// token.  A unit is three
// instructions: quants [0, 1024) and [1024, 2048) by all lanes, and the 128
// bytes of scales by lanes 0..7 (exec narrowed inside the asm and restored).
// Before the DMA overwrites a slot, lgkmcnt(0) guarantees that the wave's
// LDS reads of the slot's previous unit have completed.
__device__ __forceinline__ void dma_unit(uint32_t lds_slot, const int8_t *q, const uint16_t *d, int lane, bool live) {
    const int8_t *q0 = q + lane * 16;
    const int8_t *q1 = q0 + 1024;
    const char *dd = (const char *)d + (lane & 7) * 16;
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_slot);
    // a unit the wave does not own (15 of the 105 slots of a layer at the
    // TSLM shape) loads with one lane: the instructions still count in vmcnt,
    // which the ring's waits rely on, but cost the address unit and the
    // memory side almost nothing (627 -> 622 us per token)
    const uint64_t mq = live ? ~0ull : 1ull, md = live ? 0xffull : 1ull;
    uint64_t saved;
    uint32_t saved_m0;
    // m0 and exec are saved and restored inside the statement, so the
    // compiler's view of both is unchanged
    asm volatile(
        "s_waitcnt lgkmcnt(0)\n\t"
        "s_mov_b32 %1, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, %6\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %3, off nt\n\t"
        "s_add_u32 m0, m0, 1024\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %4, off nt\n\t"
        "s_add_u32 m0, m0, 1024\n\t"
        "s_mov_b64 exec, %7\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %5, off nt\n\t"
        "s_mov_b64 exec, %0\n\t"
        "s_mov_b32 m0, %1"
        : "=&s"(saved), "=&s"(saved_m0)
        : "s"(m0v), "v"(q0), "v"(q1), "v"(dd), "s"(mq), "s"(md)
        : "memory", "scc");
}

// Wait until at most N vector memory instructions of the wave are pending
// (they retire in order).
template <int N>
__device__ __forceinline__ void ring_wait() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The four weight streams of one layer (quants and scales of QKV, O,
// gate/up, down), read from the table once per layer and then held in
// registers: the DMA statement clobbers memory, so an address derived from a
// table load inside the ring would be re-fetched (and waited for) before
// every unit's DMAs.  valid = 0 past the last layer.
struct UnitBases {
    const int8_t *q[4];
    const uint16_t *d[4];
    int valid;
};

__device__ __forceinline__ UnitBases unit_bases(const vxm_pparams &p, int l) {
    UnitBases b{};
    b.valid = l < p.n_layers;
    if (b.valid) {
        vxm_ptab Ly = layer_at(p, l);
        b.q[0] = Ly->qkv_qs; b.q[1] = Ly->o_qs; b.q[2] = Ly->gu_qs; b.q[3] = Ly->d_qs;
        b.d[0] = Ly->qkv_d;  b.d[1] = Ly->o_d;  b.d[2] = Ly->gu_d;  b.d[3] = Ly->d_d;
    }
    return b;
}

// Weight addresses of slot s for compute wave ci in the layer of B (the zero
// buffers past the last layer or for a unit the wave does not own, so every
// wave issues the same count of loads).
template <class S, int s>
__device__ __forceinline__ void unit_addr(const vxm_pparams &p, const UnitBases &B, int wg, int ci,
                                          const int8_t *&q, const uint16_t *&d, bool &live) {
    using T = Slot<S, s>;
    const int u = ci + kCW * T::k;
    q = p.dummy_q;
    d = p.dummy_d;
    live = u < T::U && B.valid;
    if (live) {
        const int row = wg * T::R + u / T::C, c = u % T::C;
        constexpr int K = T::C * kUnit;
        q = B.q[T::ph] + (int64_t)row * K + c * kUnit;
        d = B.d[T::ph] + (int64_t)row * (K / 32) + c * (kUnit / 32);
    }
}

// Ring slot of stream position l*NS + s (l is uniform: a scalar computation).
template <class S, int s>
__device__ __forceinline__ int ring_slot(int l) {
    return __builtin_amdgcn_readfirstlane((l * S::NS + s) % S::RING);
}

// Issue the DMAs of slot s of layer l (weights of B) into its ring slot.
template <class S, int s>
__device__ __forceinline__ void ring_issue(const vxm_pparams &p, const UnitBases &B, uint32_t ring_lds, int l, int wg,
                                           int ci, int lane) {
    const int8_t *q;
    const uint16_t *d;
    bool live;
    unit_addr<S, s>(p, B, wg, ci, q, d, live);
    dma_unit(ring_lds + ring_slot<S, s>(l) * kSlot, q, d, lane, live);
}

template <class S, int... ss>
__device__ __forceinline__ void ring_prime(const vxm_pparams &p, const UnitBases &B0, uint32_t ring_lds, int wg,
                                           int ci, int lane, std::integer_sequence<int, ss...>) {
    (ring_issue<S, ss>(p, B0, ring_lds, 0, wg, ci, lane), ...);
}

// The operands of one ring unit for lane l (block l of the unit): its 32
// weight quants and scale, and the activation's block of the unit's K chunk.
struct UnitOps {
    v4i w0, w1, x0, x1;
    float xs;
    uint32_t dw;
};

template <class S, int s>
__device__ __forceinline__ UnitOps unit_load(const int8_t *ring, int l, int ci, int lane, const int8_t *xq,
                                             const float *xd) {
    using T = Slot<S, s>;
    const int u = ci + kCW * T::k;
    const int c = u % T::C;
    const int8_t *slot = ring + ring_slot<S, s>(l) * kSlot;
    UnitOps o;
    o.x0 = *(const v4i *)(xq + c * kUnit + lane * 32);
    o.x1 = *(const v4i *)(xq + c * kUnit + lane * 32 + 16);
    o.xs = xd[c * (kUnit / 32) + lane];
    o.w0 = *(const v4i *)(slot + lane * 32);
    o.w1 = *(const v4i *)(slot + lane * 32 + 16);
    o.dw = *(const uint16_t *)(slot + kUnit + lane * 2);
    return o;
}

// This lane's term of the unit's partial: the exact int32 block sum times
// d_w * d_x.
__device__ __forceinline__ float unit_term(const UnitOps &o) {
    const int si = dot16(o.w1, o.x1) + dot16(o.w0, o.x0);   // exact int32 block sum
    return (float)si * (vxm_h2f((uint16_t)o.dw) * o.xs);
}

// Makes every operand of a group live at one point, so all of the group's LDS
// reads are issued before its first product (the compiler otherwise reuses one
// register set and serialises the units on the LDS latency).
// The activation's operands are left out: a phase whose K is one unit reads
// the same block for every unit, which the compiler loads once.
__device__ __forceinline__ void ops_ready(UnitOps &o) {
    asm volatile("" : "+v"(o.w0), "+v"(o.w1), "+v"(o.dw));
}

// Sums of four values over the 64 lanes, transposed: one permlane32 swap per
// pair folds lanes 32..63 onto 0..31 for two values at once, one permlane16
// swap folds the result to a 16-lane row per value, and a row sum ends the
// total in lane 15 of row r: v[0], v[2], v[1], v[3] for r = 0, 1, 2, 3.
// 10 instructions for four values; a 64-lane DPP sum takes 6 (and two
// broadcasts across rows) per value.
__device__ __forceinline__ float wave_sum4_rows(const float (&v)[4]) {
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[0]), __float_as_uint(v[1]), false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[2]), __float_as_uint(v[3]), false, false);
    const float r01 = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const float r23 = __uint_as_float(b[0]) + __uint_as_float(b[1]);
    const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(r01), __float_as_uint(r23), false, false);
    return row16_sum_15(__uint_as_float(c[0]) + __uint_as_float(c[1]));
}

// Consume slots OFF + G .. OFF + G + 3 (at most K - G of them) of one phase:
// wait until they are in LDS, read every operand of the group, form the four
// units' terms, and reduce them together (wave_sum4_rows); partials to
// part[u].  The ring's waits count loads: at phase start every slot of the
// phase is in flight or landed, and the only ring loads issued after slot k's
// are those of the next P - 1 - k stream positions, 3 instructions each, so
// vmcnt(3 (P - G - n)) means slots G .. G + n - 1 are in LDS.  (Other vector
// memory instructions of the wave are issued later and only make the wait
// stricter.)  No loads are issued here: the refills of the phase's slots go
// out after its outputs are published (ring_refill), while the workgroup
// waits for the next phase's inputs.  All 7 compute waves issuing DMAs at
// once saturate the CU's address unit, and a wave's load issue blocks until
// it is accepted, so refills issued between units stalled the compute by
// about as long as the compute itself.
// X: of the P - K stream positions after the phase's slots that are in flight at its
// start, the last X were issued by the reader wave (ring_refill_readers), not by this
// wave, and do not count in its vmcnt.
template <class S, int OFF, int K, int G = 0, int X = 0>
__device__ __forceinline__ void ring_phase(const int8_t *ring, int l, int ci, int lane, const int8_t *xq,
                                           const float *xd, float *part) {
    static_assert(K <= S::P, "a phase's slots are all in the ring at its start");
    static_assert(X <= S::P - K, "positions after the phase");
    if constexpr (G < K) {
        constexpr int n = K - G < 4 ? K - G : 4;
        ring_wait<3 * (S::P - G - n - X)>();
        UnitOps o[4];
        o[0] = unit_load<S, OFF + G>(ring, l, ci, lane, xq, xd);
        if constexpr (n > 1) o[1] = unit_load<S, OFF + G + 1>(ring, l, ci, lane, xq, xd);
        if constexpr (n > 2) o[2] = unit_load<S, OFF + G + 2>(ring, l, ci, lane, xq, xd);
        if constexpr (n > 3) o[3] = unit_load<S, OFF + G + 3>(ring, l, ci, lane, xq, xd);
#pragma unroll
        for (int i = 0; i < n; i++) ops_ready(o[i]);
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < n; i++) v[i] = unit_term(o[i]);
        const float tot = wave_sum4_rows(v);
        if ((lane & 15) == 15) {
            const int r = lane >> 4;
            const int i = r == 1 ? 2 : r == 2 ? 1 : r;   // rows hold v[0], v[2], v[1], v[3]
            int u = -1;
            if (i < n) u = ci + kCW * (Slot<S, OFF + G>::k + i);
            // units past the phase's (or a wave's dummy units) are not stored
            if (u >= 0 && u < Slot<S, OFF + G>::U) part[u] = tot;
        }
        ring_phase<S, OFF, K, G + 4, X>(ring, l, ci, lane, xq, xd, part);
    }
}

// Refill the K slots of the phase at OFF with the units P positions ahead
// (in the next layer's weights past the end of the schedule).
template <class S, int OFF, int K, int k = 0>
__device__ __forceinline__ void ring_refill(const vxm_pparams &p, const UnitBases &cur, const UnitBases &nxt,
                                            uint32_t ring_lds, int l, int wg, int ci, int lane) {
    if constexpr (k < K) {
        constexpr int s = OFF + k, sn = (s + S::P) % S::NS;
        constexpr bool wrap = s + S::P >= S::NS;
        ring_issue<S, sn>(p, wrap ? nxt : cur, ring_lds, l + (wrap ? 1 : 0), wg, ci, lane);
        ring_refill<S, OFF, K, k + 1>(p, cur, nxt, ring_lds, l, wg, ci, lane);
    }
}

// The same refills, slots OFF + K0 .. OFF + K - 1, for every compute wave's ring,
// issued by a reader wave (ring0 = the LDS address of compute wave 0's ring).  Units
// a wave does not own are skipped: no compute wave counts these loads.  The reader
// wave's later loads (its share of the next exchange reads) retire after them, so by
// the time it passes the barrier that follows its next exchange read they are in LDS.
template <class S, int OFF, int K0, int K, int k = K0>
__device__ __forceinline__ void ring_refill_slots(const vxm_pparams &p, const UnitBases &cur, const UnitBases &nxt,
                                                  uint32_t ring_ci, int l, int wg, int ci, int lane) {
    if constexpr (k < K) {
        constexpr int s = OFF + k, sn = (s + S::P) % S::NS;
        constexpr bool wrap = s + S::P >= S::NS;
        const int8_t *q;
        const uint16_t *d;
        bool live;
        unit_addr<S, sn>(p, wrap ? nxt : cur, wg, ci, q, d, live);
        if (live) dma_unit(ring_ci + ring_slot<S, sn>(l + (wrap ? 1 : 0)) * kSlot, q, d, lane, true);
        ring_refill_slots<S, OFF, K0, K, k + 1>(p, cur, nxt, ring_ci, l, wg, ci, lane);
    }
}

template <class S, int OFF, int K0, int K>
__device__ __forceinline__ void ring_refill_readers(const vxm_pparams &p, const UnitBases &cur, const UnitBases &nxt,
                                                    uint32_t ring0, int l, int wg, int lane) {
    // (the profiling build keeps this loop rolled: unrolled, its timestamps' registers
    // made it spill here, and each spill reload waited for the DMAs before it)
#ifdef VXM_PERSISTENT_TRACE
#pragma unroll 1
#endif
    for (int ci = 0; ci < kCW; ci++)
        ring_refill_slots<S, OFF, K0, K>(p, cur, nxt, ring0 + ci * (S::RING * kSlot), l, wg, ci, lane);
}

// Rows of one attention batch into registers.  K: lane (kin, sub) of wave w
// loads dims sub*16 .. +16 (two 16-byte loads) of key jb + (k * kWaves + w) * 8
// + kin, k < KBK: eight lanes per key, so a score is 8 v_dot2 and three DPP
// steps.  V: dims sub*8 .. +8 (one load) of key jb + (k * kWaves + w) * 4 + kin,
// k < KB, sixteen lanes per key.  Keys at or past lim (the current token, which
// comes from LDS, or the chunk's end) load nothing.
template <int KBK, int HD>
__device__ __forceinline__ void attn_load_k(const uint16_t *base, int jb, int lim, uint4 (&r)[KBK][2]) {
    static_assert(HD == 128, "eight lanes of 16 dims per key");
    const int tid = tid_now(), wave = tid >> 6, lane = tid & 63, sub = lane & 7, kin = lane >> 3;
#pragma unroll
    for (int k = 0; k < KBK; k++) {
        const int j = jb + (k * kWaves + wave) * 8 + kin;
        const uint4 *src = (const uint4 *)(base + (int64_t)j * HD + sub * 16);
        r[k][0] = j < lim ? src[0] : make_uint4(0, 0, 0, 0);
        r[k][1] = j < lim ? src[1] : make_uint4(0, 0, 0, 0);
    }
}
template <int KB, int HD>
__device__ __forceinline__ void attn_load(const uint16_t *base, int jb, int lim, uint4 (&r)[KB]) {
    constexpr int LPK = HD / 8, KPW = 64 / LPK;
    const int tid = tid_now(), wave = tid >> 6, lane = tid & 63, sub = lane % LPK, kin = lane / LPK;
#pragma unroll
    for (int k = 0; k < KB; k++) {
        const int j = jb + (k * kWaves + wave) * KPW + kin;
        r[k] = j < lim ? *(const uint4 *)(base + (int64_t)j * HD + sub * 8) : make_uint4(0, 0, 0, 0);
    }
}

// the sum over each aligned group of 8 lanes, the same bits in all 8 (each step
// adds the same two values in either order)
__device__ __forceinline__ float sum8_all(float v) {
    v = v + dpp_f<kDppXor1>(v);
    v = v + dpp_f<kDppXor2>(v);
    return v + dpp_f<kDppMirror8>(v);
}

// q . k for eight lanes of 16 dims: v_dot2_f32_f16 on f16 pairs (the BF16-valued q
// and the f16 cache are exact in f16, the products exact in f32; only the
// summation order differs from a sequential fp32 dot product)
__device__ __forceinline__ float score8(const half2_t (&q2)[8], const uint4 (&kr)[2]) {
    const uint32_t w[8] = {kr[0].x, kr[0].y, kr[0].z, kr[0].w, kr[1].x, kr[1].y, kr[1].z, kr[1].w};
    float pt = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) pt = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w[i]), q2[i], pt, false);
    return sum8_all(pt);
}

// Attention of query head h for layer l (vcpm_attention's gqa_group_attn,
// src/minicpm4.c:232-248).  The cached K and V rows [0, pos) do not depend
// on this layer's projections, so every wave issues its loads of the first
// batch (up to 320 keys) before wave 0 reads q_h, k_g, v_g: the cache fetch
// overlaps the QKV exchange.  The current token's k, v come from LDS; the
// group's first head appends them to the cache.  Output: 128 fp32.
//
// Softmax in three barriers: the scores (scaled) go to LDS with each wave's
// max, the exponentials replace them with each wave's double sum, and P.V
// multiplies each exponential by (float)(1 / sum) as it reads it -- the
// normalised p of the reference, formed where it is used.  The current key (row
// pos) is the last key of its lanes in both loops, so its score and its P.V
// term are added after the loops, from LDS, in the same order.
//
// With p.att_split = S > 1 (long contexts) this workgroup takes chunk c of
// the keys, [c CH, (c + 1) CH) with CH = ceil((pos + 1) / S): a softmax
// within the chunk, its normalised output o_c, max m_c and exp sum l_c.
// Chunks c > 0 publish (o_c, m_c, l_c); chunk 0 gathers them and combines in
// chunk order, o = sum_c w_c o_c / sum_c w_c with w_c = l_c exp(m_c - m),
// m = max_c m_c (the softmax over all keys, regrouped).  With S = 1 this is
// the unsplit attention, unchanged.
template <class S>
__device__ __forceinline__ void attention_phase(const vxm_pparams &p, int l, int h, int chunk, float *lds,
                                                int *bail, uint32_t ep) {
    constexpr int QD = S::QD, KVD = S::KVD, HD = S::HD;
    constexpr int SQ = rep_stride(S::NQKV / 2), SAT = rep_stride(QD);
    constexpr int LPK = HD / 8, KPW = 64 / LPK;                  // V: lanes per key, keys per wave
    constexpr int KB = 10;                                       // V: keys per lane per batch
    constexpr int PERB = kWaves * KPW * KB;                      // keys per batch (320)
    constexpr int KBK = 5;                                       // K: keys per lane per batch
    static_assert(kWaves * 8 * KBK == PERB, "K and V batches cover the same keys");
    const int tid = tid_now(), wave = tid >> 6, lane = tid & 63;
    const int rp = blockIdx.x % kRep, g = h / S::QPK, pos = p.pos;
    vxm_ptab Ly = layer_at(p, l);
    float *aq = lds + S::L_AQ, *red = lds + S::L_RED, *sc = lds + S::L_BIG;   // scores: BIG is free in phase B
    float *wmax = lds + S::L_PART;                      // unit partials are free in phase B
    double *wsum = (double *)(lds + S::L_PART + 8);
    uint16_t *const kc = Ly->kc, *const vc = Ly->vc;
    const uint16_t *kb = kc + (int64_t)g * p.cap * HD;
    const uint16_t *vb = vc + (int64_t)g * p.cap * HD;
    const int kv_len = pos + 1, nsplit = p.att_split;
    const int chl = (kv_len + nsplit - 1) / nsplit;
    const int j0 = chunk * chl, j1 = min(kv_len, j0 + chl), lim = min(j1, pos);
    uint4 kr[KBK][2], vr[KB];
    attn_load_k<KBK, HD>(kb, j0, lim, kr);
    attn_load<KB, HD>(vb, j0, lim, vr);
    if (wave == 0) {
        // q_h and k_g (pair-interleaved: word w = dims w, w + HD/2) and v_g
        // (natural pairs) -> aq[0..3HD) in natural order; lane l owns word w = l
        // of each of the three parts
        const uint64_t *qkvb = p.qkvb + rp * SQ;
        const uint64_t *src[3] = {qkvb + h * (HD / 2), qkvb + (QD + g * HD) / 2, qkvb + (QD + KVD + g * HD) / 2};
        const uint32_t tag = make_tag(ep, l, PH_QKV);
        uint32_t pending = 7;
        int it = 0;
        while (true) {
            uint64_t w[3];
#pragma unroll
            for (int k = 0; k < 3; k++)
                if (pending & (1u << k)) w[k] = get_word(src[k] + lane);
#pragma unroll
            for (int k = 0; k < 3; k++) {
                if ((pending & (1u << k)) && (uint32_t)(w[k] >> 32) == tag) {
                    const uint32_t v = (uint32_t)w[k];
                    const float a = __uint_as_float(v << 16), b = __uint_as_float(v & 0xffff0000u);
                    float *dst = aq + k * HD;
                    if (k < 2) {
                        dst[lane] = a;
                        dst[lane + HD / 2] = b;
                    } else {
                        *(float2 *)(dst + 2 * lane) = make_float2(a, b);
                    }
                    pending &= ~(1u << k);
                }
            }
            if (__all(pending == 0)) break;
            if (give_up(p, it, bail)) break;
            __builtin_amdgcn_s_sleep(1);
        }
    }
    lds_barrier();
    if (*bail) return;
    VXM_TS(tid_now() == 0, 3);
    const float *qh = aq, *kcur = aq + HD, *vcur = aq + 2 * HD;
    // KV append: the first query head of each group writes the f16 rows at pos
    if (h % S::QPK == 0 && chunk == 0) {
        uint16_t *kw = kc + ((int64_t)g * p.cap + pos) * HD;
        uint16_t *vw = vc + ((int64_t)g * p.cap + pos) * HD;
        for (int d = tid; d < HD; d += kThreads) {
            kw[d] = vxm_f2h(kcur[d]);
            vw[d] = vxm_f2h(vcur[d]);
        }
    }
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn((float)HD));
    const bool has_pos = pos >= j0 && pos < j1;   // the last chunk holds the current key
    // ---- scores: lane (kin8, sub8) holds q dims sub8*16 .. +16 as f16 pairs ----
    const int sub8 = lane & 7, kin8 = lane >> 3;
    half2_t q2[8];
#pragma unroll
    for (int i = 0; i < 8; i++) q2[i] = half2_t{(_Float16)qh[sub8 * 16 + 2 * i], (_Float16)qh[sub8 * 16 + 2 * i + 1]};
    float mx = -INFINITY;
    for (int jb = j0; jb < j1; jb += PERB) {
        if (jb > j0) attn_load_k<KBK, HD>(kb, jb, lim, kr);
#pragma unroll
        for (int k = 0; k < KBK; k++) {
            const int j = jb + (k * kWaves + wave) * 8 + kin8;
            const float s2 = score8(q2, kr[k]) * scale;
            if (j < lim) {
                if (sub8 == 0) sc[j - j0] = s2;
                mx = fmaxf(mx, s2);
            }
        }
    }
    if (has_pos) {
        // the current key from LDS, on the lanes whose key it is (the last key of those lanes)
        const int d = pos - j0, rel = d % PERB, wp = (rel / 8) % kWaves, kp = rel % 8;
        if (wave == wp && kin8 == kp) {
            uint4 kq[2];
            uint32_t *kw = (uint32_t *)kq;
#pragma unroll
            for (int i = 0; i < 8; i++)
                kw[i] = (uint32_t)vxm_f2h(kcur[sub8 * 16 + 2 * i]) | ((uint32_t)vxm_f2h(kcur[sub8 * 16 + 2 * i + 1]) << 16);
            const float s2 = score8(q2, kq) * scale;
            if (sub8 == 0) sc[d] = s2;
            mx = fmaxf(mx, s2);
        }
    }
    VXM_TS(tid_now() == 0, 2);
    mx = wave_max_63(mx);
    if (lane == 63) wmax[wave] = mx;
    lds_barrier();   // scores and wave maxima in LDS
    mx = wmax[0];
#pragma unroll
    for (int w = 1; w < kWaves; w++) mx = fmaxf(mx, wmax[w]);
    double sum = 0.0;
    for (int j = tid; j < j1 - j0; j += kThreads) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        sum += (double)e;
    }
    sum = wave_sum_63_d(sum);
    if (lane == 63) wsum[wave] = sum;
    lds_barrier();   // exponentials and wave sums in LDS
    sum = 0.0;
#pragma unroll
    for (int w = 0; w < kWaves; w++) sum += wsum[w];
    const float inv = (float)(1.0 / sum);
    VXM_TS(tid_now() == 0, 11);
    // out[d] = sum_j p_j v_j[d], p_j = e_j * inv: lane (kin, sub) accumulates dims sub*8..+8 over its keys
    const int sub = lane % LPK, kin = lane / LPK;
    float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int jb = j0; jb < j1; jb += PERB) {
        if (jb > j0) attn_load<KB, HD>(vb, jb, lim, vr);
#pragma unroll
        for (int k = 0; k < KB; k++) {
            const int j = jb + (k * kWaves + wave) * KPW + kin;
            if (j >= lim) continue;
            const float pj = sc[j - j0] * inv;
            // one mixed-precision fma per value: the f16 operand is widened exactly
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t wv = i == 0 ? vr[k].x : i == 1 ? vr[k].y : i == 2 ? vr[k].z : vr[k].w;
                const half2_t v2 = __builtin_bit_cast(half2_t, wv);
                o[2 * i] = __builtin_fmaf(pj, (float)v2.x, o[2 * i]);
                o[2 * i + 1] = __builtin_fmaf(pj, (float)v2.y, o[2 * i + 1]);
            }
        }
    }
    if (has_pos) {
        const int d = pos - j0, rel = d % PERB, wp = (rel / KPW) % kWaves, kp = rel % KPW;
        if (wave == wp && kin == kp) {
            const float pj = sc[d] * inv;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float vf = (float)__builtin_bit_cast(_Float16, vxm_f2h(vcur[sub * 8 + i]));
                o[i] = __builtin_fmaf(pj, vf, o[i]);
            }
        }
    }
    // reduce over the KPW = 4 key rows of the wave (lanes l, l^16, l^32,
    // l^48) with permlane swaps, then over waves in a fixed order
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(o[i]), __float_as_uint(o[i]), false, false);
        o[i] = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
        const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(o[i]), __float_as_uint(o[i]), false, false);
        o[i] = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
    }
    if (kin == 0) {
        *(float4 *)(red + wave * HD + sub * 8) = make_float4(o[0], o[1], o[2], o[3]);
        *(float4 *)(red + wave * HD + sub * 8 + 4) = make_float4(o[4], o[5], o[6], o[7]);
    }
    lds_barrier();   // the wave partials in LDS
    const uint32_t tg = make_tag(ep, l, PH_ATT);
    static_assert(HD % 32 == 0 && HD / 4 <= 64, "one wave quantizes a head");
    if (nsplit == 1) {
        // wave 0: lane i < HD / 4 adds the wave partials of dims 4i .. 4i + 3 in wave
        // order, quantizes them (Q8_0, the O projection's input rule) and publishes:
        // word h HD/4 + i holds the quants of dims 4i .. 4i + 3 of head h, word
        // NH HD/4 + h HD/32 + b the scale of its block b -- a quarter of the words
        // of fp32 outputs, so each of the 256 readers of phase C loads a quarter
        // of the bytes
        if (wave == 0) {
            const int i = lane % (HD / 4);   // lanes past HD / 4 repeat the first ones
            float4 a = *(const float4 *)(red + 4 * i);
#pragma unroll
            for (int w = 1; w < kWaves; w++) {
                const float4 b = *(const float4 *)(red + w * HD + 4 * i);
                a.x = a.x + b.x; a.y = a.y + b.y; a.z = a.z + b.z; a.w = a.w + b.w;
            }
            const float q4[4] = {a.x, a.y, a.z, a.w};
            uint32_t w;
            float dsc;
            quant4_reg(q4, w, dsc);
            if (lane < HD / 4) {
#pragma unroll
                for (int r = 0; r < kRep; r++) {
                    put_word(p.attb + r * SAT + h * (HD / 4) + i, w, tg);
                    if ((i & 7) == 0) put_word(p.attb + r * SAT + S::NH * (HD / 4) + h * (HD / 32) + i / 8, __float_as_uint(dsc), tg);
                }
            }
        }
        VXM_TS(tid_now() == 0, 4);
        return;
    }
    // key chunks: thread t owns dim t % HD; the wave partials are summed once, in a fixed order
    const int d = tid % HD;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) v += red[w * HD + d];
    {
        constexpr int CW = HD + 2;   // o[HD], m, l of one chunk in LDS
        const uint32_t tp = make_tag(ep, l, PH_ATTP);
        uint64_t *mine = p.attp + ((int64_t)h * kAttSplitMax + chunk) * kAttpWords;
        if (chunk > 0) {
            if (tid < HD) put_word(mine + d, __float_as_uint(v), tp);
            else if (tid == HD) put_word(mine + HD, __float_as_uint(mx), tp);
            else if (tid == HD + 1) put_word(mine + HD + 1, __float_as_uint((float)sum), tp);
            VXM_TS(tid_now() == 0, 4);
            return;
        }
        // chunk 0: its own (o, m, l) at sc[0..CW), the other chunks' words to sc[CW c ..]
        // (the scores are dead: every P.V read of sc precedes the barrier above)
        if (tid < HD) sc[d] = v;
        else if (tid == HD) sc[HD] = mx;
        else if (tid == HD + 1) sc[HD + 1] = (float)sum;
        const int nw = (nsplit - 1) * CW;
        constexpr int NPT = cdiv((kAttSplitMax - 1) * CW, kThreads);
        const uint64_t *base = p.attp + (int64_t)h * kAttSplitMax * kAttpWords;
        uint32_t pend = 0;
#pragma unroll
        for (int k = 0; k < NPT; k++)
            if (tid + k * kThreads < nw) pend |= 1u << k;
        int it = 0;
        while (true) {
            uint64_t w[NPT];
#pragma unroll
            for (int k = 0; k < NPT; k++) {
                const int i = tid + k * kThreads;
                if (pend & (1u << k)) w[k] = get_word(base + (int64_t)(1 + i / CW) * kAttpWords + i % CW);
            }
#pragma unroll
            for (int k = 0; k < NPT; k++) {
                if ((pend & (1u << k)) && (uint32_t)(w[k] >> 32) == tp) {
                    sc[CW + tid + k * kThreads] = __uint_as_float((uint32_t)w[k]);
                    pend &= ~(1u << k);
                }
            }
            if (__all(pend == 0)) break;
            if (give_up(p, it, bail)) break;
            __builtin_amdgcn_s_sleep(1);
        }
        lds_barrier();
        if (*bail) return;
        float m = -INFINITY;
        for (int c = 0; c < nsplit; c++) m = fmaxf(m, sc[c * CW + HD]);
        double num = 0.0, den = 0.0;
        for (int c = 0; c < nsplit; c++) {
            const double wc = (double)sc[c * CW + HD + 1] * (double)expf(sc[c * CW + HD] - m);
            den += wc;
            num += wc * (double)sc[c * CW + d];
        }
        v = (float)(num / den);
        // every wave's reads of the gathered partials end before any wave moves on:
        // the next phase's input lands in the same LDS
        lds_barrier();
    }
    // Q8_0 of the merged head output (quant4 over aligned 32-value blocks) and the
    // publication, as in the unsplit case; aq's q, k, v are dead here
    if (tid < HD) aq[tid] = v;
    lds_barrier();
    if (wave == 0) {
        const int i = lane % (HD / 4);
        const float4 a = *(const float4 *)(aq + 4 * i);
        const float q4[4] = {a.x, a.y, a.z, a.w};
        uint32_t w;
        float dsc;
        quant4_reg(q4, w, dsc);
        if (lane < HD / 4) {
#pragma unroll
            for (int r = 0; r < kRep; r++) {
                put_word(p.attb + r * SAT + h * (HD / 4) + i, w, tg);
                if ((i & 7) == 0) put_word(p.attb + r * SAT + S::NH * (HD / 4) + h * (HD / 32) + i / 8, __float_as_uint(dsc), tg);
            }
        }
    }
    VXM_TS(tid_now() == 0, 4);
}

// The whole decode.  The inputs of each phase are read by the waves named by
// k*Readers (each forming its share of RMSNorm's sum of squares on the way);
// waves 1..7 also stream weights and publish the outputs.  All waves walk
// the same phase schedule and barrier sequence.
template <class S>
__device__ __forceinline__ void decode_run(const vxm_pparams &p, float *lds, int *bail, uint32_t ep) {
    constexpr int H = S::H, QD = S::QD, KVD = S::KVD, HD = S::HD, F = S::F, NH = S::NH;
    constexpr int SX = rep_stride(H / 2), SQ = rep_stride(S::NQKV / 2), SAT = rep_stride(QD), SP = rep_stride(F / 2);
    const int wg = blockIdx.x;
    const int rp = wg % kRep;
    float *xs = lds + S::L_XS, *h1s = lds + S::L_H1, *gn = lds + S::L_GN, *big = lds + S::L_BIG;
    float *xd = lds + S::L_XD, *cs = lds + S::L_CS, *part = lds + S::L_PART, *red = lds + S::L_RED;
    double *ssq = (double *)red;   // sum of squares from the reading wave
    int8_t *xq = (int8_t *)lds + S::XQ_OFF;
    const int wave = tid_now() >> 6, lane = tid_now() & 63;
    const bool reader = wave < kNR;
    const int ci = __builtin_amdgcn_readfirstlane(wave - kNR);   // compute wave index (uniform)
    const int t = tid_now() - 64 * kNR;                         // compute thread index
    const int pos = p.pos;
    // the query head this workgroup attends for, or -1
    int head = -1, chunk = 0;
    for (int h = 0; h < NH; h++)
        for (int c = 0; c < p.att_split; c++)
            if (attn_wg_chunk<S>(h, c) == wg) {
                head = h;
                chunk = c;
            }

    // rope cos/sin of this token's position (ggml_rope_ext NEOX angles, host table)
    if (!p.no_rope) {
        for (int i = tid_now(); i < HD / 2; i += kThreads) {
            const float2 r = p.rope_cs[(int64_t)pos * (HD / 2) + i];
            cs[2 * i] = r.x;
            cs[2 * i + 1] = r.y;
        }
    }

    // this wave's ring slots in LDS (compute waves only)
    const int8_t *ring = (const int8_t *)lds + S::RING_OFF + (reader ? 0 : ci) * S::RING * kSlot;
    const uint32_t ring_lds = (uint32_t)(uintptr_t)ring;
    UnitBases cur = unit_bases(p, 0);
    if (!reader) ring_prime<S>(p, cur, ring_lds, wg, ci, lane, std::make_integer_sequence<int, S::P>{});

    for (int l = 0; l < p.n_layers; l++) {
        vxm_ptab Ly = layer_at(p, l);
        const UnitBases nxt = unit_bases(p, l + 1);
        // ---------------- A: norm + QKV + rope ----------------
        static_assert((H / 2) % (128 * kXReaders) == 0 && H / 2 / kXReaders <= 64 * 64, "x readers");
        if (wave == 0) stage_f32(Ly->g_in, H, gn);
        if (wave < kXReaders) {
            // waves 0 .. kXReaders-1 each read a share of x (and its sum of squares)
            constexpr int XW = H / 2 / kXReaders;   // words per reading wave
            double ss = 0.0;
            if (l == 0) {
                if (wave == 0) {
                    for (int i = lane * 4; i < H; i += 256) {
                        const float4 v = *(const float4 *)(p.x + i);
                        *(float4 *)(xs + i) = v;
                        ss += (double)(v.x * v.x) + (double)(v.y * v.y) + (double)(v.z * v.z) + (double)(v.w * v.w);
                    }
                }
            } else {
                ss = read_words<cdiv(XW / 2, 64), true>(p, p.xb + ((l & 1) * kRep + rp) * SX + wave * XW, XW / 2,
                                                        make_tag(ep, l, PH_X), xs + 2 * wave * XW, bail);
            }
            ss = wave_sum_63_d(ss);
            if (lane == 63) ssq[wave] = ss;
        }
        lds_barrier();
        if (*bail) return;
        VXM_TS(tid_now() == 0, 0);
        if (p.dump && wg == 0)
            for (int i = tid_now() * 4; i < H; i += kThreads * 4)
                *(float4 *)(p.dump + (size_t)l * H + i) = *(const float4 *)(xs + i);
        {
            double sst = 0.0;
#pragma unroll
            for (int w = 0; w < kXReaders; w++) sst += ssq[w];
            norm_quant<H>(xs, gn, sst, p.eps, xq, xd);
        }
        lds_barrier();
        VXM_TS(tid_now() == 0, 12);
        if (!reader) ring_phase<S, S::OA, S::SA>(ring, l, ci, lane, xq, xd, part);
        lds_barrier();
        VXM_TS(tid_now() == 0, 1);
        if (!reader && t < S::RA / 2 * kRep) {
            // RA/2 output words x kRep replicas, one store per thread
            const int wi = t / kRep, r = t % kRep;
            const int gw = wg * (S::RA / 2) + wi;        // global word = row pair
            float y[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                float a = 0.0f;
#pragma unroll
                for (int c = 0; c < S::CA; c++) a += part[(2 * wi + j) * S::CA + c];
                y[j] = bf16r(a);
            }
            float y0 = y[0], y1 = y[1];
            if (2 * gw < QD + KVD && !p.no_rope) {
                const int i = gw % (HD / 2);
                const float c = cs[2 * i], s = cs[2 * i + 1];
                y0 = bf16r(y[0] * c - y[1] * s);
                y1 = bf16r(y[0] * s + y[1] * c);
            }
            put_word(p.qkvb + r * SQ + gw, pack_bf16x2(y0, y1), make_tag(ep, l, PH_QKV));
        }
        // A's refills (the layer's D units 4 and 5, needed about 8 us later).  In an attention
        // workgroup they go out after the attention: issued first, the K / V row loads of
        // every wave retired behind them (loads retire in order).  593 -> 579 us per token.
        // (The same deferral of E's refills, to after the next layer's A, measured 601 and
        // 624 us: those loads then sit in front of the attention's and phase C's reads.)
        if (!reader && head < 0) ring_refill<S, S::OA, S::SA>(p, cur, nxt, ring_lds, l, wg, ci, lane);
        // ---------------- B: attention, one workgroup per query head ----------------
        if (head >= 0) {
            attention_phase<S>(p, l, head, chunk, lds, bail, ep);
            if (*bail) return;
            if (!reader) ring_refill<S, S::OA, S::SA>(p, cur, nxt, ring_lds, l, wg, ci, lane);
        }
        // ---------------- C: O rows + residual ----------------
        if (wave < kAttReaders) {
            // waves 0 .. kAttReaders-1 each read a share of the Q8_0 attention output
            // (quants and scales straight into xq / xd); their rounds of loads are in
            // flight together
            const uint64_t *src = p.attb + rp * SAT;
            const uint32_t tag = make_tag(ep, l, PH_ATT);
            constexpr int NQW = NH * (HD / 4), NW = NQW + NH * (HD / 32), AP = cdiv(NW / 2, kAttReaders);
            static_assert(NW % 2 == 0 && NQW % 2 == 0 && AP <= 64 * 32, "attention channel shares");
            wait_sentinels(p, src, NH, HD / 4, tag, bail);
            const int p0 = wave * AP;
            if (!*bail) read_q8_words<cdiv(AP, 64)>(p, src, p0, min(AP, NW / 2 - p0), NQW, tag, xq, xd, bail);
        }
        lds_barrier();
        if (*bail) return;
        VXM_TS(tid_now() == 0, 5);
        if (!reader) ring_phase<S, S::OC, S::SC>(ring, l, ci, lane, xq, xd, part);
        lds_barrier();
        VXM_TS(tid_now() == 0, 6);
        if (!reader && t < S::RC / 2 * kRep) {
            const int wi = t / kRep, r = t % kRep;
            const int row = wg * S::RC + 2 * wi;
            float hh[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                float a = 0.0f;
#pragma unroll
                for (int c = 0; c < S::CC; c++) a += part[(2 * wi + j) * S::CC + c];
                float o = bf16r(a);
                if (p.res_scale != 1.0f) o = o * p.res_scale;
                hh[j] = bf16r(xs[row + j] + o);
            }
            put_word(p.h1b + r * SX + row / 2, pack_bf16x2(hh[0], hh[1]), make_tag(ep, l, PH_H1));
        }
        if (!reader) ring_refill<S, S::OC, S::SC>(p, cur, nxt, ring_lds, l, wg, ci, lane);
        // ---------------- D: post norm + gate/up + SwiGLU ----------------
        if (wave == 0) stage_f32(Ly->g_post, H, gn);
        if (wave < kH1Readers) {
            constexpr int HW = H / 2 / kH1Readers;   // words per reading wave
            static_assert(HW % 128 == 0 && HW / 128 <= 32, "h1 readers");
            double ss = read_words<HW / 128, true>(p, p.h1b + rp * SX + wave * HW, HW / 2, make_tag(ep, l, PH_H1),
                                                   h1s + 2 * wave * HW, bail);
            ss = wave_sum_63_d(ss);
            if (lane == 63) ssq[wave] = ss;
        }
        lds_barrier();
        if (*bail) return;
        VXM_TS(tid_now() == 0, 7);
        {
            double sst = 0.0;
#pragma unroll
            for (int w = 0; w < kH1Readers; w++) sst += ssq[w];
            norm_quant<H>(h1s, gn, sst, p.eps, xq, xd);
        }
        lds_barrier();
        VXM_TS(tid_now() == 0, 13);
        if (!reader) ring_phase<S, S::OD, S::SD>(ring, l, ci, lane, xq, xd, part);
        lds_barrier();
        VXM_TS(tid_now() == 0, 8);
        if (!reader && t < S::RD / 4 * kRep) {
            const int wi = t / kRep, r = t % kRep;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                float a = 0.0f;
#pragma unroll
                for (int c = 0; c < S::CD; c++) a += part[(4 * wi + j) * S::CD + c];
                v[j] = a;
            }
            const float p0 = swiglu(v[0], v[1]), p1 = swiglu(v[2], v[3]);
            put_word(p.pb + r * SP + wg * (S::RD / 4) + wi, pack_bf16x2(p0, p1), make_tag(ep, l, PH_P));
        }
        // D's refills in two parts.  The units of E (the positions before the
        // layer's end) go out now; the next layer's A / C units only after the
        // p read below, which would otherwise retire behind them in each reading
        // wave: 667 -> 649 us per token.  Holding back more measured slower (the
        // units then arrive late for their phase): E's refills after the next
        // layer's x read 709, the part of them that lands on D 684, C's refills
        // after the h1 read 700.
        constexpr int kDE = S::NS - S::OD - S::P > 0 ? S::NS - S::OD - S::P : 0;
        if (!reader) ring_refill<S, S::OD, kDE>(p, cur, nxt, ring_lds, l, wg, ci, lane);
        // ---------------- E: down rows + residual ----------------
        if (wave < kPReaders) {
            // waves 0 .. kPReaders-1 each read a share of p
            constexpr int QW = F / 2 / kPReaders;
            static_assert(QW % 128 == 0 && QW / 128 <= 32, "p channel shares");
            const uint32_t tag = make_tag(ep, l, PH_P);
            read_words<QW / 128, true, true>(p, p.pb + rp * SP + wave * QW, QW / 2, tag, big + wave * QW, bail);
        }
        lds_barrier();
        if (*bail) return;
        VXM_TS(tid_now() == 0, 9);
        if (!kD2Reader && !reader) ring_refill<S, S::OD, S::SD, kDE>(p, cur, nxt, ring_lds, l, wg, ci, lane);
        VXM_TS(tid_now() == 0, 15);
        quantize_lds_bf16x2((const uint32_t *)big, F, xq, xd);
        lds_barrier();
        VXM_TS(tid_now() == 0, 14);
        // The rest of D's refills (the next layer's first A / C units) go out from the
        // reader wave while the compute waves form E's units: issued by the compute
        // waves before the Q8_0 of p, they held it (and the units) back by about as long
        // as the address unit took to accept them.
        if (!reader) ring_phase<S, S::OE, S::SE, 0, kD2Reader ? S::SD - kDE : 0>(ring, l, ci, lane, xq, xd, part);
        else if (kD2Reader) ring_refill_readers<S, S::OD, kDE, S::SD>(p, cur, nxt, ring_lds, l, wg, lane);
        lds_barrier();
        VXM_TS(tid_now() == 0, 10);
        if (!reader && t < S::RE / 2 * kRep) {
            const int wi = t / kRep, r = t % kRep;
            const int row = wg * S::RE + 2 * wi;
            float x2[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                float a = 0.0f;
#pragma unroll
                for (int c = 0; c < S::CE; c++) a += part[(2 * wi + j) * S::CE + c];
                float d = bf16r(a);
                if (p.res_scale != 1.0f) d = d * p.res_scale;
                x2[j] = bf16r(h1s[row + j] + d);
            }
            put_word(p.xb + (((l + 1) & 1) * kRep + r) * SX + row / 2, pack_bf16x2(x2[0], x2[1]),
                     make_tag(ep, l + 1, PH_X));
        }
        if (!reader) ring_refill<S, S::OE, S::SE>(p, cur, nxt, ring_lds, l, wg, ci, lane);
        cur = nxt;
    }
    // ---------------- final norm (workgroup 0) ----------------
    if (wg != 0) return;
    const int Lyr = p.n_layers;
    if (wave == 0) {
        if (p.final_norm) stage_f32(p.final_norm, H, gn);
        read_words<cdiv(H / 4, 64), true>(p, p.xb + ((Lyr & 1) * kRep + rp) * SX, H / 4, make_tag(ep, Lyr, PH_X), xs,
                                          bail);
    }
    lds_barrier();
    if (*bail) return;
#ifdef VXM_PERSISTENT_TRACE
    if (tid_now() == 0 && p.trace) p.trace[1] = __builtin_amdgcn_s_memrealtime();
#endif
    if (p.dump)
        for (int i = tid_now() * 4; i < H; i += kThreads * 4)
            *(float4 *)(p.dump + (size_t)Lyr * H + i) = *(const float4 *)(xs + i);
    if (p.final_norm) {
        rmsnorm_lds(xs, gn, H, p.eps, big, red);
        for (int i = tid_now(); i < H; i += kThreads) p.x[i] = big[i];
    } else {
        for (int i = tid_now(); i < H; i += kThreads) p.x[i] = xs[i];
    }
}

}  // namespace

// The tag epoch of a launch lives in device memory: every workgroup reads it at
// start, and the last workgroup to finish advances it.  A launch recorded into a
// HIP graph therefore tags its words anew on every replay.  Tags hold 20 bits
// of it; when it wraps (every 1,048,575 launches, about 10 minutes of decode at
// 575 us per token), that last workgroup first resets every channel word to
// all-ones, so no word written before the wrap (for instance a key-chunk
// partial of a head split that later launches did not repeat) can carry a live
// tag again.
constexpr uint32_t kEpochMask = 0xfffffu;

template <class S>
__global__ __launch_bounds__(kThreads, 1) void k_decode_persistent(vxm_pparams p) {
    // All of the workgroup's LDS is this one dynamic array, so it starts at
    // address 0 and every 16-byte layout offset is 16-byte aligned.  (A static
    // __shared__ variable beside it would place the dynamic array right after
    // the static bytes, at only 4-byte alignment: every ds_read_b128 of the
    // ring and the activations would then be split by the LDS.)  The bail and
    // last-workgroup flags live past the layout, at byte S::BYTES.
    extern __shared__ __attribute__((aligned(16))) float lds[];
    int *bail = (int *)((char *)lds + S::BYTES);
    int *last = bail + 1;
    if (threadIdx.x == 0) *bail = 0;
#ifdef VXM_PERSISTENT_TRACE
    if (threadIdx.x == 0 && p.trace) p.trace[(size_t)blockIdx.x * p.trace_stride] = __builtin_amdgcn_s_memrealtime();
#endif
    // a scalar load: the previous launch's last workgroup wrote it before that launch ended
    const uint32_t ep = __builtin_amdgcn_readfirstlane(*(const volatile uint32_t *)p.state);
    // bail is read only after the first barrier of decode_run
    decode_run<S>(p, lds, bail, ep);
    // every ring load of the wave (the refills past the last layer, or those in
    // flight when a wait gave up) lands before the workgroup ends
    ring_wait<0>();
    lds_barrier();
    if (threadIdx.x == 0) {
        const uint32_t done = __hip_atomic_fetch_add(p.state + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last = done == kG - 1;
    }
    lds_barrier();
    if (!*last) return;
    // the last workgroup: every other workgroup has read the epoch and finished
    // with the channels
    uint32_t next = (ep + 1u) & kEpochMask;
    if (next == 0) {
        next = 1;
        for (uint64_t i = threadIdx.x; i < p.n_chan; i += kThreads)
            __hip_atomic_store(p.xb + i, ~0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lds_barrier();
    }
    if (threadIdx.x == 0) {
        __hip_atomic_store(p.state + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p.err, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // the live word
        __hip_atomic_store(p.state, next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
using ShapeTslm = Shape<2048, 16, 2, 128, 6144>;

struct vxm_persistent_state {
    void *base = nullptr;
    vxm_player *layers = nullptr;
    uint64_t *xb = nullptr, *qkvb = nullptr, *attb = nullptr, *h1b = nullptr, *pb = nullptr, *attp = nullptr;
    int8_t *dummy_q = nullptr;
    uint16_t *dummy_d = nullptr;
    int *err = nullptr;         // [0] live, [1] sticky
    uint32_t *state = nullptr;  // [0] epoch, [1] arrivals
    uint64_t n_chan = 0;        // channel words (xb .. attp)
    // the cache whose K/V pointers are in the layer table: its unique id, base
    // and capacity (a freed cache's struct address can come back for a new one)
    uint64_t kv_id = 0;
    const void *kv_base = nullptr;
    int kv_cap = 0;
};

static constexpr int kMaxLds = 160 * 1024;

// Every workgroup of the decode waits on words the others publish, so all 256
// must be resident at once: one per CU, since the LDS layout takes more than
// half of a CU's 160 KB.  A plain launch of 256 workgroups places them all on
// a device whose other work finishes on its own.  hipLaunchCooperativeKernel
// guarantees it, but measured 19 us more per token (649 against 630).  Other
// work on the device can only delay the waits, and every wait is bounded
// (kSpin rounds, then the error word): an error, never a hang.  Eager launches
// are ordered after the device's previous single-launch kernel
// (vxm_ordered_launch_begin), so two of them on different streams never
// interleave their workgroups.
template <class S>
static int launch_decode(vxm_ctx *ctx, const vxm_pparams &prm) {
    const int lds = S::BYTES + 16;   // the layout + the bail and last-workgroup flags
    auto kern = k_decode_persistent<S>;
    if (lds > kMaxLds)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "persistent decode: kv capacity %d needs %d B of LDS", prm.cap, lds);
    VXM_HIP(ctx, hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
    vxm_launch_slot *slot = nullptr;
    bool capturing = false;
    int rc = vxm_ordered_launch_begin(ctx, &slot, &capturing);
    if (rc) return rc;
    hipLaunchKernelGGL(kern, dim3(kG), dim3(kThreads), (unsigned)lds, ctx->stream, prm);
    const hipError_t le = hipGetLastError();
    rc = vxm_ordered_launch_end(ctx, slot, capturing);
    if (le != hipSuccess) return vxm_fail(ctx, VXM_ERR_BACKEND, "persistent decode launch failed: %s", hipGetErrorString(le));
    return rc;
}

// Supported shapes: (hidden, heads, kv heads, head dim, ffn).
static bool persistent_shape(const vxm_block_dims &d, int n_cu) {
    if (n_cu != kG) return false;
    if (d.H == 2048 && d.nh == 16 && d.nkv == 2 && d.hd == 128 && d.F == 6144) return true;
    return false;
}

// Largest cache capacity: kAttSplitMax key chunks whose scores each fit the LDS.
int vxm_persistent_max_cap(const vxm_block_dims &d) {
    (void)d;
    return ShapeTslm::MAX_CAP;
}

// Key chunks per head for kv_len keys.  One workgroup per head up to
// kAttSplitFrom keys; beyond, about kAttChunk keys per chunk, never more than
// kAttSplitMax chunks, each at most BIG keys and none empty.  The merge costs
// one more exchange, which pays once a workgroup's key stream is longer:
// measured over the 28-layer stack, splitting 256-320 keys in chunks of 64-192
// took 759-771 us per token against 746 unsplit, while at 512 keys two chunks
// took 777 us against 851 and at 1024 keys four took 789 against 860.
#ifndef VXM_ATT_SPLIT_FROM
#define VXM_ATT_SPLIT_FROM 384
#endif
#ifndef VXM_ATT_CHUNK
#define VXM_ATT_CHUNK 256
#endif
constexpr int kAttSplitFrom = VXM_ATT_SPLIT_FROM;
constexpr int kAttChunk = VXM_ATT_CHUNK;
template <class S>
static int att_split_for(int kv_len) {
    if (kv_len <= kAttSplitFrom) return 1;
    int n = (kv_len + kAttChunk - 1) / kAttChunk;
    if (n > kAttSplitMax) n = kAttSplitMax;
    while (n < kAttSplitMax && (kv_len + n - 1) / n > S::BIG) n++;
    return n;
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

int vxm_persistent_decode(vxm_minicpm4 *m, vxm_kv_cache *kv, float *x, int32_t pos, float *dump) {
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
    hipStreamCaptureStatus cap_st = hipStreamCaptureStatusNone;
    VXM_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cap_st));
    const bool capturing = cap_st != hipStreamCaptureStatusNone;
    if (capturing && (!s.base || s.kv_id != kv->id || s.kv_base != kv->base || s.kv_cap != kv->cap))
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG,
                        "persistent decode: its buffers and layer table are set up by an eager call; run one "
                        "decode on this model and cache before capturing");
    if (!s.base) {
        const size_t tab = ((size_t)L * sizeof(vxm_player) + 255) & ~(size_t)255;
        const int nx = rep_stride((int)d.H / 2), nq = rep_stride((int)(qd + 2 * kvd) / 2),
                  na = rep_stride((int)qd), np_ = rep_stride((int)d.F / 2);
        const size_t words = (size_t)kRep * (2 * nx + nq + na + nx + np_) + (size_t)d.nh * kAttSplitMax * kAttpWords;
        const size_t dummy = kUnit + 256;
        const size_t total = tab + words * 8 + dummy + 256 + 64;
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
        s.attp = (uint64_t *)b; b += (size_t)d.nh * kAttSplitMax * kAttpWords * 8;
        s.dummy_q = (int8_t *)b; b += kUnit;
        s.dummy_d = (uint16_t *)b; b += 256;
        s.err = (int *)b;
        s.state = (uint32_t *)(b + 64);
        s.n_chan = words;
        // tags start as all-ones: never equal to a live (epoch >= 1) tag; the first launch has epoch 1
        const uint32_t st0[2] = {1u, 0u};
        VXM_HIP(ctx, hipMemsetAsync((char *)s.base + tab, 0xff, words * 8, ctx->stream));
        VXM_HIP(ctx, hipMemsetAsync(s.dummy_q, 0, dummy + 256 + 64, ctx->stream));
        VXM_HIP(ctx, hipMemcpyAsync(s.state, st0, sizeof st0, hipMemcpyHostToDevice, ctx->stream));
        VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        s.kv_id = 0;
    }
    if (s.kv_id != kv->id || s.kv_base != kv->base || s.kv_cap != kv->cap) {
        std::vector<vxm_player> tabh(L);
        for (int l = 0; l < L; l++) {
            const vxm_block &b = m->blocks[l];
            tabh[l] = vxm_player{b.wqkv->qs, b.wo->qs, b.wgu->qs, b.wd->qs, b.wqkv->d, b.wo->d, b.wgu->d,
                                 b.wd->d, b.g_in, b.g_post, kv->k(l), kv->v(l)};
        }
        VXM_HIP(ctx, hipMemcpyAsync(s.layers, tabh.data(), L * sizeof(vxm_player), hipMemcpyHostToDevice,
                                    ctx->stream));
        VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        s.kv_id = kv->id;
        s.kv_base = kv->base;
        s.kv_cap = kv->cap;
    }
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
    prm.attp = s.attp;
    prm.att_split = att_split_for<ShapeTslm>(pos + 1);
    {
        const int n = prm.att_split, chl = (pos + 1 + n - 1) / n;
        if (chl > ShapeTslm::BIG || (n - 1) * chl >= pos + 1)
            return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "persistent decode: %d keys do not split into %d chunks", pos + 1, n);
    }
    prm.dummy_q = s.dummy_q;
    prm.dummy_d = s.dummy_d;
    prm.err = s.err;
    prm.state = s.state;
    prm.n_chan = s.n_chan;
    prm.dump = dump;
    prm.rope_cs = d.rope_cs;
    prm.eps = d.eps;
    prm.res_scale = d.res_scale;
    prm.pos = pos;
    prm.cap = kv->cap;
    prm.no_rope = d.no_rope;
#ifdef VXM_PERSISTENT_TRACE
    // profiling builds: one trace buffer per process, dumped after every launch
    static uint64_t *tbuf = nullptr;
    static size_t tcap = 0;
    static int ncall = 0;
    const int stride = 2 + L * kTraceSlots;
    const size_t tbytes = (size_t)kG * stride * 8;
    if (tbytes > tcap) {
        VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        if (tbuf) VXM_HIP(ctx, hipFree(tbuf));
        VXM_HIP(ctx, hipMalloc(&tbuf, tbytes));
        tcap = tbytes;
    }
    VXM_HIP(ctx, hipMemsetAsync(tbuf, 0, tbytes, ctx->stream));
    prm.trace = tbuf;
    prm.trace_stride = stride;
    int rc_ = launch_decode<ShapeTslm>(ctx, prm);
    if (rc_) return rc_;
    std::vector<uint64_t> th((size_t)kG * stride);
    VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    VXM_HIP(ctx, hipMemcpy(th.data(), tbuf, tbytes, hipMemcpyDeviceToHost));
    const char *dir = getenv("VXM_TRACE_DIR");
    char fn[512];
    snprintf(fn, sizeof fn, "%s/trace_L%d_%04d.bin", dir ? dir : ".", L, ncall++);
    if (FILE *f = fopen(fn, "wb")) {
        fwrite(th.data(), 8, th.size(), f);
        fclose(f);
    }
    return VXM_OK;
#else
    return launch_decode<ShapeTslm>(ctx, prm);
#endif
}

int vxm_persistent_check(vxm_minicpm4 *m) {
    if (!m->pstate || !m->pstate->err) return VXM_OK;
    int e = 0;
    VXM_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    VXM_HIP(m->ctx, hipMemcpy(&e, m->pstate->err + 1, 4, hipMemcpyDeviceToHost));
    if (e) {
        VXM_HIP(m->ctx, hipMemset(m->pstate->err + 1, 0, 4));
        return vxm_fail(m->ctx, VXM_ERR_BACKEND, "persistent decode: a workgroup timed out waiting for data");
    }
    return VXM_OK;
}

// Test hook: the tag epoch of the next launch (1 .. 2^20 - 1), and the current one.
int vxm_persistent_set_epoch(vxm_minicpm4 *m, uint32_t epoch) {
    if (!m->pstate || !m->pstate->state)
        return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "decode epoch: no single-launch decode has run on this model");
    if (epoch == 0 || epoch > kEpochMask)
        return vxm_fail(m->ctx, VXM_ERR_INVALID_ARG, "decode epoch %u outside 1 .. %u", epoch, kEpochMask);
    VXM_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    VXM_HIP(m->ctx, hipMemcpy(m->pstate->state, &epoch, 4, hipMemcpyHostToDevice));
    return VXM_OK;
}

int vxm_persistent_get_epoch(vxm_minicpm4 *m, uint32_t *epoch) {
    *epoch = 0;
    if (!m->pstate || !m->pstate->state) return VXM_OK;
    VXM_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    VXM_HIP(m->ctx, hipMemcpy(epoch, m->pstate->state, 4, hipMemcpyDeviceToHost));
    return VXM_OK;
}
