// locdit_persistent.hip -- every block of one LocDiT (or LocEnc) evaluation
// in a single launch on gfx950: the M <= 48 rows of both CFG branches through
// the blocks of vcpm_locdit_forward (src/locdit.c:300-372) / the encoder
// (src/locenc.c:86-116), each block the non-causal MiniCPM4 block of
// vcpm_minicpm4_block (src/minicpm4.c:467-532).
//
// Launch-based, a block is seven dependent kernels of a few microseconds each,
// every one of them latency-bound (the weights of a whole evaluation stream in
// 27 us at 8 TB/s).  Here 256 workgroups, one per CU, stay resident for all
// blocks and hand each phase's output to the next phase's workgroups through
// tagged 64-bit words (32-bit tag, 32-bit payload; written with agent-scope
// relaxed atomic stores, read in pairs with 16-byte loads that bypass the
// non-coherent caches as agent-scope atomic loads do): a word is valid exactly
// when its tag is the expected one, so no fences or grid barriers are needed.
// Per block:
//
//   N1  row owners (one workgroup per row): x += the down projection's K-split
//       partials of the previous block; RMSNorm(g_in) -> Q8_0 rows
//   QKV 16-column tiles of W_qkv over all rows: MFMA, BF16, NEOX RoPE of the
//       pair-interleaved q/k rows, f16 rounding of K and V -> BF16 pairs
//   ATT one (head, segment, 8 query rows) per workgroup: softmax attention of
//       vcpm_attention (src/minicpm4.c:232-248) -> Q8_0 of its head's columns
//   O   (16-column tile, quarter of K) units: partial products
//   N2  row owners: x += O; RMSNorm(g_post) -> Q8_0 rows
//   GU  64-row tiles of the interleaved gate/up weight: MFMA, SwiGLU
//       (src/minicpm4.c:441-456), Q8_0 of its 32 outputs
//   D   (32-column tile, eighth of K) units: partial products
//
// The rounding steps are those of the launch-based kernels (k_rmsnorm,
// k_attention_local, k_swiglu_quant); the fp32 summation order of the matrix
// products differs (blocks of K per wave, waves added in order), the attention
// scores at head dim 128 add eight runs of 16 dims, and P.V sums the keys in
// order (the oracle's attend_one).
//
// Every workgroup knows its weight tiles for all phases in advance, so wave 7
// streams them into LDS with global_load_lds_dwordx4 one or more phases ahead
// (its waits never delay the exchange reads of waves 0-6).  Weight tiles and
// staged activations share one LDS layout per 32-byte Q8_0 block: 512 bytes
// holding the 8-byte piece q of row r at 16 (16 (q >> 1) + r) + 8 (q & 1), which
// is where lane (q, r) of v_mfma_i32_16x16x32_i8 reads it (conflict-free).
#include <cstdio>
#include <cstdlib>

#include "vxm_model.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8, kThreads = kWaves * 64, kG = 256;
constexpr int kPollThreads = 7 * 64;   // waves 0-6 read exchanged words; wave 7 streams weights
constexpr int kSpin = 1 << 17;         // poll rounds before giving up
constexpr int kMaxM = 48, kMT = 3, kMP = 48, kMaxS = 32, kRB = 8;
constexpr int kMaxQT = 3;   // QKV column tiles per workgroup
// A CFM solve in one launch: at most kMaxEval Euler steps of x [P][kFeat], P * kFeat <= kSolveMaxN
constexpr int kMaxEval = 64, kFeat = 64, kSolveMaxN = 2048;
constexpr int kXqWords = kFeat / 4 + kFeat / 32;   // words per row of the Q8_0 x channel
constexpr int kH = 1024, kF = 4096, kNH = 16;
constexpr int kXPitch = kH / 4 + kH / 32;   // words per row of a norm output (quants, then scales)
constexpr int kPPitch = kF / 4 + kF / 32;   // words per row of the SwiGLU output
constexpr int kOSplits = 4, kDSplits = 8, kDChunk = kF / kDSplits;
enum { PH_X1, PH_QKV, PH_ATT, PH_O, PH_X2, PH_P, PH_D };

template <int NKV_, int HD_>
struct LShape {
    static constexpr int NKV = NKV_, HD = HD_, HALF = HD / 2;
    static constexpr int QD = kNH * HD, KVD = NKV * HD, NQKV = QD + 2 * KVD;
    static constexpr int UQ = NQKV / 16;                  // QKV units
    static constexpr int KO = QD / kOSplits, BO = KO / 32;  // O units: K bytes / blocks per split
    static constexpr int APitch = QD / 4 + QD / 32;         // words per row of the attention output
    // exchange channels, words (allocated for kMaxM rows)
    static constexpr int WX = kMaxM * kXPitch, WQKV = kMaxM * NQKV / 2, WA = kMaxM * APitch;
    static constexpr int WOP = kOSplits * kMaxM * kH, WP = kMaxM * kPPitch, WDP = kDSplits * kMaxM * kH;
    // LDS layout (bytes; every region 1 KiB aligned)
    static constexpr int RA = 0;                              // QKV (16 rows) / gate-up (64 rows) tile
    static constexpr int RA_SC = RA + 64 * kH;                // its scales, f16 [rows][32]
    static constexpr int RO = RA_SC + 64 * 32 * 2;            // O tile: 16 rows x KO
    static constexpr int RO_SC = RO + 16 * KO;                // f16 [16][BO]
    static constexpr int RD = RO_SC + 1024;                   // down tile: 32 rows x 512
    static constexpr int RD_SC = RD + 32 * kDChunk;           // f16 [32][16]
    static constexpr int ST = RD_SC + 1024;                   // staged activations [3][32 blocks][512]
    static constexpr int ST_SC = ST + kMT * 32 * 512;         // their scales, f32 [32][kMP]
    static constexpr int XR = ST_SC + 32 * kMP * 4;           // a row owner's x, f32 [1024]
    static constexpr int GN = XR + kH * 4;                    // a row owner's norm gain, f32 [1024]
    static constexpr int MISC = GN + kH * 4;                  // 8 doubles of reductions, then flags
    static constexpr int BYTES = MISC + 128;
    static_assert(16 * BO * 2 <= 1024, "O scales");
    static_assert(UQ <= kMaxQT * ((kG - kMaxM) / kMT) && kMaxQT * 16 * kH <= RA_SC - RA && kMaxQT * 1024 <= RO - RA_SC,
                  "QKV tiles of a workgroup");
    static_assert(kMP * 33 * 4 <= MISC - XR, "gate/up outputs in the row-owner area");
    static_assert(kWaves * 2 * kMT * 64 * 16 <= ST_SC - ST, "gate/up partial sums in the stage");
    static_assert(BYTES <= 160 * 1024, "LDS");
    // attention scratch inside the stage: k (rotated, f16-rounded) [S][HD+4], v [S][HD],
    // q [kRB][HD+4], out [kRB][HD], p [kRB][S+1], row max and 1/sum [kRB] each
    static_assert((kMaxS * (HD + 4) + kMaxS * HD + kRB * (HD + 4) + kRB * HD + kRB * (kMaxS + 1) + 2 * kRB) * 4 <=
                      ST_SC - ST + 32 * kMP * 4,
                  "attention scratch");
};

struct vxm_lblock {
    const int8_t *qkv_q, *o_q, *gu_q, *dn_q;
    const uint16_t *qkv_d, *o_d, *gu_d, *dn_d;
    const float *g_in, *g_post;
};

struct vxm_lparams {
    const vxm_lblock *blocks;
    int L, M, S, nseg, qb;   // blocks, rows, rows per segment, segments, query blocks per (head, segment)
    float eps;
    int variant;
    const float2 *cs;        // rope (cos, sin) [position][HD/2]
    float *x;                // [M][1024]: block 0's input in, the last block's output out
    uint64_t *x1, *qkv, *att, *op, *x2, *pp, *dp;   // exchange channels
    // [0] live: set by a workgroup that gave up waiting, polled by the others, cleared
    // at the end of the launch by its last workgroup (so one failed launch never makes
    // later ones give up); [1] sticky: also set, read and cleared by the check calls
    int *err;
    uint32_t *state;         // [0] epoch, [1] workgroups finished in this launch
    float *dump;             // debug: [L + 1][M][1024] rows entering each block, then the output; or null
    // the final RMSNorm of rows fin_r0 .. S - 1 of each segment (gain fin_g, or none: null)
    // as Q8_0 rows fin_q / fin_d, segment-major
    const float *fin_g;
    int fin_r0;
    int8_t *fin_q;
    uint16_t *fin_d;
    // solve mode (n_eval > 0): n_eval Euler steps of vxm_cfm_solve in this launch.  Each
    // evaluation starts with the row owners assembling their rows (mu, the step's time
    // row tc, the cond rows ch + cb, the x rows' in_proj), runs the L blocks, and ends
    // with the x rows' final norm (fin_g) going to workgroup kG - 1, which forms
    // out_proj, the CFG-Zero* blend and the Euler step of xs, and hands the Q8_0 of the
    // new x to the next evaluation's row owners.
    int n_eval, P, Pc, n_seg, n_mu, use_cfg;
    float cfg;
    const float *tc;                 // [n_eval][1024] time rows
    const float *mu;                 // [2][1024] mu rows of segment 0, or null
    const float *ch, *cb;            // [Pc][1024] raw cond projection, its bias (or null)
    const int8_t *in_q;              // in_proj [1024][kFeat], scales [1024][2], bias (or null)
    const uint16_t *in_d;
    const float *in_b;
    const int8_t *out_q;             // out_proj [kFeat][1024], scales [kFeat][32], bias (or null)
    const uint16_t *out_d;
    const float *out_b;
    float *xs;                       // [P][kFeat] x, updated in place by every step
    const int8_t *xq0;               // its Q8_0 at the start [P][kFeat], scales [P][2]
    const uint16_t *xd0;
    uint64_t *fq, *xqc;              // channels: the final norm's Q8_0 rows, the new x's Q8_0
    float dts[kMaxEval];             // the steps' sizes
    uint64_t *trace;         // profiling build: per workgroup, the start and 16 timestamps per block
};

// slots per block; a solve's blocks are numbered over its evaluations (it = k L + l), and the
// solve's own phases take slots 24-31 (assemble inputs / done, update inputs / done, then inside
// the update: products, out_proj rows, the CFG sums, the Euler step and Q8_0)
constexpr int kTraceSlots = 32;
#ifdef VXM_PERSISTENT_TRACE
#define VXM_LTS(k)                                                                                                 \
    do {                                                                                                           \
        if (threadIdx.x == 0 && p.trace)                                                                           \
            p.trace[(size_t)blockIdx.x * (1 + kTraceSlots * p.L * max(p.n_eval, 1)) + 1 + kTraceSlots * it + (k)] = \
                __builtin_amdgcn_s_memrealtime();                                                                  \
    } while (0)
#else
#define VXM_LTS(k) do { } while (0)
#endif

// Block l's table entry through the constant address space and a read-first-lane
// address, so its fields are scalar (lgkmcnt) loads: a vector load here would make
// wave 7 wait (vmcnt, which retires in order) for every weight prefetch it has in
// flight before it could use the pointers.
typedef const __attribute__((address_space(4))) vxm_lblock *vxm_lbtab;
__device__ __forceinline__ vxm_lblock block_at(const vxm_lparams &p, int l) {
    const uint64_t a = (uint64_t)(uintptr_t)(p.blocks + l);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    const vxm_lbtab t = (vxm_lbtab)(uintptr_t)(((uint64_t)hi << 32) | lo);
    return vxm_lblock{t->qkv_q, t->o_q, t->gu_q, t->dn_q, t->qkv_d, t->o_d, t->gu_d, t->dn_d, t->g_in, t->g_post};
}

// The tag of (launch epoch, block, phase).  Consecutive writes of a word always carry
// different tags; a word left from an older launch (rows past a later launch's M) could
// only match again after 2^31 / (8 L) launches, 22 million at 12 blocks.
__device__ __forceinline__ uint32_t make_tag(uint32_t ep, int L, int l, int ph) {
    return ((ep * (uint32_t)(8 * L) + (uint32_t)(8 * l + ph)) << 1) | 1u;   // odd: never a zeroed word
}

__device__ __forceinline__ void put_word(uint64_t *dst, uint32_t payload, uint32_t tag) {
    __hip_atomic_store(dst, ((uint64_t)tag << 32) | (uint64_t)payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t get_word(const uint64_t *src) {
    return __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float bf16r(float f) { return (float)(__bf16)f; }

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xffff0000u);
}

// Workgroup barrier ordering LDS only: the weight loads of wave 7 stay in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ bool give_up(const vxm_lparams &p, int &it, int *bail) {
    if (++it > kSpin || ((it & 31) == 0 && __hip_atomic_load(p.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
        __hip_atomic_store(p.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p.err + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *bail = 1;
        return true;
    }
    return false;
}

constexpr int kVmcnt0 = 0x0F70;   // s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15)

__device__ __forceinline__ int opaque_tid() {
    int v;
    asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "v"((int)threadIdx.x));
    return v;
}

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// A channel of exchanged words as a buffer resource (reads past `bytes` return zeros).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t chan_rsrc(const uint64_t *chan, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)chan, (short)0, (int)bytes, 0x00020000);
}

// Waves 0-6: thread t polls items t, t + 448, ... (< n, at most NPT per thread).  Item i
// is the aligned pair of words at byte offset off(i) of channel rs, read with one
// 16-byte load that bypasses the non-coherent caches like an agent-scope atomic load
// (sc1; each 8-byte word is written by one atomic store, so each half is whole);
// sink(i, a, b) stores the two payloads once both words carry `tag`.  The 16-byte
// loads halve the address work of 8-byte ones, which sets the rate at which a CU
// reads the words of a phase.
template <int NPT, class A, class K>
__device__ __forceinline__ void poll(const vxm_lparams &p, __amdgpu_buffer_rsrc_t rs, int n, uint32_t tag, A off,
                                     K sink, int *bail) {
    static_assert(NPT <= 32, "items per thread");
    uint32_t pending = 0;
    const int t0 = opaque_tid();
#pragma unroll
    for (int k = 0; k < NPT; k++)
        if (t0 + kPollThreads * k < n) pending |= 1u << k;
    int it = 0;
    while (true) {
        // the thread index through an opaque move: the items' offsets are recomputed
        // in every round instead of being hoisted out of the block loop and held in
        // registers across all phases
        const int t = opaque_tid();
        v4u w[NPT];
#pragma unroll
        for (int k = 0; k < NPT; k++)
            if (pending & (1u << k)) w[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, off(t + kPollThreads * k), 0, 16);
#pragma unroll
        for (int k = 0; k < NPT; k++)
            if ((pending & (1u << k)) && w[k].y == tag && w[k].w == tag) {
                sink(t + kPollThreads * k, w[k].x, w[k].z);
                pending &= ~(1u << k);
            }
        if (__all(pending == 0)) break;
        if (give_up(p, it, bail)) break;
        __builtin_amdgcn_s_sleep(1);
    }
    // vmcnt(0) as the compiler's own wait: its wait insertion then knows that no load of
    // this wave is outstanding, and inserts none after the phases' joins -- where wave 7
    // would otherwise wait for its weight prefetches too
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
}

__device__ __forceinline__ int slot_of(int q, int r) { return 16 * (16 * (q >> 1) + r) + 8 * (q & 1); }

// Rows [r0, r0 + M) x blocks [kb0, kb0 + nb) of a Q8_0 channel (row pitch `pitch` words:
// qwords quant words, then one scale word per block; pitch, qwords, kb0 and nb even)
// into the stage as rows 0 .. M - 1: quants in the block-slot layout [row tile][block][512],
// scales f32 [block][kMP].  A pair of quant words is one 8-byte piece of a block.
template <int NPT>
__device__ __forceinline__ void poll_stage(const vxm_lparams &p, __amdgpu_buffer_rsrc_t rs, int pitch, int qwords,
                                           int kb0, int nb, int r0, int M, uint32_t tag, uint8_t *lds, int st,
                                           int st_sc, int *bail) {
    const int per = 4 * nb + nb / 2;   // pairs per row
    poll<NPT>(
        p, rs, M * per, tag,
        [&](int i) {
            const int m = i / per, j = i - m * per;
            return ((r0 + m) * pitch + (j < 4 * nb ? 8 * kb0 + 2 * j : qwords + kb0 + 2 * (j - 4 * nb))) * 8;
        },
        [&](int i, uint32_t a, uint32_t b) {
            const int m = i / per, j = i - m * per;
            if (j < 4 * nb) {
                const int blk = j >> 2, q = j & 3;
                *(uint64_t *)(lds + st + ((m >> 4) * nb + blk) * 512 + slot_of(q, m & 15)) =
                    (uint64_t)a | ((uint64_t)b << 32);
            } else {
                const int k = 2 * (j - 4 * nb);
                *(float *)(lds + st_sc + (k * kMP + m) * 4) = __uint_as_float(a);
                *(float *)(lds + st_sc + ((k + 1) * kMP + m) * 4) = __uint_as_float(b);
            }
        },
        bail);
}

// Row owner: the ns partial rows [s][M][1024] of row `row` into the stage as f32 [ns][1024].
template <int NPT>
__device__ __forceinline__ void poll_partials(const vxm_lparams &p, __amdgpu_buffer_rsrc_t rs, int ns, int M, int row,
                                              uint32_t tag, uint8_t *lds, int st, int *bail) {
    poll<NPT>(
        p, rs, ns * (kH / 2), tag, [&](int i) { return (((i >> 9) * M + row) * kH + 2 * (i & 511)) * 8; },
        [&](int i, uint32_t a, uint32_t b) {
            *(float2 *)(lds + st + ((i >> 9) * kH + 2 * (i & 511)) * 4) = make_float2(__uint_as_float(a), __uint_as_float(b));
        },
        bail);
}

// Lane l loads 16 bytes at g into LDS at lds_addr + 16 l (lanes outside mask load
// nothing).  Called by wave 7 with all lanes active.
__device__ __forceinline__ void dma16(uint32_t lds_addr, const void *g, uint64_t mask) {
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_addr);
    uint64_t saved;
    uint32_t saved_m0;
    asm volatile(
        "s_mov_b32 %1, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_mov_b64 %0, exec\n\t"
        "s_and_b64 exec, exec, %4\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %3, off\n\t"
        "s_mov_b64 exec, %0\n\t"
        "s_mov_b32 m0, %1"
        : "=&s"(saved), "=&s"(saved_m0)
        : "s"(m0v), "v"(g), "s"(mask)
        : "memory", "scc");
}

template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// 16 weight rows [n0, n0 + 16) x blocks [kb0, kb0 + nb) (nb even) of a weight with
// K bytes per row, as tile c of a region at `wt`: nb / 2 instructions, each two
// blocks of the 16 rows.
__device__ __forceinline__ void dma_tile(int wt, int c, const int8_t *wq, int K, int n0, int kb0, int nb, int lane) {
    const int e = lane >> 5, j = (lane >> 4) & 1, r = lane & 15;
    const int8_t *g = wq + (size_t)(n0 + r) * K + (kb0 + e) * 32 + 16 * j;
    for (int k = 0; k < nb / 2; k++) dma16(wt + (c * (nb / 2) + k) * 1024, g + 64 * k, ~0ull);
}

// Scales of rows [n0, n0 + nrows) x blocks [kb0, kb0 + nb) (nb % 8 == 0): f16 [nrows][nb]
// at `wsc`; ceil(nrows * nb / 512) instructions.
__device__ __forceinline__ void dma_scales(int wsc, const uint16_t *wd, int nbk, int n0, int nrows, int kb0, int nb,
                                           int lane) {
    const int per = nb / 8, total = nrows * per;
    for (int k0 = 0; k0 < total; k0 += 64) {
        const int cnt = min(64, total - k0);
        const int i = k0 + min(lane, cnt - 1);
        const int row = i / per, part = i - row * per;
        dma16(wsc + 16 * k0, wd + (size_t)(n0 + row) * nbk + kb0 + 8 * part, cnt == 64 ? ~0ull : ((1ull << cnt) - 1));
    }
}

typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

// The scale products d_w * d_x of a 16 x 16 int32 block product go to the matrix core
// as well: v_mfma_f32_16x16x4_4b_f16 forms four 16 x 16 outer products at once (lane
// 16 k + i supplies element i of block k's two vectors, as fp16 bits in k-slot 0 with
// the other slots zero; block k's result sits in registers 4 k .. 4 k + 3 in the layout
// of the int8 product's result).  A product of two fp16 values has at most 22
// significant bits, so each is the exact fp32 value d_w * d_x that a VALU multiply of
// the converted scales gives (subnormal scales included), and the VALU is left with the
// convert and the fma per value and block (3 -> 2 instructions).  The stage's scales are
// kept as fp32 copies of fp16 values, so converting them back is exact.  The fp16 form
// takes a quarter of the matrix-core cycles of v_mfma_f32_16x16x1_4b_f32 on the
// converted scales, which made the gate/up products (mfma_run2) slower when they used it.
__device__ __forceinline__ v16f scale_outer16_f16(uint32_t a, uint32_t b) {
    const v2u av = {a, 0u}, bv = {b, 0u};
    return __builtin_amdgcn_mfma_f32_16x16x4f16(__builtin_bit_cast(v4h, av), __builtin_bit_cast(v4h, bv), v16f{}, 0,
                                                0, 0);
}

// acc[t][v] += products of tile rows 16 c + 4 q + v with stage rows 16 t + r (t < MT)
// over the NB blocks from b0: weight tile (nbw blocks per row) at wt / wsc, stage
// (nbs blocks) at st / st_sc.  MT and NB are compile-time: groups of up to 4 blocks
// unroll, so each group's LDS reads are issued ahead of the products that need them;
// one scale product per row tile covers the group (blocks past NB get zero scales).
template <int MT, int NB, int G = (NB < 4 ? NB : 4)>
__device__ __forceinline__ void mfma_run(const uint8_t *lds, int wt, int wsc, int nbw, int c, int st, int st_sc,
                                         int nbs, int b0, int lane, float (&acc)[MT][4]) {
    static_assert(NB % G == 0 && G <= 4, "block groups");
    const int q = lane >> 4, r = lane & 15, sl = slot_of(q, r);
#pragma unroll 1
    for (int i0 = 0; i0 < NB; i0 += G) {
        // scale products of blocks b0 + i0 + k, k < 4: lane (k = q, i = r) supplies weight
        // row 16 c + r and stage row 16 t + r of block b0 + i0 + q
        const bool sv = q < G;
        const int bs = b0 + i0 + (sv ? q : 0);
        const uint32_t aw = sv ? *(const uint16_t *)(lds + wsc + ((16 * c + r) * nbw + bs) * 2) : 0u;
        v16f sc[MT];
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const uint32_t bxs = sv ? vxm_f2h(*(const float *)(lds + st_sc + (bs * kMP + 16 * t + r) * 4)) : 0u;
            sc[t] = scale_outer16_f16(aw, bxs);
        }
#pragma unroll
        for (int i = 0; i < G; i++) {
            const int b = b0 + i0 + i;
            const long a = *(const long *)(lds + wt + (c * (nbw / 2) + (b >> 1)) * 1024 + (b & 1) * 512 + sl);
            long bx[MT];
#pragma unroll
            for (int t = 0; t < MT; t++) bx[t] = *(const long *)(lds + st + (t * nbs + b) * 512 + sl);
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const v4i cc = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bx[t], v4i{}, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++) acc[t][v] = __builtin_fmaf((float)cc[v], sc[t][4 * i + v], acc[t][v]);
            }
        }
    }
}

// The same for the two tiles c0, c0 + 1 at once: each block's activation pieces and
// scales are read once for both (gate/up: 5 instead of 8 LDS operand reads per block
// pair, the stage being read by every wave).
template <int MT, int NB, int G>
__device__ __forceinline__ void mfma_run2(const uint8_t *lds, int wt, int wsc, int nbw, int c0, int st, int st_sc,
                                          int nbs, int b0, int lane, float (&acc)[2][MT][4]) {
    static_assert(NB % G == 0 && G <= 4, "block groups");
    const int q = lane >> 4, r = lane & 15, sl = slot_of(q, r);
#pragma unroll 1
    for (int i0 = 0; i0 < NB; i0 += G) {
        // every operand of the group first: each block's activation pieces are read once
        // for both tiles; then per tile its scale products (one per row tile, covering the
        // group: lane (k = q, i = r) supplies weight row 16 (c0 + cc) + r and stage row
        // 16 t + r of block b0 + i0 + q) and its products, blocks in order
        const bool sv = q < G;
        const int bs = b0 + i0 + (sv ? q : 0);
        long a[2][G], bx[G][MT];
        uint32_t aw[2], bxs[MT];
#pragma unroll
        for (int cc = 0; cc < 2; cc++) {
            aw[cc] = sv ? *(const uint16_t *)(lds + wsc + ((16 * (c0 + cc) + r) * nbw + bs) * 2) : 0u;
#pragma unroll
            for (int i = 0; i < G; i++) {
                const int b = b0 + i0 + i;
                a[cc][i] = *(const long *)(lds + wt + ((c0 + cc) * (nbw / 2) + (b >> 1)) * 1024 + (b & 1) * 512 + sl);
            }
        }
#pragma unroll
        for (int t = 0; t < MT; t++) {
            bxs[t] = sv ? vxm_f2h(*(const float *)(lds + st_sc + (bs * kMP + 16 * t + r) * 4)) : 0u;
#pragma unroll
            for (int i = 0; i < G; i++) bx[i][t] = *(const long *)(lds + st + (t * nbs + b0 + i0 + i) * 512 + sl);
        }
#pragma unroll
        for (int cc = 0; cc < 2; cc++) {
            v16f sc[MT];
#pragma unroll
            for (int t = 0; t < MT; t++) sc[t] = scale_outer16_f16(aw[cc], bxs[t]);
#pragma unroll
            for (int i = 0; i < G; i++)
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const v4i ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[cc][i], bx[i][t], v4i{}, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        acc[cc][t][v] = __builtin_fmaf((float)ci[v], sc[t][4 * i + v], acc[cc][t][v]);
                }
        }
    }
}

// After mfma_run in every wave: the partial sums go to LDS (the stage, no longer
// read) and out(ct, t, lane) = sum over kk of wave (ct + ncol * kk)'s partial, in kk order.
// (The four sums of a lane are one 16-byte LDS word: one write and one read per row tile.)
template <int MT>
__device__ __forceinline__ void red_store(uint8_t *lds, int st, int wave, int lane, const float (&acc)[MT][4]) {
    float4 *red = (float4 *)(lds + st);
#pragma unroll
    for (int t = 0; t < MT; t++) red[(wave * MT + t) * 64 + lane] = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
}

template <int MT>
__device__ __forceinline__ void red_sum(const uint8_t *lds, int st, int ncol, int ct, int t, int lane, float (&o)[4]) {
    const float4 *red = (const float4 *)(lds + st);
    float4 s = red[(ct * MT + t) * 64 + lane];
    for (int kk = 1; kk < kWaves / ncol; kk++) {
        const float4 a = red[((ct + ncol * kk) * MT + t) * 64 + lane];
        s.x = s.x + a.x;
        s.y = s.y + a.y;
        s.z = s.z + a.z;
        s.w = s.w + a.w;
    }
    o[0] = s.x;
    o[1] = s.y;
    o[2] = s.z;
    o[3] = s.w;
}

// Q8_0 rule of quant_block_4lanes for one value: x86 = id 127/amax, round half even;
// otherwise id = 1/d, round half away.
__device__ __forceinline__ uint32_t q8_byte(float v, float id, int variant) {
    float q = variant == VXM_QUANT_X86 ? rintf(v * id) : roundf(v * id);
    q = fminf(fmaxf(q, -128.0f), 127.0f);
    return (uint32_t)(uint8_t)(int8_t)(int)q;
}

__device__ __forceinline__ void q8_scale(float amax, int variant, float &d, float &id) {
    d = __fdiv_rn(amax, 127.0f);
    if (variant == VXM_QUANT_X86) id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    else id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
}

// Cross-lane steps on DPP (a few cycles) instead of ds_bpermute (an LDS round trip
// each): quad_perm [1,0,3,2] and [2,3,0,1] (xor 1, xor 2), row_half_mirror (lane i of
// 8 <- 7 - i) and row_mirror (lane i of 16 <- 15 - i).  After xor 1 and xor 2 a quad
// is reduced, after the half mirror 8 lanes, after the mirror a row of 16, and every
// lane holds the same bits (each step adds the same two values in either order).
constexpr int kDppX1 = 0xB1, kDppX2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __uint_as_float(dpp_u<CTRL>(__float_as_uint(v))); }
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint64_t r = (uint64_t)dpp_u<CTRL>((uint32_t)u) | ((uint64_t)dpp_u<CTRL>((uint32_t)(u >> 32)) << 32);
    return __longlong_as_double((long long)r);
}
__device__ __forceinline__ float max4(float v) {
    v = fmaxf(v, dpp_f<kDppX1>(v));
    return fmaxf(v, dpp_f<kDppX2>(v));
}
__device__ __forceinline__ float max16(float v) {
    v = max4(v);
    v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
    return fmaxf(v, dpp_f<kDppMirror>(v));
}
__device__ __forceinline__ float sum8(float v) {
    v = v + dpp_f<kDppX1>(v);
    v = v + dpp_f<kDppX2>(v);
    return v + dpp_f<kDppHalfMirror>(v);
}
__device__ __forceinline__ double sum16_d(double v) {
    v = v + dpp_d<kDppX1>(v);
    v = v + dpp_d<kDppX2>(v);
    v = v + dpp_d<kDppHalfMirror>(v);
    return v + dpp_d<kDppMirror>(v);
}
// the four rows of a wave (all lanes active): row values read back as scalars
__device__ __forceinline__ double rows_sum_d(double v) {
    const long long b = __double_as_longlong(v);
    double t = 0.0;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)b, 16 * r);
        const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)b >> 32), 16 * r);
        t += __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
    }
    return t;
}
__device__ __forceinline__ float rows_max(float v) {
    float m = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
#pragma unroll
    for (int r = 1; r < 4; r++) m = fmaxf(m, __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16 * r)));
    return m;
}

__device__ __forceinline__ double wg_sum_d(double v, uint8_t *lds, int misc) {
    v = rows_sum_d(sum16_d(v));   // the wave's sum (exact: sums of squares of BF16 values)
    double *r = (double *)(lds + misc);
    lds_barrier();
    if ((threadIdx.x & 63) == 0) r[threadIdx.x >> 6] = v;
    lds_barrier();
    double t = 0.0;
    for (int i = 0; i < kWaves; i++) t += r[i];
    return t;
}

// Row owner: x = bf16(x + bf16(sum of ns partial rows, in order)) for row m (the
// partials already in the stage as f32 [ns][1024]); with norm, the RMSNorm of
// k_rmsnorm (gain staged in LDS at gn) and the Q8_0 of its output published as
// row m of chan.
__device__ __forceinline__ void row_update(uint8_t *lds, int st, int xr, int gn, int misc, int ns, float eps,
                                           int variant, uint64_t *chan_row, uint32_t tag, bool norm) {
    const int t = threadIdx.x, c = 2 * t;
    const float *sum = (const float *)(lds + st);
    float *x = (float *)(lds + xr);
    float2 g = make_float2(1.0f, 1.0f);
    if (norm) g = *(const float2 *)(lds + gn + 4 * c);
    float xv[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        float dsum = sum[c + e];
        for (int s = 1; s < ns; s++) dsum = dsum + sum[s * kH + c + e];
        xv[e] = ns ? bf16r(x[c + e] + bf16r(dsum)) : x[c + e];
        x[c + e] = xv[e];
    }
    if (!norm) return;
    const double tot = wg_sum_d((double)(xv[0] * xv[0]) + (double)(xv[1] * xv[1]), lds, (int)misc);
    const float mean = (float)(tot / (double)kH);
    const float sc = __fdiv_rn(1.0f, __fsqrt_rn(mean + eps));
    const float y0 = bf16r(bf16r(xv[0] * sc) * g.x), y1 = bf16r(bf16r(xv[1] * sc) * g.y);
    // Q8_0: 16 threads per 32-value block
    float amax = fmaxf(fabsf(y0), fabsf(y1));
    amax = max16(amax);
    float d, id;
    q8_scale(amax, variant, d, id);
    const uint32_t h = q8_byte(y0, id, variant) | (q8_byte(y1, id, variant) << 8);
    const uint32_t ho = dpp_u<kDppX1>(h);
    if ((t & 1) == 0) put_word(chan_row + t / 2, h | (ho << 16), tag);
    if ((t & 15) == 0) put_word(chan_row + kH / 4 + t / 16, __float_as_uint(vxm_h2f(vxm_f2h(d))), tag);
}

// Row owner, after the last block: the final RMSNorm of its row x (LDS, with the gain
// staged at gn) as plain Q8_0 (k_rmsnorm's steps and Q8_0 rule: what the launch after
// the blocks would compute), q [1024] and d [32] of the output row.
__device__ __forceinline__ void row_final_norm(uint8_t *lds, int xr, int gn, int misc, float eps, int variant,
                                               int8_t *q, uint16_t *dsc) {
    const int t = threadIdx.x, c = 2 * t;
    const float *x = (const float *)(lds + xr);
    const float2 g = *(const float2 *)(lds + gn + 4 * c);
    const float x0 = x[c], x1 = x[c + 1];
    const double tot = wg_sum_d((double)(x0 * x0) + (double)(x1 * x1), lds, misc);
    const float mean = (float)(tot / (double)kH);
    const float sc = __fdiv_rn(1.0f, __fsqrt_rn(mean + eps));
    const float y0 = bf16r(bf16r(x0 * sc) * g.x), y1 = bf16r(bf16r(x1 * sc) * g.y);
    float amax = fmaxf(fabsf(y0), fabsf(y1));
    amax = max16(amax);
    float d, id;
    q8_scale(amax, variant, d, id);
    *(uint16_t *)(q + c) = (uint16_t)(q8_byte(y0, id, variant) | (q8_byte(y1, id, variant) << 8));
    if ((t & 15) == 0) dsc[t / 16] = vxm_f2h(d);
}

// One wave's program for all blocks.  DMA = wave 7: it streams the weight tiles and
// computes with the others, but reads no exchanged words and loads nothing else, so
// its only outstanding vector loads are its prefetches and the compiler, which sees
// none of them, never makes it wait for one.  Waves 0-6 read the exchanged words.
template <class LS, int MT, bool DMA>
__device__ __forceinline__ void run_blocks(const vxm_lparams &p, uint8_t *lds, int *bail, uint32_t ep) {
    const int wg = blockIdx.x, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int M = p.M, S = p.S, L = p.L;
    const int row = wg < M ? wg : -1;
    const int n_att = kNH * p.nseg * p.qb;
    const bool is_att = wg < n_att;
    // QKV units: (16-column tile, row group).  The rows are cut into ngq groups of at most
    // 16 (one MFMA row tile), each read by wpq workgroups; workgroup jq of group gq takes
    // the tiles jq, jq + wpq, ... (at most kMaxQT), so a workgroup reads only its group's
    // activations from the exchange.  Up to 32 rows the row owners (workgroups below M) take
    // none: their norms and the weight loads of QKV units hold each other up (380.5 against
    // 382.7 us per evaluation at 2 x 11 rows; at 2 x 24, 472 against 465 with them excluded).
    const int q0 = M <= 32 ? M : 0;
    const int ngq = (M + 15) / 16, wpq = (kG - q0) / ngq, wq = wg - q0;
    const int gq = wq >= 0 ? wq / wpq : ngq, jq = wq >= 0 ? wq % wpq : 0;
    const int qrows = (M + ngq - 1) / ngq, qr0 = gq * qrows, nrq = min(qrows, M - qr0);
    const int nct = gq < ngq && jq < LS::UQ ? (LS::UQ - 1 - jq) / wpq + 1 : 0;
    const bool is_qkv = nct > 0;
    // gate/up units: (64-row tile, row group): above 16 rows two groups on all 256
    // workgroups, else one group on workgroups 128-255
    const int ngg = M > 16 ? 2 : 1, gu = ngg == 2 ? wg : wg - 128;
    const bool is_gu = gu >= 0;
    const int ugu = gu & 127, grows = (M + ngg - 1) / ngg, gr0 = (gu >> 7) * grows, nrg = min(grows, M - gr0);
    const int oc = wg & 63, os = wg >> 6;   // O unit: 16-column tile, K quarter
    // down unit: 32-column tile dc over K eighth ds (all rows); above 16 rows (drow) a
    // 64-column tile dc2 over K eighth ds2 for the gate/up row groups, its weights in the
    // QKV / gate-up region once the gate/up products are done (the rows of each consumer
    // halved: 55 -> 28 KB of exchanged words at 48 rows)
    const int dc = wg & 31, ds = wg >> 5;
    const bool drow = M > 16;
    const int dc2 = wg & 15, ds2 = (wg >> 4) & 7;
    const int dgrp = wg >> 7, dr0 = dgrp * grows, nrd = min(grows, M - dr0);
    // loads per prefetch (16 rows x 2 blocks, or 64 f16 scale rows of 8 blocks, per instruction)
    constexpr int nO = LS::BO / 2 + 1, nD = 17, nQKV = 17, nGA = 36;
    const int dlane = threadIdx.x & 63;
    // Wave 7 issues each prefetch at the start of a phase's wait, while waves 0-6 poll
    // (an issue costs it ~50 ns per 1 KiB instruction when every CU streams at once).
    // With Q = a QKV role, G = a gate/up role:
    //   start:            O(0) and, with Q, QKV(0) (QKV first without G)
    //   O(l) wait:        D(l); gate/up rows 0-31 (l) with G; QKV(l+1) with Q only
    //   GU(l) wait (G):   gate/up rows 32-63 (l), O(l+1)
    //   D(l) wait:        O(l+1) without G; QKV(l+1) with Q and G
    // The waits before each phase's products count the loads issued after its own.  A
    // workgroup with Q and no G has one QKV tile (one row group: M <= 16), so nQKV loads;
    // with Q and G every wait covers the QKV loads whatever their number (at most
    // nO + kMaxQT nQKV = 60 loads are in flight, below vmcnt's 63).
    static_assert(nO + kMaxQT * nQKV <= 63 && nD + nGA + nO <= 63, "loads in flight");
    auto issue_o = [&](const vxm_lblock &b) {
        dma_tile(LS::RO, 0, b.o_q, LS::QD, 16 * oc, LS::BO * os, LS::BO, dlane);
        dma_scales(LS::RO_SC, b.o_d, LS::QD / 32, 16 * oc, 16, LS::BO * os, LS::BO, dlane);
    };
    auto issue_qkv = [&](const vxm_lblock &b) {
        for (int k = 0; k < kMaxQT; k++) {
            if (k >= nct) break;
            const int n0 = 16 * (jq + k * wpq);
            dma_tile(LS::RA, k, b.qkv_q, kH, n0, 0, 32, dlane);
            dma_scales(LS::RA_SC + 1024 * k, b.qkv_d, kH / 32, n0, 16, 0, 32, dlane);
        }
    };
    auto issue_d = [&](const vxm_lblock &b) {
        for (int c = 0; c < 2; c++) dma_tile(LS::RD, c, b.dn_q, kF, 32 * dc + 16 * c, 16 * ds, 16, dlane);
        dma_scales(LS::RD_SC, b.dn_d, kF / 32, 32 * dc, 32, 16 * ds, 16, dlane);
    };
    auto issue_d2 = [&](const vxm_lblock &b) {   // 34 loads
        for (int c = 0; c < 4; c++) dma_tile(LS::RA, c, b.dn_q, kF, 64 * dc2 + 16 * c, 16 * ds2, 16, dlane);
        dma_scales(LS::RA_SC, b.dn_d, kF / 32, 64 * dc2, 64, 16 * ds2, 16, dlane);
    };
    auto issue_gu_a = [&](const vxm_lblock &b) {
        for (int c = 0; c < 2; c++) dma_tile(LS::RA, c, b.gu_q, kH, 64 * ugu + 16 * c, 0, 32, dlane);
        dma_scales(LS::RA_SC, b.gu_d, kH / 32, 64 * ugu, 64, 0, 32, dlane);
    };
    auto issue_gu_b = [&](const vxm_lblock &b) {
        for (int c = 2; c < 4; c++) dma_tile(LS::RA, c, b.gu_q, kH, 64 * ugu + 16 * c, 0, 32, dlane);
    };
    if (DMA) {
        const vxm_lblock b0 = block_at(p, 0);
        if (is_qkv && !is_gu) {
            issue_qkv(b0);
            issue_o(b0);
        } else {
            issue_o(b0);
            if (is_qkv) issue_qkv(b0);
        }
    }
    // waves 0-6: a norm gain into LDS
    auto stage_gain = [&](const float *g) {
        const int t = opaque_tid();
        for (int c = t * 4; c < kH; c += kPollThreads * 4) *(float4 *)(lds + LS::GN + 4 * c) = *(const float4 *)(g + c);
    };
    float acc[MT][4];
    auto zero_acc = [&]() {
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[t][v] = 0.0f;
    };

    // solve mode: the evaluations' tags are those of n_eval (L + 1) blocks, block l of
    // evaluation k being k (L + 1) + l and k (L + 1) + L its final exchanges
    const bool solve = p.n_eval > 0;
    const int nev = solve ? p.n_eval : 1, LT = solve ? nev * (L + 1) : L;
    const bool upd = solve && wg == kG - 1;   // the workgroup of out_proj and the Euler step
    // out_proj's weights into the region of the QKV / gate-up tiles: tiles 0-1 and the scales
    // at the last down wait of an evaluation, tiles 2-3 at the update's wait
    // (the lane through an opaque move: out_proj's addresses do not change from one
    // evaluation to the next, and hoisted they would hold 72 VGPRs across every phase)
    auto issue_out_a = [&]() {
        const int ol = opaque_tid() & 63;
        for (int c = 0; c < 2; c++) dma_tile(LS::RA, c, p.out_q, kH, 16 * c, 0, 32, ol);
        dma_scales(LS::RA_SC, p.out_d, kH / 32, 0, kFeat, 0, 32, ol);
    };
    auto issue_out_b = [&]() {
        const int ol = opaque_tid() & 63;
        for (int c = 2; c < 4; c++) dma_tile(LS::RA, c, p.out_q, kH, 16 * c, 0, 32, ol);
    };
    static_assert(kFeat == 64 && 4 * 16 * 32 * 2 <= LS::RO - LS::RA_SC, "out_proj tile");
    // one flat loop over (evaluation k, block l): a nested evaluation loop made the compiler
    // hold more values across it (220 against 160 VGPRs)
    for (int it = 0; it < nev * L; it++) {
    const int k = it / L, l = it - k * L;
    auto tagb = [&](int lb, int ph) { return make_tag(ep, LT, solve ? k * (L + 1) + lb : lb, ph); };
    // above 16 rows the QKV tiles of block l share the region with the previous block's down
    // tile, so they go out here (the first block's at the start, the update workgroup's after
    // its out_proj products)
    if (DMA && drow && is_qkv && it > 0 && !(upd && l == 0)) issue_qkv(block_at(p, l));
    // ---- solve mode: the row owners assemble evaluation k's rows (k_locdit_assemble) ----
    if (solve && l == 0 && row >= 0) {
        const int r = row % S, g = row / S, xi = r - 3 - p.Pc;
        int8_t *aq = (int8_t *)(lds + LS::ST);               // the x row's Q8_0: 64 quants,
        uint16_t *ad = (uint16_t *)(lds + LS::ST + kFeat);   // 2 scales
        if (!DMA) {
            const int t = opaque_tid();
            if (xi >= 0 && k == 0) {
                if (t < kFeat / 4) *(uint32_t *)(aq + 4 * t) = *(const uint32_t *)(p.xq0 + (size_t)xi * kFeat + 4 * t);
                if (t < kFeat / 32) ad[t] = p.xd0[(size_t)xi * (kFeat / 32) + t];
            } else if (xi >= 0) {
                // the previous step's Q8_0 of x (its tail exchange: block index -1 of this
                // evaluation): kXqWords words (quants, then fp16 scales) as pairs
                poll<1>(
                    p, chan_rsrc(p.xqc, kMaxS * kXqWords * 8), kXqWords / 2, tagb(-1, PH_X2),
                    [&](int i) { return (xi * kXqWords + 2 * i) * 8; },
                    [&](int i, uint32_t a, uint32_t b) {
                        if (i < kFeat / 8) {
                            *(uint32_t *)(aq + 8 * i) = a;
                            *(uint32_t *)(aq + 8 * i + 4) = b;
                        } else {
                            ad[0] = (uint16_t)a;
                            ad[1] = (uint16_t)b;
                        }
                    },
                    bail);
            } else {
                for (int c = t * 4; c < kH; c += kPollThreads * 4) {
                    float4 v;
                    if (r < 2) {
                        v = g < p.n_mu && p.mu ? *(const float4 *)(p.mu + (size_t)r * kH + c) : make_float4(0, 0, 0, 0);
                    } else if (r == 2) {
                        v = *(const float4 *)(p.tc + (size_t)k * kH + c);
                    } else {
                        v = *(const float4 *)(p.ch + (size_t)(r - 3) * kH + c);
                        if (p.cb) {
                            const float4 b = *(const float4 *)(p.cb + c);
                            v.x = v.x + b.x; v.y = v.y + b.y; v.z = v.z + b.z; v.w = v.w + b.w;
                        }
                        v = make_float4(bf16r(v.x), bf16r(v.y), bf16r(v.z), bf16r(v.w));
                    }
                    *(float4 *)(lds + LS::XR + 4 * c) = v;
                }
            }
        }
        lds_barrier();
        if (*bail) return;
        VXM_LTS(24);
        if (xi >= 0 && !DMA) {
            // in_proj: per output the exact int32 block sums times d_w * d_x, added in block
            // order, + bias, BF16 (the arithmetic of k_locdit_assemble)
            for (int i = opaque_tid(); i < kH; i += kPollThreads) {
                const int8_t *wr = p.in_q + (size_t)i * kFeat;
                float acc = 0.0f;
#pragma unroll
                for (int b = 0; b < kFeat / 32; b++) {
                    int si = 0;
#pragma unroll
                    for (int h = 0; h < 32; h += 16)
                        si = vxm_dot16(*(const int4 *)(wr + 32 * b + h), *(const int4 *)(aq + 32 * b + h), si);
                    const float t = (float)si * (vxm_h2f(p.in_d[(size_t)i * (kFeat / 32) + b]) * vxm_h2f(ad[b]));
                    acc = b ? acc + t : t;
                }
                if (p.in_b) acc = acc + p.in_b[i];
                *(float *)(lds + LS::XR + 4 * i) = bf16r(acc);
            }
        }
        lds_barrier();
        VXM_LTS(25);
    }
    {
        const vxm_lblock blk = block_at(p, l);
        const bool last = l == L - 1 && k == nev - 1, end = l == L - 1;
        VXM_LTS(0);
        // ---- N1: x += down partials of block l - 1; RMSNorm(g_in) -> Q8_0 ----
        if (row >= 0) {
            const int ns = l ? kDSplits : 0;
            if (!DMA) {
                stage_gain(blk.g_in);
                if (ns)
                    poll_partials<(kDSplits * kH / 2 + kPollThreads - 1) / kPollThreads>(
                        p, chan_rsrc(p.dp, LS::WDP * 8), ns, M, row, tagb(l - 1, PH_D), lds, LS::ST, bail);
            }
            lds_barrier();
            if (*bail) return;
            VXM_LTS(1);
            row_update(lds, LS::ST, LS::XR, LS::GN, LS::MISC, ns, p.eps, p.variant, p.x1 + (size_t)row * kXPitch,
                       tagb(l, PH_X1), true);
            lds_barrier();
            // debug dump of the row entering block l (waves 0-6: wave 7's vmcnt counts only its DMAs)
            if (!DMA && p.dump)
                for (int c = opaque_tid() * 4; c < kH; c += kPollThreads * 4)
                    *(float4 *)(p.dump + ((size_t)l * M + row) * kH + c) = *(const float4 *)(lds + LS::XR + c * 4);
        }
        VXM_LTS(2);
        // ---- QKV ----
        if (is_qkv) {
            const int tid = opaque_tid(), lane = tid & 63, q4 = lane >> 4, r16 = lane & 15;
            // the rope (cos, sin) of this thread's two output pairs, fetched before the wait:
            // wave k < nct holds tile k, lane (q4, r16) row qr0 + r16 at position row % S,
            // pairs i, i + 1 of the head
            const int qk = min(tid >> 6, kMaxQT - 1);
            const int n0 = 16 * (jq + qk * wpq) + 4 * q4, ip = (n0 % LS::HD) / 2, mrow = qr0 + min(r16, nrq - 1);
            float2 rc0 = make_float2(1.0f, 0.0f), rc1 = rc0;
            if (!DMA && tid < nct * 64 && n0 < LS::QD + LS::KVD) {
                rc0 = p.cs[(size_t)(mrow % S) * LS::HALF + ip];
                rc1 = p.cs[(size_t)(mrow % S) * LS::HALF + ip + 1];
            }
            if (!DMA) {
                const uint32_t tg = tagb(l, PH_X1);
                poll_stage<(16 * kXPitch / 2 + kPollThreads - 1) / kPollThreads>(
                    p, chan_rsrc(p.x1, LS::WX * 8), kXPitch, kH / 4, 0, 32, qr0, nrq, tg, lds, LS::ST, LS::ST_SC, bail);
            } else {
                vm_wait<0>();
            }
            lds_barrier();
            if (*bail) return;
            VXM_LTS(3);
            float qacc[kMaxQT][1][4];
#pragma unroll
            for (int k = 0; k < kMaxQT; k++) {
#pragma unroll
                for (int v = 0; v < 4; v++) qacc[k][0][v] = 0.0f;
                if (k < nct) mfma_run<1, 4>(lds, LS::RA, LS::RA_SC, 32, k, LS::ST, LS::ST_SC, 32, 4 * wave, lane, qacc[k]);
            }
            lds_barrier();
            VXM_LTS(16);
#pragma unroll
            for (int k = 0; k < kMaxQT; k++)
                if (k < nct) red_store<1>(lds, LS::ST + 8192 * k, wave, lane, qacc[k]);
            lds_barrier();
            VXM_LTS(17);
            if (!DMA && tid < nct * 64) {
                const uint32_t tg = tagb(l, PH_QKV);
                const int m = qr0 + r16;
                float o[4];
                red_sum<1>(lds, LS::ST + 8192 * qk, 1, 0, 0, lane, o);
                if (r16 < nrq) {
                    const int n = n0;   // columns n .. n + 3: two pairs
                    uint64_t *dst = p.qkv + (size_t)m * (LS::NQKV / 2) + n / 2;
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const int nc = n + 2 * e;
                        float y0 = bf16r(o[2 * e]), y1 = bf16r(o[2 * e + 1]);
                        if (nc < LS::QD + LS::KVD) {
                            // pair (2i, 2i+1) of a q / k head row: dims i and i + HD/2
                            const float2 r = e ? rc1 : rc0;
                            const float z0 = bf16r(y0 * r.x - y1 * r.y), z1 = bf16r(y0 * r.y + y1 * r.x);
                            y0 = z0;
                            y1 = z1;
                        }
                        if (nc >= LS::QD) {
                            y0 = vxm_h2f(vxm_f2h(y0));
                            y1 = vxm_h2f(vxm_f2h(y1));
                        }
                        put_word(dst + e, pack_bf16x2(y0, y1), tg);
                    }
                }
            }
            lds_barrier();
        }
        VXM_LTS(4);
        // ---- attention ----
        if (is_att) {
            const int tid = opaque_tid(), lane = tid & 63;
            constexpr int HD = LS::HD, HALF = LS::HALF, HP = HD + 4;
            const int h = wg % kNH, g = (wg / kNH) % p.nseg, qb = wg / (kNH * p.nseg);
            const int kvh = h / (kNH / LS::NKV);
            const int m0 = g * S, q0 = qb * kRB, nq = min(kRB, S - q0);
            const int SP = S + 1;
            float *Kf = (float *)(lds + LS::ST), *V = Kf + S * HP, *Q = V + S * HD, *O = Q + kRB * HP,
                  *P = O + kRB * HD, *mx = P + kRB * SP, *inv = mx + kRB;
            if (!DMA) {
                // word pairs: a row of a head holds HALF words, so HP2 = HALF / 2 pairs
                constexpr int W = LS::NQKV / 2, HP2 = HALF / 2;
                const int nqp = nq * HP2, n = nqp + 2 * S * HP2;
                poll<((kRB + 2 * kMaxS) * HP2 + kPollThreads - 1) / kPollThreads>(
                    p, chan_rsrc(p.qkv, LS::WQKV * 8), n, tagb(l, PH_QKV),
                    [&](int i) {
                        if (i < nqp) return ((m0 + q0 + i / HP2) * W + h * HALF + 2 * (i % HP2)) * 8;
                        const int e = i - nqp, part = e / (S * HP2), j = (e / HP2) % S, wi = 2 * (e % HP2);
                        return ((m0 + j) * W + (part ? LS::QD + LS::KVD : LS::QD) / 2 + kvh * HALF + wi) * 8;
                    },
                    [&](int i, uint32_t a, uint32_t b) {
                        // q / k word w: dims w and w + HD/2; v word w: dims 2w, 2w + 1
                        const float a0 = __uint_as_float(a << 16), a1 = __uint_as_float(a & 0xffff0000u);
                        const float b0 = __uint_as_float(b << 16), b1 = __uint_as_float(b & 0xffff0000u);
                        float *d;
                        if (i < nqp) {
                            d = Q + (i / HP2) * HP + 2 * (i % HP2);
                        } else {
                            const int e = i - nqp, part = e / (S * HP2), j = (e / HP2) % S, wi = 2 * (e % HP2);
                            if (part) {
                                *(float4 *)(V + j * HD + 2 * wi) = make_float4(a0, a1, b0, b1);
                                return;
                            }
                            d = Kf + j * HP + wi;
                        }
                        d[0] = a0;
                        d[1] = b0;
                        d[HALF] = a1;
                        d[HALF + 1] = b1;
                    },
                    bail);
            }
            lds_barrier();
            if (*bail) return;
            VXM_LTS(5);
            // scores s_ij = (k_j . q_i) * scale: LPS lanes per score (8 at HD = 128, where the
            // serial 128-term sum was the longer wait; 1 at HD = 64), each a run of HD / LPS dims
            // in order, the partial sums added pairwise across the lanes
            constexpr int LPS = HD == 128 ? 8 : 1, RUN = HD / 4 / LPS;
            const float scale = __fdiv_rn(1.0f, __fsqrt_rn((float)HD));
            for (int idx = tid; idx < nq * S * LPS; idx += kThreads) {
                const int ij = idx / LPS, part = idx % LPS, i = ij / S, j = ij % S;
                const float4 *kr = (const float4 *)(Kf + j * HP) + part * RUN,
                             *qr = (const float4 *)(Q + i * HP) + part * RUN;
                float sc = 0.0f;
#pragma unroll 8
                for (int d4 = 0; d4 < RUN; d4++) {
                    const float4 a = kr[d4], b = qr[d4];
                    sc += a.x * b.x;
                    sc += a.y * b.y;
                    sc += a.z * b.z;
                    sc += a.w * b.w;
                }
                if (LPS == 8) sc = sum8(sc);
                if (part == 0) P[i * SP + j] = sc * scale;
            }
            lds_barrier();
            VXM_LTS(22);
            // softmax: wave i takes query row i, lane j key j
            {
                const int i = wave, j = lane;
                if (i < nq) {
                    const float sj = j < S ? P[i * SP + j] : -INFINITY;
                    const float m = rows_max(max16(sj));
                    const float e = j < S ? expf(sj - m) : 0.0f;
                    if (j < S) P[i * SP + j] = e;
                    // exact: at most 64 exponentials of one row, all in double
                    const double sum = rows_sum_d(sum16_d((double)e));
                    if (j == 0) {
                        mx[i] = m;
                        inv[i] = (float)(1.0 / sum);
                    }
                }
            }
            lds_barrier();
            VXM_LTS(23);
            // out[i][d] = sum_j v[j][d] p_ij, p_ij = e_ij * (1/sum_i), j in order (the
            // oracle's attend_one): one output per thread
            for (int idx = tid; idx < nq * HD; idx += kThreads) {
                const int i = idx / HD, d = idx % HD;
                const float iv = inv[i], *pr = P + i * SP;
                float o = 0.0f;
#pragma unroll 8
                for (int j = 0; j < S; j++) o += V[j * HD + d] * (pr[j] * iv);
                O[i * HD + d] = o;
            }
            lds_barrier();
            VXM_LTS(21);
            // Q8_0 of the output rows: thread (i, c) holds dims 8c .. 8c+7, four threads a block
            constexpr int CPR = HD / 8;
            if (!DMA && tid < nq * CPR) {
                const uint32_t tg = tagb(l, PH_ATT);
                const int i = tid / CPR, c = tid % CPR;
                float o[8], amax = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    o[e] = O[i * HD + 8 * c + e];
                    amax = fmaxf(amax, fabsf(o[e]));
                }
                amax = max4(amax);
                float d, id;
                q8_scale(amax, p.variant, d, id);
                uint32_t lo = 0, hi = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    lo |= q8_byte(o[e], id, p.variant) << (8 * e);
                    hi |= q8_byte(o[4 + e], id, p.variant) << (8 * e);
                }
                uint64_t *dst = p.att + (size_t)(m0 + q0 + i) * LS::APitch;
                const int col = h * HD + 8 * c;
                put_word(dst + col / 4, lo, tg);
                put_word(dst + col / 4 + 1, hi, tg);
                if ((c & 3) == 0) put_word(dst + LS::QD / 4 + col / 32, __float_as_uint(vxm_h2f(vxm_f2h(d))), tg);
            }
            lds_barrier();
        }
        VXM_LTS(6);
        // ---- O: 16-column tile oc over K quarter os ----
        {
            const int tid = opaque_tid(), lane = tid & 63, q4 = lane >> 4, r16 = lane & 15;
            if (!DMA) {
                const uint32_t tg = tagb(l, PH_ATT);
                poll_stage<(kMaxM * 9 * LS::BO / 2 + kPollThreads - 1) / kPollThreads>(
                    p, chan_rsrc(p.att, LS::WA * 8), LS::APitch, LS::QD / 4, LS::BO * os, LS::BO, 0, M, tg, lds, LS::ST,
                    LS::ST_SC, bail);
            } else {
                if (!drow) issue_d(blk);
                if (is_gu) issue_gu_a(blk);
                else if (is_qkv && !last) issue_qkv(block_at(p, (l + 1) % L));
                if (is_gu && is_qkv)
                    vm_wait<63>();
                else if (is_gu && drow)
                    vm_wait<nGA>();
                else if (is_gu)
                    vm_wait<nD + nGA>();
                else
                    vm_wait<nD>();
            }
            lds_barrier();
            if (*bail) return;
            VXM_LTS(7);
            zero_acc();
            mfma_run<MT, LS::BO / kWaves>(lds, LS::RO, LS::RO_SC, LS::BO, 0, LS::ST, LS::ST_SC, LS::BO,
                                          (LS::BO / kWaves) * wave, lane, acc);
            lds_barrier();
            red_store<MT>(lds, LS::ST, wave, lane, acc);
            lds_barrier();
            if (!DMA && tid < MT * 64) {
                const uint32_t tg = tagb(l, PH_O);
                const int t = tid >> 6, m = 16 * t + r16;
                float o[4];
                red_sum<MT>(lds, LS::ST, 1, 0, t, lane, o);
                if (m < M) {
                    uint64_t *dst = p.op + ((size_t)os * M + m) * kH + 16 * oc + 4 * q4;
#pragma unroll
                    for (int v = 0; v < 4; v++) put_word(dst + v, __float_as_uint(o[v]), tg);
                }
            }
            lds_barrier();
        }
        VXM_LTS(8);
        // ---- N2: x += O; RMSNorm(g_post) -> Q8_0 ----
        if (row >= 0) {
            if (!DMA) {
                stage_gain(blk.g_post);
                poll_partials<(kOSplits * kH / 2 + kPollThreads - 1) / kPollThreads>(
                    p, chan_rsrc(p.op, LS::WOP * 8), kOSplits, M, row, tagb(l, PH_O), lds, LS::ST, bail);
            }
            lds_barrier();
            if (*bail) return;
            VXM_LTS(9);
            row_update(lds, LS::ST, LS::XR, LS::GN, LS::MISC, kOSplits, p.eps, p.variant,
                       p.x2 + (size_t)row * kXPitch, tagb(l, PH_X2), true);
            lds_barrier();
        }
        VXM_LTS(10);
        // ---- gate/up: 64 interleaved rows -> 32 SwiGLU outputs -> one Q8_0 block per row,
        // for the rows gr0 .. gr0 + nrg - 1 of this unit's group ----
        if (is_gu) {
            constexpr int MTG = MT == 3 ? 2 : 1;   // row tiles of a group: at most 24 rows
            const int tid = opaque_tid(), lane = tid & 63, q4 = lane >> 4, r16 = lane & 15;
            if (!DMA) {
                const uint32_t tg = tagb(l, PH_X2);
                poll_stage<(16 * MTG * kXPitch / 2 + kPollThreads - 1) / kPollThreads>(
                    p, chan_rsrc(p.x2, LS::WX * 8), kXPitch, kH / 4, 0, 32, gr0, nrg, tg, lds, LS::ST, LS::ST_SC, bail);
            } else {
                issue_gu_b(blk);
                if (last) {
                    vm_wait<0>();
                } else {
                    issue_o(block_at(p, (l + 1) % L));
                    vm_wait<nO>();
                }
            }
            lds_barrier();
            if (*bail) return;
            VXM_LTS(11);
            // wave w: tiles 2 (w & 1) and 2 (w & 1) + 1 over the K quarter w >> 1
            const int ch = wave & 1, kq = wave >> 1;
            float acc2[2][MTG][4];
#pragma unroll
            for (int cc = 0; cc < 2; cc++)
#pragma unroll
                for (int t = 0; t < MTG; t++)
#pragma unroll
                    for (int v = 0; v < 4; v++) acc2[cc][t][v] = 0.0f;
            mfma_run2<MTG, 8, 4>(lds, LS::RA, LS::RA_SC, 32, 2 * ch, LS::ST, LS::ST_SC, 32, 8 * kq, lane, acc2);
            lds_barrier();
            VXM_LTS(18);
            {
                float4 *red = (float4 *)(lds + LS::ST);   // [wave][2][MTG][64]: 32 KiB at MTG = 2
#pragma unroll
                for (int cc = 0; cc < 2; cc++)
#pragma unroll
                    for (int t = 0; t < MTG; t++)
                        red[((wave * 2 + cc) * MTG + t) * 64 + lane] =
                            make_float4(acc2[cc][t][0], acc2[cc][t][1], acc2[cc][t][2], acc2[cc][t][3]);
            }
            lds_barrier();
            VXM_LTS(19);
            // the SwiGLU outputs after the partial sums in the stage area ([group row][33])
            static_assert(32 * 1024 + (kMaxM / 2) * 33 * 4 <= LS::ST_SC - LS::ST, "gate/up outputs in the stage");
            float *ps = (float *)(lds + LS::ST + 32 * 1024);
            for (int idx = tid; idx < 4 * MTG * 64; idx += kThreads) {
                const int ct2 = idx / (MTG * 64), t = (idx / 64) % MTG;
                float o[4];
                {
                    // the four K quarters in order
                    const float4 *red = (const float4 *)(lds + LS::ST);
                    const int h2 = ct2 >> 1, cc = ct2 & 1;
                    float4 s = red[(((0 * 2 + h2) * 2 + cc) * MTG + t) * 64 + lane];
#pragma unroll
                    for (int k = 1; k < 4; k++) {
                        const float4 u = red[(((2 * k + h2) * 2 + cc) * MTG + t) * 64 + lane];
                        s.x = s.x + u.x;
                        s.y = s.y + u.y;
                        s.z = s.z + u.z;
                        s.w = s.w + u.w;
                    }
                    o[0] = s.x;
                    o[1] = s.y;
                    o[2] = s.z;
                    o[3] = s.w;
                }
                const int m = 16 * t + r16;
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    // rows 2j (gate) and 2j + 1 (up) of the interleaved weight
                    const float gb = bf16r(o[2 * e]);
                    const float s = bf16r(__fdiv_rn(gb, 1.0f + expf(-gb)));
                    ps[m * 33 + 8 * ct2 + 2 * q4 + e] = bf16r(s * bf16r(o[2 * e + 1]));
                }
            }
            lds_barrier();
            VXM_LTS(20);
            if (!DMA && tid < 4 * nrg) {
                const uint32_t tg = tagb(l, PH_P);
                const int mi = tid >> 2, part = tid & 3;
                float o[8], amax = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    o[e] = ps[mi * 33 + 8 * part + e];
                    amax = fmaxf(amax, fabsf(o[e]));
                }
                amax = max4(amax);
                float d, id;
                q8_scale(amax, p.variant, d, id);
                uint32_t lo = 0, hi = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    lo |= q8_byte(o[e], id, p.variant) << (8 * e);
                    hi |= q8_byte(o[4 + e], id, p.variant) << (8 * e);
                }
                uint64_t *dst = p.pp + (size_t)(gr0 + mi) * kPPitch;
                const int col = 32 * ugu + 8 * part;
                put_word(dst + col / 4, lo, tg);
                put_word(dst + col / 4 + 1, hi, tg);
                if (part == 0) put_word(dst + kF / 4 + ugu, __float_as_uint(vxm_h2f(vxm_f2h(d))), tg);
            }
            lds_barrier();
        }
        VXM_LTS(12);
        // ---- down, above 16 rows: 64-column tile dc2 over K eighth ds2 for one row group ----
        if (drow) {
            constexpr int MTD = MT == 3 ? 2 : 1;   // row tiles of a group: at most 24 rows
            const int tid = opaque_tid(), lane = tid & 63, q4 = lane >> 4, r16 = lane & 15;
            if (!DMA) {
                const uint32_t tg = tagb(l, PH_P);
                poll_stage<(16 * MTD * 9 * 16 / 2 + kPollThreads - 1) / kPollThreads>(
                    p, chan_rsrc(p.pp, LS::WP * 8), kPPitch, kF / 4, 16 * ds2, 16, dr0, nrd, tg, lds, LS::ST,
                    LS::ST_SC, bail);
            } else {
                // the gate/up products are done: the region takes this block's down tile now
                issue_d2(blk);
                vm_wait<0>();
            }
            lds_barrier();
            if (*bail) return;
            VXM_LTS(13);
            // wave w: column tile w & 3 over the K half w >> 2 of the eighth
            float ad[MTD][4];
#pragma unroll
            for (int t = 0; t < MTD; t++)
#pragma unroll
                for (int v = 0; v < 4; v++) ad[t][v] = 0.0f;
            mfma_run<MTD, 8>(lds, LS::RA, LS::RA_SC, 16, wave & 3, LS::ST, LS::ST_SC, 16, 8 * (wave >> 2), lane, ad);
            lds_barrier();
            // the region is free again: at an evaluation's end the update workgroup takes
            // out_proj's first half (the next block's QKV tiles go out at its top, where the
            // wave is not in a workgroup barrier's way: issued here, they held up the reduction
            // by ~2 us)
            if (DMA && upd && end) issue_out_a();
            red_store<MTD>(lds, LS::ST, wave, lane, ad);
            lds_barrier();
            // 4 MTD (column tile, row tile) pairs of 64 lanes over waves 0-6 (up to 512 threads)
            if (!DMA) {
                const uint32_t tg = tagb(l, PH_D);
                for (int idx = tid; idx < 4 * MTD * 64; idx += kPollThreads) {
                    const int ct2 = idx / (MTD * 64), t = (idx / 64) % MTD, ln = idx & 63;
                    const int m = 16 * t + (ln & 15);
                    float o[4];
                    red_sum<MTD>(lds, LS::ST, 4, ct2, t, ln, o);
                    if (m < nrd) {
                        uint64_t *dst = p.dp + ((size_t)ds2 * M + dr0 + m) * kH + 64 * dc2 + 16 * ct2 + 4 * (ln >> 4);
#pragma unroll
                        for (int v = 0; v < 4; v++) put_word(dst + v, __float_as_uint(o[v]), tg);
                    }
                }
            }
            lds_barrier();
        }
        // ---- down: 32-column tile dc over K eighth ds ----
        else {
            const int tid = opaque_tid(), lane = tid & 63, q4 = lane >> 4, r16 = lane & 15;
            if (!DMA) {
                const uint32_t tg = tagb(l, PH_P);
                poll_stage<(kMaxM * 9 * 16 / 2 + kPollThreads - 1) / kPollThreads>(
                    p, chan_rsrc(p.pp, LS::WP * 8), kPPitch, kF / 4, 16 * ds, 16, 0, M, tg, lds, LS::ST, LS::ST_SC, bail);
            } else {
                if (!last && !is_gu) issue_o(block_at(p, (l + 1) % L));
                // the update workgroup takes out_proj into the QKV region here and the next
                // evaluation's QKV tiles after its products
                if (!last && is_gu && is_qkv && !(upd && end)) issue_qkv(block_at(p, (l + 1) % L));
                if (upd && end) issue_out_a();
                if (is_gu)
                    vm_wait<63>();
                else if (last)
                    vm_wait<0>();
                else if (is_qkv)
                    vm_wait<nQKV + nO>();
                else
                    vm_wait<nO>();
            }
            lds_barrier();
            if (*bail) return;
            VXM_LTS(13);
            zero_acc();
            const int ct = wave & 1, kq = wave >> 1;
            mfma_run<MT, 4>(lds, LS::RD, LS::RD_SC, 16, ct, LS::ST, LS::ST_SC, 16, 4 * kq, lane, acc);
            lds_barrier();
            red_store<MT>(lds, LS::ST, wave, lane, acc);
            lds_barrier();
            if (!DMA && tid < 2 * MT * 64) {
                const uint32_t tg = tagb(l, PH_D);
                const int ct2 = tid / (MT * 64), t = (tid / 64) % MT, m = 16 * t + r16;
                float o[4];
                red_sum<MT>(lds, LS::ST, 2, ct2, t, lane, o);
                if (m < M) {
                    uint64_t *dst = p.dp + ((size_t)ds * M + m) * kH + 32 * dc + 16 * ct2 + 4 * q4;
#pragma unroll
                    for (int v = 0; v < 4; v++) put_word(dst + v, __float_as_uint(o[v]), tg);
                }
            }
            lds_barrier();
        }
        VXM_LTS(14);
        // solve mode, an evaluation's last block: the x rows' owners add its down projection
        // and publish their final norm's Q8_0 (segment-major rows) for the update workgroup
        if (solve && end && row >= 0 && row % S >= p.fin_r0) {
            if (!DMA) {
                stage_gain(p.fin_g);
                poll_partials<(kDSplits * kH / 2 + kPollThreads - 1) / kPollThreads>(
                    p, chan_rsrc(p.dp, LS::WDP * 8), kDSplits, M, row, tagb(l, PH_D), lds, LS::ST, bail);
            }
            lds_barrier();
            if (*bail) return;
            VXM_LTS(15);
            const int orow = (row / S) * (S - p.fin_r0) + row % S - p.fin_r0;
            row_update(lds, LS::ST, LS::XR, LS::GN, LS::MISC, kDSplits, p.eps, p.variant,
                       p.fq + (size_t)orow * kXPitch, tagb(L, PH_X1), true);
            lds_barrier();
        }
        // the last block: row owners add its down projection and write x out (and with
        // fin_g, the x rows their final norm)
        if (!solve && last && row >= 0) {
            const bool fin = p.fin_g && row % S >= p.fin_r0;
            if (!DMA) {
                if (fin) stage_gain(p.fin_g);
                poll_partials<(kDSplits * kH / 2 + kPollThreads - 1) / kPollThreads>(
                    p, chan_rsrc(p.dp, LS::WDP * 8), kDSplits, M, row, tagb(l, PH_D), lds, LS::ST, bail);
            }
            lds_barrier();
            if (*bail) return;
            VXM_LTS(15);
            row_update(lds, LS::ST, LS::XR, LS::GN, LS::MISC, kDSplits, 0.0f, p.variant, nullptr, 0, false);
            lds_barrier();
            const int tid = opaque_tid();
            for (int c = tid * 4; c < kH; c += kThreads * 4)
                *(float4 *)(p.x + (size_t)row * kH + c) = *(const float4 *)(lds + LS::XR + c * 4);
            if (!DMA && p.dump)
                for (int c = tid * 4; c < kH; c += kPollThreads * 4)
                    *(float4 *)(p.dump + ((size_t)L * M + row) * kH + c) = *(const float4 *)(lds + LS::XR + c * 4);
            if (fin) {
                const int orow = (row / S) * (S - p.fin_r0) + row % S - p.fin_r0;
                row_final_norm(lds, LS::XR, LS::GN, LS::MISC, p.eps, p.variant, p.fin_q + (size_t)orow * kH,
                               p.fin_d + (size_t)orow * (kH / 32));
            }
        }
    }
    // ---- solve mode: out_proj, CFG-Zero* and the Euler step (k_cfm_update's steps) ----
    if (upd && l == L - 1) {
        const int NR = p.n_seg * p.P, n = p.P * kFeat, tid = opaque_tid(), lane = tid & 63;
        if (!DMA) {
            poll_stage<(kMaxM * kXPitch / 2 + kPollThreads - 1) / kPollThreads>(
                p, chan_rsrc(p.fq, LS::WX * 8), kXPitch, kH / 4, 0, 32, 0, NR, tagb(L, PH_X1), lds, LS::ST,
                LS::ST_SC, bail);
        } else {
            vm_wait<31>();
            issue_out_b();
            vm_wait<0>();
        }
        lds_barrier();
        if (*bail) return;
        VXM_LTS(26);
        // wave w: out_proj column tile w & 3 over the K half w >> 2, on the x rows' one
        // row tile (NR <= 16: the solve's fit)
        float acco[1][4] = {};
        mfma_run<1, 16>(lds, LS::RA, LS::RA_SC, 32, wave & 3, LS::ST, LS::ST_SC, 32, 16 * (wave >> 2), lane, acco);
        lds_barrier();
        VXM_LTS(28);
        red_store<1>(lds, LS::ST, wave, lane, acco);
        lds_barrier();
        // vo [NR][64] fp32 after the partials: the two K halves in order
        float *vo = (float *)(lds + LS::ST + kWaves * 1024);
        static_assert(kWaves * 1024 + kMaxM * kFeat * 4 <= LS::ST_SC - LS::ST, "out_proj rows in the stage");
        for (int idx = tid; idx < 4 * 64; idx += kThreads) {
            const int ct = idx / 64, t = 0, ln = idx & 63, m = ln & 15;
            float o[4];
            red_sum<1>(lds, LS::ST, 4, ct, t, ln, o);
            if (m < NR)
#pragma unroll
                for (int v = 0; v < 4; v++) vo[m * kFeat + 16 * ct + 4 * (ln >> 4) + v] = o[v];
        }
        lds_barrier();
        VXM_LTS(29);
        // element j of the conditional rows [0, n) and the unconditional [n, 2n): waves 0-6,
        // elements tid + 448 e held in registers; the products for the sums in double go to
        // the weight region (out_proj is read)
        constexpr int UPT = (kSolveMaxN + kPollThreads - 1) / kPollThreads;
        double *prod = (double *)(lds + LS::RA);
        static_assert(2 * kSolveMaxN * 8 <= LS::RA_SC - LS::RA, "CFG products");
        float pv[UPT], qv[UPT], xv[UPT];
        if (!DMA) {
#pragma unroll
            for (int e = 0; e < UPT; e++) {
                const int j = tid + kPollThreads * e;
                if (j >= n) break;
                const int c = j % kFeat;
                float pp = vo[j];
                if (p.out_b) pp = pp + p.out_b[c];
                pv[e] = bf16r(pp);
                if (p.use_cfg) {
                    float qq = vo[n + j];
                    if (p.out_b) qq = qq + p.out_b[c];
                    qv[e] = bf16r(qq);
                    prod[j] = (double)bf16r(pv[e] * qv[e]);
                    prod[n + j] = (double)bf16r(qv[e] * qv[e]);
                }
                xv[e] = p.xs[j];
            }
        }
        lds_barrier();
        float *st_sh = (float *)(lds + LS::MISC + 72);
        if (p.use_cfg && tid == 0) {
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
            const float dot_b = bf16r((float)dot);
            const float norm_b = bf16r((float)sq + 1.0e-8f);
            *st_sh = bf16r(__fdiv_rn(dot_b, norm_b));
        }
        lds_barrier();
        VXM_LTS(30);
        const bool more = k + 1 < nev;
        int8_t *nq = (int8_t *)(lds + LS::ST);                        // the new x's Q8_0
        uint16_t *nd = (uint16_t *)(lds + LS::ST + kSolveMaxN);
        if (!DMA) {
            const float st = p.use_cfg ? *st_sh : 0.0f, cfg_b = bf16r(p.cfg), dt = p.dts[k];
            // n % 32 == 0 and 448 % 32 == 0: the 32 lanes of a half wave hold one block of x
#pragma unroll
            for (int e = 0; e < UPT; e++) {
                const int j = tid + kPollThreads * e;
                if (j >= n) break;
                float v = pv[e];
                if (p.use_cfg) {
                    const float ns = bf16r(qv[e] * st);
                    const float gd = bf16r(pv[e] - ns);
                    const float gg = bf16r(cfg_b * gd);
                    v = bf16r(ns + gg);
                }
                const float xn = bf16r(xv[e] + bf16r(dt * v));
                p.xs[j] = xn;
                if (more) {
                    float amax = fabsf(xn);
#pragma unroll
                    for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
                    float d, id;
                    q8_scale(amax, p.variant, d, id);
                    nq[j] = (int8_t)q8_byte(xn, id, p.variant);
                    if ((j & 31) == 0) nd[j / 32] = vxm_f2h(d);
                }
            }
        }
        lds_barrier();
        VXM_LTS(31);
        if (more) {
            // the new x's Q8_0 to the next evaluation's row owners, then its QKV tiles (the
            // weight region is free again)
            if (!DMA)
                for (int w = tid; w < p.P * kXqWords; w += kPollThreads) {
                    const int xi = w / kXqWords, e = w % kXqWords;
                    const uint32_t pay = e < kFeat / 4 ? *(const uint32_t *)(nq + xi * kFeat + 4 * e)
                                                       : (uint32_t)nd[xi * (kFeat / 32) + e - kFeat / 4];
                    put_word(p.xqc + w, pay, tagb(L, PH_X2));
                }
            if (DMA && is_qkv) issue_qkv(block_at(p, 0));
            lds_barrier();
        }
        VXM_LTS(27);
    }
    }
}

template <class LS, int MT>
__global__ __launch_bounds__(kThreads, 1) void k_locdit_persistent(vxm_lparams p) {
    // All of the workgroup's LDS is this one dynamic array, so it starts at address 0
    // (the weight DMAs address it absolutely) and every layout offset is aligned.
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int *bail = (int *)(lds + LS::MISC + 64);
    uint32_t *ep_sh = (uint32_t *)(lds + LS::MISC + 68);
    const int wg = blockIdx.x, tid = threadIdx.x;
    if (tid == 0) {
        *bail = 0;
        *ep_sh = __hip_atomic_load(p.state, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#ifdef VXM_PERSISTENT_TRACE
        if (p.trace) p.trace[(size_t)wg * (1 + kTraceSlots * p.L * max(p.n_eval, 1))] = __builtin_amdgcn_s_memrealtime();
#endif
    }
    // block 0's input rows (in solve mode the row owners assemble them)
    if (wg < p.M && p.n_eval == 0)
        for (int c = tid * 4; c < kH; c += kThreads * 4)
            *(float4 *)(lds + LS::XR + c * 4) = *(const float4 *)(p.x + (size_t)wg * kH + c);
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    lds_barrier();
    const uint32_t ep = *ep_sh;
    if ((tid >> 6) == kWaves - 1) run_blocks<LS, MT, true>(p, lds, bail, ep);
    else run_blocks<LS, MT, false>(p, lds, bail, ep);
    // every weight load of wave 7 has landed before the workgroup ends
    vm_wait<0>();
    lds_barrier();
    if (tid == 0) {
        const uint32_t done = __hip_atomic_fetch_add(p.state + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == kG - 1) {
            // the last workgroup: every workgroup has read the epoch; the next launch uses the
            // next one and starts with a clear live error word
            __hip_atomic_store(p.state + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.err, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p.state, ep + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

using ShapeDitMha = LShape<16, 64>;
using ShapeDitGqa = LShape<2, 128>;

}  // namespace

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct vxm_lpersist {
    void *base = nullptr;
    vxm_lblock *blocks = nullptr;
    int L = 0;
    std::vector<const void *> key;   // the weight pointers the table holds
    uint64_t *chan[9] = {};
    int *err = nullptr;
    uint32_t *state = nullptr;
};

// Supported: hidden 1024, FFN 4096, 16 query heads of (16 kv heads x 64) or
// (2 kv heads x 128), M <= 48 rows in segments of S <= 32, 256 CUs.
bool vxm_locdit_persistent_fits(vxm_ctx *ctx, const vxm_block_dims &d, int64_t M, int S) {
    if (ctx->n_cu != kG || d.H != kH || d.F != kF || d.nh != kNH || d.no_rope || d.res_scale != 1.0f) return false;
    if (!((d.nkv == 16 && d.hd == 64) || (d.nkv == 2 && d.hd == 128))) return false;
    if (M <= 0 || M > kMaxM || S <= 0 || S > kMaxS || M % S) return false;
    if (!d.rope_cs || d.rope_rows < S) return false;
    return true;
}

// AUTO takes the single launch wherever it fits: with QKV and gate/up split by row
// groups it measured faster than launch by launch at both layouts (per LocDiT
// evaluation: 486.6 against 518.6 us at 16 x 64 heads and 2 x 24 rows, 410 against 474
// at 16 / 2 x 128 and 2 x 11).
bool vxm_locdit_persistent_pick(vxm_ctx *ctx, const vxm_block_dims &d, int64_t M, int S, int mode) {
    if (mode == VXM_DECODE_KERNELS || !vxm_locdit_persistent_fits(ctx, d, M, S)) return false;
    return true;
}

void vxm_locdit_persistent_free(vxm_lpersist *st) {
    if (!st) return;
    if (st->base) (void)hipFree(st->base);
    delete st;
}

static bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15) == 0; }

bool vxm_locdit_persistent_solve_fits(vxm_ctx *ctx, const vxm_block_dims &d, int64_t M, int S,
                                      const vxm_lsolve &sv) {
    if (!vxm_locdit_persistent_fits(ctx, d, M, S)) return false;
    if (sv.n_eval <= 0 || sv.n_eval > kMaxEval || sv.feat != kFeat || sv.P <= 0 || sv.Pc < 0 ||
        sv.P * kFeat > kSolveMaxN || 3 + sv.Pc + sv.P != S || sv.n_seg * S != M || sv.n_seg < 1 || sv.n_seg > 2)
        return false;
    if (sv.use_cfg && sv.n_seg != 2) return false;
    if (sv.n_seg * sv.P > 16) return false;   // out_proj takes the x rows as one row tile
    if (!sv.in_proj || !sv.out_proj || sv.in_proj->n != kH || sv.in_proj->k != kFeat || sv.out_proj->n != kFeat ||
        sv.out_proj->k != kH || !aligned16(sv.in_proj->qs) || !aligned16(sv.out_proj->qs) ||
        !aligned16(sv.out_proj->d))
        return false;
    // float4 reads of the assembled rows
    if (!aligned16(sv.tc) || !aligned16(sv.mu) || !aligned16(sv.ch) || !aligned16(sv.cb)) return false;
    return sv.dts && sv.tc && sv.x && sv.xq0 && sv.xd0 && (sv.Pc == 0 || sv.ch);
}

int vxm_locdit_persistent_run(vxm_ctx *ctx, const vxm_block_dims &d, const std::vector<vxm_block> &blocks,
                              vxm_lpersist **stp, float *x, int64_t M, int S, float *dump, const vxm_lfinal &fin,
                              const vxm_lsolve *sv) {
    if (!vxm_locdit_persistent_fits(ctx, d, M, S))
        return vxm_fail(ctx, VXM_ERR_NOT_IMPLEMENTED, "persistent blocks: unsupported shape (M=%lld S=%d)",
                        (long long)M, S);
    if (sv && (!vxm_locdit_persistent_solve_fits(ctx, d, M, S, *sv) || !fin.g || fin.r0 != 3 + sv->Pc || dump))
        return vxm_fail(ctx, VXM_ERR_NOT_IMPLEMENTED, "persistent blocks: unsupported solve (M=%lld S=%d)",
                        (long long)M, S);
    const int L = (int)blocks.size();
    if (L <= 0) return VXM_OK;
    std::vector<const void *> key;
    for (const vxm_block &b : blocks) {
        const vxm_weight *w[4] = {b.wqkv, b.wo, b.wgu, b.wd};
        for (const vxm_weight *wi : w) {
            if (!wi || !aligned16(wi->qs) || !aligned16(wi->d))
                return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "persistent blocks: weights not 16-byte aligned");
            key.push_back(wi->qs);
            key.push_back(wi->d);
        }
        key.push_back(b.g_in);
        key.push_back(b.g_post);
    }
    vxm_lpersist *st = *stp;
    if (!st || st->L != L || st->key != key) {
        // the exchange buffers and block table are made (hipMalloc, synchronous copies) by an eager
        // call; under graph capture that would record nothing and fail
        hipStreamCaptureStatus cap_st = hipStreamCaptureStatusNone;
        VXM_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cap_st));
        if (cap_st != hipStreamCaptureStatusNone)
            return vxm_fail(ctx, VXM_ERR_INVALID_ARG,
                            "persistent blocks: their buffers and block table are set up by an eager call; run "
                            "one evaluation with these weights before capturing");
        vxm_locdit_persistent_free(st);
        *stp = nullptr;
        st = new vxm_lpersist();
        st->L = L;
        st->key = key;
        const int qd = kNH * d.hd, nqkv = qd + 2 * d.nkv * d.hd;
        const size_t words[9] = {(size_t)kMaxM * kXPitch,
                                 (size_t)kMaxM * nqkv / 2,
                                 (size_t)kMaxM * (qd / 4 + qd / 32),
                                 (size_t)kOSplits * kMaxM * kH,
                                 (size_t)kMaxM * kXPitch,
                                 (size_t)kMaxM * kPPitch,
                                 (size_t)kDSplits * kMaxM * kH,
                                 (size_t)kMaxM * kXPitch,
                                 (size_t)kMaxS * kXqWords};
        size_t total = 0;
        for (size_t w : words) total += (w * 8 + 255) & ~(size_t)255;
        const size_t tab = ((size_t)L * sizeof(vxm_lblock) + 255) & ~(size_t)255;
        const size_t bytes = total + tab + 256;
        if (hipMalloc(&st->base, bytes) != hipSuccess) {
            (void)hipGetLastError();
            delete st;
            return vxm_fail(ctx, VXM_ERR_OOM, "persistent blocks: %zu bytes of exchange buffers", bytes);
        }
        char *b = (char *)st->base;
        for (int c = 0; c < 9; c++) {
            st->chan[c] = (uint64_t *)b;
            b += (words[c] * 8 + 255) & ~(size_t)255;
        }
        st->blocks = (vxm_lblock *)b;
        b += tab;
        st->err = (int *)b;
        st->state = (uint32_t *)(b + 64);
        std::vector<vxm_lblock> th(L);
        for (int l = 0; l < L; l++) {
            const vxm_block &bl = blocks[l];
            th[l] = vxm_lblock{bl.wqkv->qs, bl.wo->qs, bl.wgu->qs, bl.wd->qs, bl.wqkv->d, bl.wo->d,
                               bl.wgu->d,   bl.wd->d,  bl.g_in,    bl.g_post};
        }
        // zeroed words carry an even tag, never a live (odd) one; epoch 1, no workgroup finished
        const uint32_t st0[2] = {1u, 0u};
        if (hipMemset(st->base, 0, bytes) != hipSuccess ||
            hipMemcpy(st->blocks, th.data(), L * sizeof(vxm_lblock), hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(st->state, st0, sizeof st0, hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipGetLastError();
            vxm_locdit_persistent_free(st);
            return vxm_fail(ctx, VXM_ERR_BACKEND, "persistent blocks: buffer set-up failed");
        }
        // the kernels' LDS limit, set here rather than at a launch that may be under graph capture
        const void *kern[6] = {(const void *)k_locdit_persistent<ShapeDitMha, 1>,
                               (const void *)k_locdit_persistent<ShapeDitMha, 2>,
                               (const void *)k_locdit_persistent<ShapeDitMha, 3>,
                               (const void *)k_locdit_persistent<ShapeDitGqa, 1>,
                               (const void *)k_locdit_persistent<ShapeDitGqa, 2>,
                               (const void *)k_locdit_persistent<ShapeDitGqa, 3>};
        bool attr_ok = true;
        for (int i = 0; i < 6; i++)
            attr_ok &= hipFuncSetAttribute(kern[i], hipFuncAttributeMaxDynamicSharedMemorySize,
                                           i < 3 ? ShapeDitMha::BYTES : ShapeDitGqa::BYTES) == hipSuccess;
        if (!attr_ok) {
            (void)hipGetLastError();
            vxm_locdit_persistent_free(st);
            return vxm_fail(ctx, VXM_ERR_BACKEND, "persistent blocks: LDS limit not accepted");
        }
        *stp = st;
    }
    vxm_lparams prm{};
    prm.blocks = st->blocks;
    prm.L = L;
    prm.M = (int)M;
    prm.S = S;
    prm.nseg = (int)(M / S);
    prm.qb = (S + kRB - 1) / kRB;
    prm.eps = d.eps;
    prm.variant = ctx->quant_variant;
    prm.cs = d.rope_cs;
    prm.x = x;
    prm.x1 = st->chan[0];
    prm.qkv = st->chan[1];
    prm.att = st->chan[2];
    prm.op = st->chan[3];
    prm.x2 = st->chan[4];
    prm.pp = st->chan[5];
    prm.dp = st->chan[6];
    prm.err = st->err;
    prm.state = st->state;
    prm.dump = dump;
    if (fin.g) {
        if (fin.r0 < 0 || fin.r0 >= S || (!sv && (!fin.q || !fin.d)))
            return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "persistent blocks: final norm rows %d of %d", fin.r0, S);
        prm.fin_g = fin.g;
        prm.fin_r0 = fin.r0;
        prm.fin_q = fin.q;
        prm.fin_d = fin.d;
    }
    if (sv) {
        prm.n_eval = sv->n_eval;
        prm.P = sv->P;
        prm.Pc = sv->Pc;
        prm.n_seg = sv->n_seg;
        prm.n_mu = sv->n_mu;
        prm.use_cfg = sv->use_cfg;
        prm.cfg = sv->cfg;
        prm.tc = sv->tc;
        prm.mu = sv->mu;
        prm.ch = sv->ch;
        prm.cb = sv->cb;
        prm.in_q = sv->in_proj->qs;
        prm.in_d = sv->in_proj->d;
        prm.in_b = sv->in_b;
        prm.out_q = sv->out_proj->qs;
        prm.out_d = sv->out_proj->d;
        prm.out_b = sv->out_b;
        prm.xs = sv->x;
        prm.xq0 = sv->xq0;
        prm.xd0 = sv->xd0;
        prm.fq = st->chan[7];
        prm.xqc = st->chan[8];
        for (int k = 0; k < sv->n_eval; k++) prm.dts[k] = sv->dts[k];
    }
    if (kNH * prm.nseg * prm.qb > kG)
        return vxm_fail(ctx, VXM_ERR_NOT_IMPLEMENTED, "persistent blocks: too many attention units");
    // All 256 workgroups wait on each other's words, so all must be resident: one per CU
    // (the LDS layout takes more than half of a CU's).  Every wait is bounded (kSpin
    // rounds, then the error word), so other work on the device can only turn a launch
    // into an error, never a hang (vxm_locdit_check / vxm_locenc_check report it).  Eager
    // launches are ordered after the device's previous single-launch kernel, whatever its
    // stream (vxm_ordered_launch_begin), so two never interleave their workgroups.
#ifdef VXM_PERSISTENT_TRACE
    // profiling build: timestamps of every eager launch into
    // $VXM_TRACE_DIR/ltrace_L<blocks>_M<rows>_<n>.bin (launches recorded into a graph run untraced)
    const int tblocks = L * (sv ? sv->n_eval : 1);
    const size_t tstride = 1 + (size_t)kTraceSlots * tblocks, tbytes = (size_t)kG * tstride * 8;
    static uint64_t *tbuf = nullptr;
    static size_t tcap = 0;
    static int ncall = 0;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    VXM_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cap));
    const bool traced = cap == hipStreamCaptureStatusNone;
    if (traced && tcap < tbytes) {
        if (tbuf) (void)hipFree(tbuf);
        tbuf = nullptr;
        tcap = 0;
        VXM_HIP(ctx, hipMalloc(&tbuf, tbytes));
        tcap = tbytes;
    }
    if (traced) {
        VXM_HIP(ctx, hipMemset(tbuf, 0, tbytes));
        prm.trace = tbuf;
    }
#endif
    // row tiles of 16 as a template argument: the products' loops unroll completely
    const int mt = (int)((M + 15) / 16);
    vxm_launch_slot *slot = nullptr;
    bool capturing = false;
    if (int rc = vxm_ordered_launch_begin(ctx, &slot, &capturing)) return rc;
#define VXM_LP_LAUNCH(LS, MT)                                                                                \
    hipLaunchKernelGGL((k_locdit_persistent<LS, MT>), dim3(kG), dim3(kThreads), (unsigned)LS::BYTES, ctx->stream, prm)
    if (d.nkv == 16) {
        if (mt == 1) VXM_LP_LAUNCH(ShapeDitMha, 1);
        else if (mt == 2) VXM_LP_LAUNCH(ShapeDitMha, 2);
        else VXM_LP_LAUNCH(ShapeDitMha, 3);
    } else {
        if (mt == 1) VXM_LP_LAUNCH(ShapeDitGqa, 1);
        else if (mt == 2) VXM_LP_LAUNCH(ShapeDitGqa, 2);
        else VXM_LP_LAUNCH(ShapeDitGqa, 3);
    }
#undef VXM_LP_LAUNCH
    const hipError_t le = hipGetLastError();
    if (int rc = vxm_ordered_launch_end(ctx, slot, capturing)) return rc;
    if (le != hipSuccess) return vxm_fail(ctx, VXM_ERR_BACKEND, "persistent blocks launch failed: %s", hipGetErrorString(le));
#ifdef VXM_PERSISTENT_TRACE
    if (traced) {
        std::vector<uint64_t> th((size_t)kG * tstride);
        VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        VXM_HIP(ctx, hipMemcpy(th.data(), tbuf, tbytes, hipMemcpyDeviceToHost));
        const char *dir = getenv("VXM_TRACE_DIR");
        char fn[512];
        snprintf(fn, sizeof fn, "%s/ltrace_L%d_M%d_%04d.bin", dir ? dir : ".", tblocks, (int)M, ncall++);
        if (FILE *f = fopen(fn, "wb")) {
            fwrite(th.data(), 8, th.size(), f);
            fclose(f);
        }
    }
#endif
    return VXM_OK;
}

int vxm_locdit_persistent_check(vxm_ctx *ctx, vxm_lpersist *st) {
    if (!st || !st->err) return VXM_OK;
    int e = 0;
    VXM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    VXM_HIP(ctx, hipMemcpy(&e, st->err + 1, 4, hipMemcpyDeviceToHost));
    if (e) {
        VXM_HIP(ctx, hipMemset(st->err + 1, 0, 4));
        return vxm_fail(ctx, VXM_ERR_BACKEND, "persistent blocks: a workgroup timed out waiting for data");
    }
    return VXM_OK;
}
