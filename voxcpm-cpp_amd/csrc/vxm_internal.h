// vxm_internal.h -- shared definitions of the gfx950 Q8_0 library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <string>

#include "../../include/vxm_q8.h"

#define VXM_QK 32
#define VXM_BLOCK_BYTES 34

struct vxm_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    int quant_variant = VXM_QUANT_X86;
    int path = VXM_PATH_AUTO;
    int n_cu = 256;
    // scratch for internally quantized activations (vxm_mul_mat_q8_0)
    void *act_buf = nullptr;
    size_t act_bytes = 0;
    // K-split partial tiles of the MFMA GEMM and its per-tile arrival counters
    // (zero between launches: the last workgroup of a tile resets its counter)
    void *split_buf = nullptr;
    size_t split_bytes = 0;
    int *split_cnt = nullptr;
    size_t split_ncnt = 0;
    // device word (in the error buffer) holding the tag of the last split
    // launch's partial words, advanced on the device before each split launch
    uint32_t *split_epoch_dev = nullptr;
    // device error word: set by a split fix-up whose partial words never
    // arrived (its output is NaN); vxm_sync reports and clears it
    int *dev_err = nullptr;
    bool split_launched = false;   // a split launch since the last vxm_sync check
    // K-split slices of the small-M GEMM behind the public matmul entries
    void *parts_buf = nullptr;
    size_t parts_bytes = 0;
    // this device's copy of the allocation-free matmul's scratch array (its
    // device address), or null with the reason in scratch_err
    unsigned char *scratch = nullptr;
    std::string scratch_err;
    // pinned, device-mapped host staging of small device-to-host copies (the
    // per-token hidden state): host and device addresses
    void *pin_out = nullptr;
    void *pin_out_dev = nullptr;
    unsigned pin_seq = 0;   // sequence number the copy kernel writes after the data
};

// Device layout of a Q8_0 matrix (n_rows x k).  The GGUF row of k/32 34-byte
// blocks is split so every kernel reads 16-byte aligned, fully coalesced
// spans:
//   qs : int8  [n][k]        quants, row-major
//   d  : fp16  [n][k/32]     scales, row-major (GEMM path, download)
//   dg : fp16  [n][k/32]     scales permuted for the GEMV path when
//                            k % 1024 == 0: element p*C + c of a row holds
//                            block c*32 + p (C = k/1024), so the two lanes
//                            that share block c*32 + p read their C scales
//                            from one contiguous span.
struct vxm_weight {
    int64_t n = 0, k = 0;
    int8_t *qs = nullptr;
    uint16_t *d = nullptr;
    uint16_t *dg = nullptr;
    // tile-blocked scales for the prefill GEMM (K % 256 == 0): 64-row groups
    // g < 2 ceil(n / 128), each [k/128 steps][64 rows][4 blocks]; rows past n are zero
    uint16_t *dt = nullptr;
    void *base = nullptr;   // single allocation holding qs, d, dg, dt
    size_t bytes = 0;
};

int vxm_fail(vxm_ctx *ctx, int code, const char *fmt, ...);

#define VXM_HIP(ctx, call)                                                              \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess) {                                                         \
            (void)hipGetLastError(); /* do not leave the error for the next check */    \
            return vxm_fail((ctx), VXM_ERR_BACKEND, "%s failed: %s (%s:%d)", #call,      \
                            hipGetErrorString(e_), __FILE__, __LINE__);                 \
        }                                                                               \
    } while (0)

#define VXM_CHECK_LAUNCH(ctx) VXM_HIP(ctx, hipGetLastError())

// ---- device helpers -------------------------------------------------------

__device__ __forceinline__ float vxm_h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

__device__ __forceinline__ uint16_t vxm_f2h(float f) {
    _Float16 v = (_Float16)f;   // v_cvt_f16_f32, round to nearest even
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// F32 -> BF16 -> F32 with round to nearest even (the rule of
// minicpm_bf16_round, src/minicpm4.c:39-42), on gfx950's v_cvt_pk_bf16_f32.
// Every non-NaN input rounds as the reference does; a NaN stays a quiet NaN
// (its payload bits may differ from the reference's).
__device__ __forceinline__ float vxm_bf16(float f) { return (float)(__bf16)f; }

// p = bf16(bf16(silu(bf16(g))) * bf16(u)): the SwiGLU product of vcpm_mlp
// (src/minicpm4.c:432-463) with the reference's BF16 rounding points.
__device__ __forceinline__ float vxm_swiglu(float g, float u) {
    const float gb = vxm_bf16(g);
    const float s = vxm_bf16(__fdiv_rn(gb, 1.0f + expf(-gb)));
    return vxm_bf16(s * vxm_bf16(u));
}

// Maximum over an aligned quad of lanes through DPP quad permutations (xor 1, then
// xor 2): every lane of the quad gets it, without an LDS round trip per step.  All four
// lanes must be active, as for a shuffle.
__device__ __forceinline__ float vxm_quad_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
}

// Q8_0 of one 32-value block held 8 per lane by four consecutive lanes (lane & 3
// = part) with the x86 rule (id = 127/amax, round half even) or the _ref rule;
// the lane with write_d set stores d.  write = false: compute (every lane of the
// four takes part in the amax exchange) but store nothing.
__device__ __forceinline__ void quant_block_4lanes(const float v[8], int variant, int8_t *q8,
                                                   uint16_t *dout, bool write_d, bool write = true) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = vxm_quad_max(amax);
    const float d = __fdiv_rn(amax, 127.0f);
    float id;
    if (variant == VXM_QUANT_X86) id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    else id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float q = variant == VXM_QUANT_X86 ? rintf(v[i] * id) : roundf(v[i] * id);
        q = fminf(fmaxf(q, -128.0f), 127.0f);
        const uint32_t b = (uint32_t)(uint8_t)(int8_t)(int)q;
        if (i < 4) lo |= b << (8 * i);
        else hi |= b << (8 * (i - 4));
    }
    if (!write) return;
    *(uint2 *)q8 = make_uint2(lo, hi);
    if (write_d) *dout = vxm_f2h(d);
}

// sum of 16 int8 x int8 products held as 4 packed dwords each
__device__ __forceinline__ int vxm_dot16(const int4 a, const int4 b, int acc) {
    acc = __builtin_amdgcn_sdot4(a.x, b.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

template <typename T>
__device__ __forceinline__ T vxm_shfl_xor(T v, int mask) {
    return __shfl_xor(v, mask, 64);
}

__device__ __forceinline__ float vxm_wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ float vxm_wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// ---- host-side launch helpers implemented per translation unit ------------
int vxm_launch_quantize(vxm_ctx *ctx, const float *x, int64_t M, int64_t K, int variant,
                        int8_t *xq, uint16_t *xd);
int vxm_launch_mul_mat(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd,
                       int64_t M, float *y);
// A matmul output held as n fp32 slices `stride` elements apart whose sum, added in
// slice order, is the product (the small-M GEMM's K splits, left for the consumer).
struct vxm_parts {
    const float *p;
    int n;
    int64_t stride;
};
__host__ __device__ inline vxm_parts vxm_one_part(const float *p) { return vxm_parts{p, 1, 0}; }

constexpr int VXM_SMALL_MAX_ROWS = 64;   // rows of x the small-M GEMM takes
constexpr int VXM_MAX_PARTS = 8;         // its K splits

// The product as up to max_parts slices of M x N at y, y + M*N, ...; *parts = the
// number written (1 unless the small-M GEMM splits K).
int vxm_launch_mul_mat_parts(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd,
                             int64_t M, float *y, int max_parts, int *parts);
bool vxm_launch_gate_up_swiglu(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                               int8_t *sq, uint16_t *sd, int variant, int *rc);
// What k_rope_kv does with the QKV projection's rows (BF16 rounding, NEOX rope
// of the pair-interleaved q and k rows, q out as fp32, k and v into the f16
// cache), done instead by the GEMM's epilogue.  q_out == nullptr: off.
struct vxm_qkv_epi {
    float *q_out;             // [M][nh*hd]
    uint16_t *kc, *vc;        // cache of the layer: [seg][nkv][cap][hd]
    const float2 *cs;         // rope (cos, sin) table [pos][hd/2]
    int64_t seg_stride;
    int nh, nkv, hd, pos0, S, no_rope, cap, cache_pos0;
};
bool vxm_launch_qkv_rope(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                         const vxm_qkv_epi &qe, int cs_rows, int *rc);
int vxm_ensure_act(vxm_ctx *ctx, size_t bytes);
// Finds the allocation-free matmul's scratch array on ctx's (current) device.
int vxm_scratch_setup(vxm_ctx *ctx);
int vxm_ensure_parts(vxm_ctx *ctx, size_t bytes);
int vxm_ensure_split(vxm_ctx *ctx, size_t bytes, size_t n_counters);
