// q8_matmul.hip -- activation quantization and the Q8_0 x Q8_0 matmul
// (ggml_mul_mat on GGUF Q8_0 weights) for gfx950.
//
// Semantics (ggml vec_dot_q8_0_q8_0, called from ggml_mul_mat at
// src/projections.h:24-29 and src/minicpm4.c:270-279,415,441-458):
//   y[m][n] = sum_b float(sumi[m][n][b]) * (float(d_w[n][b]) * float(d_x[m][b]))
//   sumi = sum over the 32 int8 pairs of block b (exact int32).
// Every kernel here forms exactly these per-block fp32 terms; only the order
// of the fp32 additions over b differs from ggml's (a tree over lanes).
#include <atomic>
#include <cstdint>
#include <mutex>

#include "vxm_internal.h"

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int dot16v(const v4i a, const v4i b, int acc) {
    acc = __builtin_amdgcn_sdot4(a.x, b.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

// Sum over the 32 lane pairs of a wave (lanes 2p and 2p+1 hold equal values).
__device__ __forceinline__ float pair_sum(float v) {
#pragma unroll
    for (int m = 2; m <= 32; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// ---------------------------------------------------------------------------
// Activation quantization: 8 lanes per 32-element block, 4 floats per lane.
// VARIANT 1 (x86 SIMD ggml): id = amax ? 127/amax : 0, q = rint(x*id).
// VARIANT 0 (quantize_row_q8_0_ref): id = d ? 1/d : 0, q = roundf(x*id).
// d = amax/127 is stored as fp16 (RNE).
// ---------------------------------------------------------------------------
template <int VARIANT>
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float *__restrict__ x, int64_t nblocks,
                                                       int8_t *__restrict__ xq,
                                                       uint16_t *__restrict__ xd) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = t >> 3;
    const int sub = threadIdx.x & 7;
    const bool live = blk < nblocks;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) v = *(const float4 *)(x + blk * 32 + sub * 4);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = vxm_quad_max(amax);   // xor 1, xor 2 on DPP; then the other quad of the 8
    amax = fmaxf(amax, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(amax), 0x141, 0xF, 0xF, false)));
    if (!live) return;
    const float d = __fdiv_rn(amax, 127.0f);
    float id;
    if (VARIANT == VXM_QUANT_X86) id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    else id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
    float q0, q1, q2, q3;
    if (VARIANT == VXM_QUANT_X86) {
        q0 = rintf(v.x * id); q1 = rintf(v.y * id); q2 = rintf(v.z * id); q3 = rintf(v.w * id);
        q0 = fminf(fmaxf(q0, -128.f), 127.f); q1 = fminf(fmaxf(q1, -128.f), 127.f);
        q2 = fminf(fmaxf(q2, -128.f), 127.f); q3 = fminf(fmaxf(q3, -128.f), 127.f);
    } else {
        q0 = roundf(v.x * id); q1 = roundf(v.y * id); q2 = roundf(v.z * id); q3 = roundf(v.w * id);
    }
    const uint32_t packed = ((uint32_t)(uint8_t)(int8_t)(int)q0) | ((uint32_t)(uint8_t)(int8_t)(int)q1 << 8) |
                            ((uint32_t)(uint8_t)(int8_t)(int)q2 << 16) | ((uint32_t)(uint8_t)(int8_t)(int)q3 << 24);
    *(uint32_t *)(xq + blk * 32 + sub * 4) = packed;
    if (sub == 0) xd[blk] = vxm_f2h(d);
}

int vxm_launch_quantize(vxm_ctx *ctx, const float *x, int64_t M, int64_t K, int variant,
                        int8_t *xq, uint16_t *xd) {
    const int64_t nblocks = M * (K / VXM_QK);
    if (nblocks == 0) return VXM_OK;
    const int threads = 256;
    const int64_t grid = (nblocks * 8 + threads - 1) / threads;
    if (variant == VXM_QUANT_X86)
        hipLaunchKernelGGL(k_quantize_q8_0<VXM_QUANT_X86>, dim3((unsigned)grid), dim3(threads), 0,
                           ctx->stream, x, nblocks, xq, xd);
    else
        hipLaunchKernelGGL(k_quantize_q8_0<VXM_QUANT_REF>, dim3((unsigned)grid), dim3(threads), 0,
                           ctx->stream, x, nblocks, xq, xd);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

// ---------------------------------------------------------------------------
// Decode GEMV, K % 1024 == 0 (C = K/1024 chunks of 1 KiB per row).
// One wave owns R consecutive rows.  In chunk c, lane l reads the 16 bytes at
// row*K + c*1024 + 16*l with one 128-bit load, so each load instruction of the
// wave covers one contiguous KiB.  Lane l therefore holds half (l & 1) of
// block c*32 + l/2; the two halves are summed with one lane exchange, giving
// the exact int32 block sum in both lanes of the pair.  The activation chunk a
// lane needs is the same for every row, so it stays in registers.
// All weight loads of the wave are issued before any arithmetic.
// DOTS = true writes the exact int32 block sums this kernel forms (after the
// lane-pair exchange) to dots[(m*N + n)*(K/32) + b] instead of y.
// ---------------------------------------------------------------------------
template <int C, int R, bool DOTS>
__device__ __forceinline__ void gemv_wave(const int8_t *__restrict__ qs, const uint16_t *__restrict__ dg,
                                          const int8_t *__restrict__ xq, const uint16_t *__restrict__ xd,
                                          float *__restrict__ y, int N, int M, int32_t *__restrict__ dots,
                                          int wave) {
    constexpr int K = C * 1024;
    constexpr int NB = K / 32;
    const int lane = threadIdx.x & 63;
    const int row0 = wave * R;
    if (row0 >= N) return;
    const int pair = lane >> 1;

    v4i wv[R][C];
    float dw[R][C];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = min(row0 + r, N - 1);
        const int8_t *wrow = qs + (int64_t)row * K + lane * 16;
#pragma unroll
        for (int c = 0; c < C; c++) wv[r][c] = __builtin_nontemporal_load((const v4i *)(wrow + c * 1024));
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = min(row0 + r, N - 1);
        const uint16_t *drow = dg + (int64_t)row * NB + pair * C;
#pragma unroll
        for (int c = 0; c < C; c++) dw[r][c] = vxm_h2f(__builtin_nontemporal_load(drow + c));
    }
    for (int m = 0; m < M; m++) {
        v4i xv[C];
        float xs[C];
        const int8_t *xrow = xq + (int64_t)m * K + lane * 16;
        const uint16_t *xdrow = xd + (int64_t)m * NB;
#pragma unroll
        for (int c = 0; c < C; c++) {
            xv[c] = *(const v4i *)(xrow + c * 1024);
            xs[c] = vxm_h2f(xdrow[c * 32 + pair]);
        }
        if (DOTS) {
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int c = 0; c < C; c++) {
                    int s = dot16v(wv[r][c], xv[c], 0);
                    s += __shfl_xor(s, 1, 64);
                    if ((lane & 1) == 0 && row0 + r < N) dots[((int64_t)m * N + row0 + r) * NB + c * 32 + pair] = s;
                }
            continue;
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            float a = 0.0f;
#pragma unroll
            for (int c = 0; c < C; c++) {
                int s = dot16v(wv[r][c], xv[c], 0);
                s += __shfl_xor(s, 1, 64);
                a += (float)s * (dw[r][c] * xs[c]);
            }
            acc[r] = a;
        }
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = pair_sum(acc[r]);
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; r++)
                if (row0 + r < N) y[(int64_t)m * N + row0 + r] = acc[r];
        }
    }
}

template <int C, int R, bool DOTS>
__global__ __launch_bounds__(256) void k_gemv_q8_0(const int8_t *__restrict__ qs,
                                                   const uint16_t *__restrict__ dg,
                                                   const int8_t *__restrict__ xq,
                                                   const uint16_t *__restrict__ xd, float *__restrict__ y,
                                                   int N, int M, int32_t *__restrict__ dots) {
    gemv_wave<C, R, DOTS>(qs, dg, xq, xd, y, N, M, dots, blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
}

// ---------------------------------------------------------------------------
// Many independent GEMVs of one K in one launch (the decode projections that
// share no dependency, or a stream of them).  A single GEMV of 13 MB cannot
// keep HBM busy: the launch ramp and the first loads' latency are a fixed
// ~2 us against 1.7 us of streaming at 8 TB/s.  Here the workgroups of all
// products form one grid; workgroup b runs wave (b - wg0) * 4 + w of the item
// with the largest wg0 <= b, with exactly the single GEMV's per-wave code, so
// every output is bit-identical to k_gemv_q8_0's.  The item table is a kernel
// argument (read with scalar loads through the kernarg pointer).
// ---------------------------------------------------------------------------
constexpr int kMultiMax = 64;
struct GemvItem {
    const int8_t *qs;
    const uint16_t *dg;
    const int8_t *xq;
    const uint16_t *xd;
    float *y;
    int n, wg0;
};
struct GemvBatch {
    GemvItem it[kMultiMax];
    int n_items;
};

template <int C, int R>
__global__ __launch_bounds__(256) void k_gemv_q8_0_multi(const GemvBatch b, int M) {
    const int bid = blockIdx.x;
    int lo = 0, hi = b.n_items - 1;
    while (lo < hi) {   // uniform binary search: the last item starting at or before bid
        const int mid = (lo + hi + 1) >> 1;
        if (b.it[mid].wg0 <= bid) lo = mid;
        else hi = mid - 1;
    }
    const GemvItem &t = b.it[lo];
    gemv_wave<C, R, false>(t.qs, t.dg, t.xq, t.xd, t.y, t.n, M, nullptr, (bid - t.wg0) * 4 + (threadIdx.x >> 6));
}

// ---------------------------------------------------------------------------
// Read-only stream (a measurement helper): n device ranges read once in one
// launch with the GEMV's loads, every 32-bit word XOR-folded into one word
// per wave.  It is the floor a launch of the same bytes can reach on this
// device.  Workgroup b reads 16 KiB of the range with the largest wg0 <= b;
// as in the GEMV, each wave reads 4 contiguous KiB (one KiB per load
// instruction, non-temporal) and ends with one plain store: atomics from every
// wave into shared words serialised (6.1 against 7.1 TB/s measured), and
// spreading a wave's loads over the workgroup's 16 KiB cost as much.
// ---------------------------------------------------------------------------
constexpr int kReadMax = 128;
constexpr int kReadWgBytes = 16384;
struct ReadRange {
    const uint4 *p;
    int64_t n16;   // 16-byte words
    int wg0;
};
struct ReadBatch {
    ReadRange r[kReadMax];
    int n;
};

__global__ __launch_bounds__(256) void k_stream_read(const ReadBatch b, uint32_t *__restrict__ sink) {
    const int bid = blockIdx.x;
    int lo = 0, hi = b.n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (b.r[mid].wg0 <= bid) lo = mid;
        else hi = mid - 1;
    }
    const ReadRange &t = b.r[lo];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t w0 = (int64_t)(bid - t.wg0) * (kReadWgBytes / 16) + wave * 256 + lane;
    v4i v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t w = w0 + i * 64;
        v[i] = w < t.n16 ? __builtin_nontemporal_load((const v4i *)(t.p + w)) : v4i{0, 0, 0, 0};
    }
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) x ^= (uint32_t)(v[i].x ^ v[i].y ^ v[i].z ^ v[i].w);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x ^= __shfl_xor(x, m, 64);
    if (lane == 0) sink[(int64_t)bid * 4 + wave] = x;
}

// ---------------------------------------------------------------------------
// Generic GEMV, any K % 32 == 0: one wave per row, lanes stride over the
// row's 16-byte half blocks (the two halves of a block sit in lanes 2p, 2p+1).
// DOTS = true writes the int32 block sums instead (as k_gemv_q8_0).
// ---------------------------------------------------------------------------
template <bool DOTS>
__global__ __launch_bounds__(256) void k_gemv_q8_0_generic(const int8_t *__restrict__ qs,
                                                           const uint16_t *__restrict__ d,
                                                           const int8_t *__restrict__ xq,
                                                           const uint16_t *__restrict__ xd,
                                                           float *__restrict__ y, int N, int K, int M,
                                                           int32_t *__restrict__ dots) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= N) return;
    const int nh = K / 16, nb = K / 32;
    const int8_t *wrow = qs + (int64_t)row * K;
    const uint16_t *drow = d + (int64_t)row * nb;
    for (int m = 0; m < M; m++) {
        const int8_t *xrow = xq + (int64_t)m * K;
        const uint16_t *xdrow = xd + (int64_t)m * nb;
        float acc = 0.0f;
        for (int h0 = 0; h0 < nh; h0 += 64) {
            const int h = h0 + lane;
            int s = 0;
            float sc = 0.0f;
            if (h < nh) {
                const v4i a = *(const v4i *)(wrow + h * 16);
                const v4i b = *(const v4i *)(xrow + h * 16);
                s = dot16v(a, b, 0);
                sc = vxm_h2f(drow[h >> 1]) * vxm_h2f(xdrow[h >> 1]);
            }
            s += __shfl_xor(s, 1, 64);
            if (DOTS) {
                if (h < nh && (h & 1) == 0) dots[((int64_t)m * N + row) * nb + (h >> 1)] = s;
                continue;
            }
            acc += (float)s * sc;
        }
        if (DOTS) continue;
        acc = pair_sum(acc);
        if (lane == 0) y[(int64_t)m * N + row] = acc;
    }
}


// ---------------------------------------------------------------------------
// Q8_0 x Q8_0 GEMM on int8 MFMA, for M rows of activations (prefill, CFM).
// gfx950's v_mfma_i32_32x32x32_i8 contracts K = 32 -- exactly one Q8_0
// block -- so one instruction yields the exact int32 block sums of a 32 x 32
// sub-tile.  Lane l supplies A row l % 32 and B row (weight row) l % 32, k
// half l / 32; result register v of lane l is row 8(v/4) + 4(l/32) + v%4,
// column l % 32.  Each lane then adds term = (float)sumi * (d_w * d_x) to its
// fp32 accumulators (one fused multiply-add per element and block).  That
// scale-and-add is the bound: per (element, block) it takes 3 VALU
// operations (convert, d_w * d_x, fma) against 1/1024 of a 32-cycle MFMA, so
// the VALU caps the int8 MFMA near 1/6 of its peak under exact per-block
// Q8_0 semantics.  The kernel is built so that the VALU is the only limit:
// * a wave owns a 32 (M) x 64 (N) strip -- two MFMAs per block share the A
//   operand and the 16 activation scales a lane needs, which halves the LDS
//   bytes per element (the scales would otherwise load the LDS as much as
//   the epilogue loads the VALU);
// * the MFMAs of block j+1 are issued before the epilogue of block j, so the
//   matrix core runs under the VALU work of the same wave;
// * blocks past the end of K are zero-filled in LDS and add exact zeros, so
//   the inner loop has no per-block branch.
//
// Workgroup: 512 threads (8 waves) on a 64 (M) x 64 (N) tile: wave w owns
// rows 32 (w % 2) .. +31 and K quarter w / 2 (blocks [q KS/4, (q+1) KS/4) of
// every KS-block LDS stage); the four quarters are added through LDS in
// quarter order at the end.  K moves through LDS KS blocks per stage,
// double-buffered through registers.  Tiles are ordered so that the M tiles
// sharing one weight tile run on one XCD (workgroups are dispatched round
// robin over the 8 XCDs): the weight tile is fetched into that XCD's L2 once.
//
// blockIdx.y = K split z (blocks [z*bps, (z+1)*bps)).  With splits > 1 each
// workgroup publishes its partial tile in part[z] as 64-bit words (launch
// epoch << 32 | fp32 bits, relaxed agent-scope stores: no fence, no L2
// writeback), then counts itself in cnt[tile].  The last workgroup of a tile
// to arrive resets the counter, reads every partial word until its tag shows
// this launch's epoch (a bounded wait: the words are already on their way),
// adds them in split order and writes y -- the result does not depend on the
// arrival order.  DOTS = true writes the int32 block sums to
// dots[(m*N + n)*nb + b] instead (debug; no scaling, no split).
// ---------------------------------------------------------------------------
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

// The 2 x 32 x 32 scale products of one block, d_x[m] * d_w[n], from the two
// fp16 scales in the low halves of a and b: lane l (block l / 32) supplies d_x
// of row l % 32 and d_w of column l % 32 in k-slot 0 of a two-block f16 outer
// product (v_mfma_f32_32x32x4_2b_f16), its other k-slots zero.  A product of
// two fp16 values has at most 22 significant bits, so it is exact in fp32
// (subnormal fp16 scales included), the same value the fp32 outer product of
// the converted scales gives, at a quarter of its matrix-core cycles.
__device__ __forceinline__ v32f scale_outer_f16(uint32_t a, uint32_t b) {
    const v2u av = {a & 0xffffu, 0u}, bv = {b & 0xffffu, 0u};
    return __builtin_amdgcn_mfma_f32_32x32x4f16(__builtin_bit_cast(v4h, av), __builtin_bit_cast(v4h, bv), v32f{}, 0,
                                                0, 0);
}
constexpr int GM = 64, GN = 64;              // output tile
constexpr int kGemmThreads = 512;
constexpr int kGemmSpin = 1 << 20;           // bound of the wait for one partial word
constexpr int kGemmMaxSplits = 4;

// KS = Q8_0 blocks per LDS stage (8 or 16).  LDS: 2 stages x (A + B) x 64 rows
// x (32 KS + 16) bytes + the scales; the K-quarter reduction reuses it.
template <int KS>
struct GemmLds {
    static constexpr int ROW = KS * 32 + 16;   // padded row (bytes) against bank conflicts
    int8_t a[2][GM * ROW];
    int8_t b[2][GN * ROW];
    float ad[2][KS][GM];
    float bd[2][KS][GN];
};

// The end of a tiled-GEMM workgroup, shared by both tiled kernels: acc holds
// this wave's 32 x 64 strip of K quarter kq (8 waves: wm = wave & 1, kq =
// wave >> 1).  The four quarters are added in order through LDS (red: 64 KiB,
// free), then y is written, or with K splits the partial tile is published
// as tagged words and the last workgroup of the tile adds the splits in order.
__device__ __forceinline__ void gemm_finish(float (&acc)[2][16], float *red, int *last_sh, float *__restrict__ y,
                                            uint64_t *__restrict__ part, int *__restrict__ cnt, int M, int N,
                                            int m0, int n0, int tm, int tn, int tiles_n, int z, int splits,
                                            const uint32_t *__restrict__ epoch_p, int *__restrict__ err) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, kq = wave >> 1;
    // the launch's split tag: a device word advanced before every split launch
    // (a scalar load; a graph replay reads the value its own prepare step wrote)
    const uint32_t epoch = splits > 1 ? *epoch_p : 0u;
    const int lr = lane & 31, lh = lane >> 5;
    // add the K quarters in order (quarter 0 + 1 + 2 + 3): every quarter hands its strips to
    // LDS, then quarter group kq finalizes result registers v = 4 kq .. 4 kq + 3 of both
    // strips (rows m0 + 32 wm + 8 kq + 4 lh + vv)
    // red: [4 quarters][2 strips][32 values][64 lanes]
#pragma unroll
    for (int v = 0; v < 16; v++) {
        red[((kq * 2 + wm) * 32 + v) * 64 + lane] = acc[0][v];
        red[((kq * 2 + wm) * 32 + 16 + v) * 64 + lane] = acc[1][v];
    }
    __syncthreads();
    float fin[2][4];
#pragma unroll
    for (int half = 0; half < 2; half++)
#pragma unroll
        for (int vv = 0; vv < 4; vv++) {
            const int v = 4 * kq + vv;
            float t = red[((0 * 2 + wm) * 32 + 16 * half + v) * 64 + lane];
#pragma unroll
            for (int q = 1; q < 4; q++) t = t + red[((q * 2 + wm) * 32 + 16 * half + v) * 64 + lane];
            fin[half][vv] = t;
        }
#pragma unroll
    for (int half = 0; half < 2; half++) {
        const int n = n0 + half * 32 + lr;
        if (n >= N) continue;
#pragma unroll
        for (int vv = 0; vv < 4; vv++) {
            const int m = m0 + wm * 32 + 8 * kq + 4 * lh + vv;
            if (m >= M) continue;
            const int64_t idx = (int64_t)m * N + n;
            if (splits == 1) {
                y[idx] = fin[half][vv];
            } else {
                const uint64_t word = ((uint64_t)epoch << 32) | __float_as_uint(fin[half][vv]);
                __hip_atomic_store(part + (int64_t)z * M * N + idx, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if (splits == 1) return;
    // split fix-up: count arrivals; the last one reduces the tagged partials in split order
    __syncthreads();
    const int tile = tm * tiles_n + tn;
    if (tid == 0) {
        const int prev = __hip_atomic_fetch_add(cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        (*last_sh) = prev == splits - 1;
        if ((*last_sh)) __hip_atomic_store(cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!(*last_sh)) return;
    // thread t reduces elements t + 512 j, j < 8, four at a time: all 4 x splits words
    // are requested before any tag is checked
    constexpr int EPT = GM * GN / kGemmThreads, EPP = 4;
    const int64_t MN = (int64_t)M * N;
#pragma unroll
    for (int j0 = 0; j0 < EPT; j0 += EPP) {
        uint64_t w[EPP][kGemmMaxSplits];
#pragma unroll
        for (int j = 0; j < EPP; j++) {
            const int e = tid + kGemmThreads * (j0 + j), m = m0 + e / GN, nn = n0 + e % GN;
            const bool live = m < M && nn < N;
            const int64_t i = live ? (int64_t)m * N + nn : 0;
#pragma unroll
            for (int zz = 0; zz < kGemmMaxSplits; zz++)
                w[j][zz] = (live && zz < splits)
                               ? __hip_atomic_load(part + zz * MN + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                               : ((uint64_t)epoch << 32);
        }
#pragma unroll
        for (int j = 0; j < EPP; j++) {
            const int e = tid + kGemmThreads * (j0 + j), m = m0 + e / GN, nn = n0 + e % GN;
            if (m >= M || nn >= N) continue;
            const int64_t i = (int64_t)m * N + nn;
            float s = 0.0f;
            bool stale = false;
#pragma unroll
            for (int zz = 0; zz < kGemmMaxSplits; zz++) {
                if (zz >= splits) break;
                uint64_t v = w[j][zz];
                for (int spin = 0; (uint32_t)(v >> 32) != epoch && spin < kGemmSpin; spin++) {
                    __builtin_amdgcn_s_sleep(1);
                    v = __hip_atomic_load(part + zz * MN + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                stale |= (uint32_t)(v >> 32) != epoch;
                const float p = __uint_as_float((uint32_t)v);
                s = zz ? s + p : p;
            }
            // a partial that never arrived: a visible NaN and the context's error word
            // (reported by vxm_sync), never a plausible-looking stale sum
            if (stale) {
                s = __builtin_nanf("");
                __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            y[i] = s;
        }
    }
}

template <int KS, bool DOTS>
#ifndef VXM_GEMM_PIPE
#define VXM_GEMM_PIPE 1
#endif
#ifndef VXM_GEMM_WAVES_PER_SIMD
#define VXM_GEMM_WAVES_PER_SIMD 2
#endif
__global__ __launch_bounds__(kGemmThreads, VXM_GEMM_WAVES_PER_SIMD) void k_gemm_q8_0_mfma(
    const int8_t *__restrict__ xq, const uint16_t *__restrict__ xd, const int8_t *__restrict__ wq,
    const uint16_t *__restrict__ wd, float *__restrict__ y, uint64_t *__restrict__ part, int *__restrict__ cnt,
    int32_t *__restrict__ dots, int M, int N, int K, int tiles_m, int tiles_n, int bps, int splits,
    const uint32_t *__restrict__ epoch_p, int *__restrict__ err) {
    static_assert(KS % 8 == 0, "a stage is a multiple of 8 blocks (64 KS scales per side = whole 512-thread rounds)");
    constexpr int ROW = GemmLds<KS>::ROW;
    constexpr int CH = KS / 4;                 // 16-byte chunks per thread per side and stage
    constexpr int NQ = KS / 4;                 // blocks per wave per stage
    __shared__ __align__(16) GemmLds<KS> L;
    __shared__ int last_sh;
    static_assert(sizeof(GemmLds<KS>) >= 4 * 2 * 64 * 32 * sizeof(float), "K-quarter reduction buffer");
    const int id = blockIdx.x, xcd = id % 8, k8 = id / 8;
    const int tn = (k8 / tiles_m) * 8 + xcd, tm = k8 % tiles_m;
    if (tn >= tiles_n) return;
    const int m0 = tm * GM, n0 = tn * GN;
    const int nb = K / 32;
    const int z = blockIdx.y;
    const int b0 = z * bps, b1 = min(nb, b0 + bps);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, kq = wave >> 1;

    // stage loader: chunk c = tid + 512 h of a side is row c / (2 KS), 16-byte piece
    // c % (2 KS) (block piece / 2, half piece % 2); scale c of the 2 x KS x 64 is side
    // c / (64 KS), block (c % (64 KS)) / 64, row c % 64.  All loads are unconditional
    // buffer loads: rows past M (N) fall outside the buffer's range and read as zeros;
    // blocks past b1 read real neighbours but get a zero scale at the store, so they
    // add exact zeros.  Scales stay fp16 bits until the store: converting them here
    // would make the compiler wait for the whole stage before the current MFMAs.
    const __amdgpu_buffer_rsrc_t ra_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)xq, (short)0, M * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)wq, (short)0, N * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t sa_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)xd, (short)0, M * nb * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t sb_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)wd, (short)0, N * nb * 2, 0x00020000);
    auto load = [&](int kb0, v4i (&ra)[CH], v4i (&rb)[CH], uint16_t (&sc)[CH]) {
#pragma unroll
        for (int h = 0; h < CH; h++) {
            const int c = tid + kGemmThreads * h, r = c / (2 * KS), pc = c % (2 * KS);
            const int koff = (kb0 + (pc >> 1)) * 32 + (pc & 1) * 16;
            ra[h] = __builtin_amdgcn_raw_buffer_load_b128(ra_rsrc, (m0 + r) * K + koff, 0, 0);
            rb[h] = __builtin_amdgcn_raw_buffer_load_b128(rb_rsrc, (n0 + r) * K + koff, 0, 0);
            // side is uniform: tid < 512 and 64 KS is a multiple of 512
            constexpr int kSidePer = 64 * KS / kGemmThreads;
            const bool side_b = h / kSidePer != 0;
            const int t = c % (64 * KS), sb = kb0 + t / 64, rr = t % 64;
            if (DOTS) sc[h] = 0;   // block sums only: scales are not read
            else if (!side_b) sc[h] = __builtin_amdgcn_raw_buffer_load_b16(sa_rsrc, ((m0 + rr) * nb + sb) * 2, 0, 0);
            else sc[h] = __builtin_amdgcn_raw_buffer_load_b16(sb_rsrc, ((n0 + rr) * nb + sb) * 2, 0, 0);
        }
    };
    auto store = [&](int buf, int kb0, const v4i (&ra)[CH], const v4i (&rb)[CH], const uint16_t (&sc)[CH]) {
#pragma unroll
        for (int h = 0; h < CH; h++) {
            const int c = tid + kGemmThreads * h, r = c / (2 * KS), pc = c % (2 * KS);
            *(v4i *)(L.a[buf] + r * ROW + pc * 16) = ra[h];
            *(v4i *)(L.b[buf] + r * ROW + pc * 16) = rb[h];
            constexpr int kSidePer = 64 * KS / kGemmThreads;
            const int t = c % (64 * KS);
            const float v = kb0 + t / 64 < b1 ? vxm_h2f(sc[h]) : 0.0f;
            if (h / kSidePer == 0) L.ad[buf][t / 64][t % 64] = v;
            else L.bd[buf][t / 64][t % 64] = v;
        }
    };

    float acc[2][16];
#pragma unroll
    for (int v = 0; v < 16; v++) acc[0][v] = acc[1][v] = 0.0f;
    v4i ra[CH], rb[CH];
    uint16_t sc[CH];
    load(b0, ra, rb, sc);
    store(0, b0, ra, rb, sc);
    __syncthreads();
    int buf = 0;
    const int lr = lane & 31, lh = lane >> 5;
    for (int kb0 = b0; kb0 < b1; kb0 += KS) {
        const bool more = kb0 + KS < b1;
        if (more) load(kb0 + KS, ra, rb, sc);
        const int8_t *arow = L.a[buf] + (wm * 32 + lr) * ROW + lh * 16 + kq * NQ * 32;
        const int8_t *brow0 = L.b[buf] + lr * ROW + lh * 16 + kq * NQ * 32;
        const int8_t *brow1 = brow0 + 32 * ROW;
        // per-lane scale operands of the outer product below: row scale of row lr of this
        // strip, column scale of column lr of tile half lh
        const float *adq = &L.ad[buf][kq * NQ][wm * 32 + lr];
        const float *bdq = &L.bd[buf][kq * NQ][32 * lh + lr];
        // epilogue of block j of this quarter: scale and add (or, DOTS, write the sums)
        auto epi = [&](const v16i &c0, const v16i &c1, int j) {
            if (DOTS) {
                const int kb = kb0 + kq * NQ + j;
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    const int n = n0 + half * 32 + lr;
                    const v16i &c = half ? c1 : c0;
#pragma unroll
                    for (int v = 0; v < 16; v++) {
                        const int m = m0 + wm * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                        if (kb < b1 && m < M && n < N) dots[((int64_t)m * N + n) * nb + kb] = c[v];
                    }
                }
                return;
            }
            // the 2 x 32 x 32 scale products d_x[m] * d_w[n] of this block come from one
            // two-block f32 outer product on the matrix core (block h = lanes 32h..32h+31
            // supply d_x of row lr and d_w of column 32h + lr) in the layout of c0 / c1;
            // each product of two fp16 values is exact in fp32, as the VALU product was
            const v32f sc = __builtin_amdgcn_mfma_f32_32x32x1f32(adq[j * GM], bdq[j * GN], v32f{}, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                acc[0][v] = __builtin_fmaf((float)c0[v], sc[v], acc[0][v]);
                acc[1][v] = __builtin_fmaf((float)c1[v], sc[16 + v], acc[1][v]);
            }
        };
        auto mma = [&](int j, v16i &c0, v16i &c1) {
            const v4i a = *(const v4i *)(arow + j * 32);
            c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, *(const v4i *)(brow0 + j * 32), v16i{}, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, *(const v4i *)(brow1 + j * 32), v16i{}, 0, 0, 0);
        };
        // next block's products first: the matrix core runs under this block's epilogue
        if (VXM_GEMM_PIPE) {
            v16i c0, c1;
            mma(0, c0, c1);
#pragma unroll(KS == 8 ? NQ : 1)
            for (int j = 0; j < NQ - 1; j++) {
                v16i n0v, n1v;
                mma(j + 1, n0v, n1v);
                epi(c0, c1, j);
                c0 = n0v;
                c1 = n1v;
            }
            epi(c0, c1, NQ - 1);
        } else {
#pragma unroll(KS == 8 ? NQ : 1)
            for (int j = 0; j < NQ; j++) {
                v16i c0, c1;
                mma(j, c0, c1);
                epi(c0, c1, j);
            }
        }
        if (more) {
            store(buf ^ 1, kb0 + KS, ra, rb, sc);
            buf ^= 1;
        }
        __syncthreads();
    }
    if (DOTS) return;
    gemm_finish(acc, (float *)&L, &last_sh, y, part, cnt, M, N, m0, n0, tm, tn, tiles_n, z, splits, epoch_p, err);
}

// ---------------------------------------------------------------------------
// Tiled Q8_0 x Q8_0 GEMM for prefill-sized M (> 64): one TM x TN output tile
// per workgroup (64 x 64, 64 x 128 or 128 x 128; 512 threads), every operand
// byte brought into LDS by direct HBM -> LDS loads (global_load_lds_dwordx4:
// lane l of an instruction writes 16 bytes at M0 + 16 l) into a ring of
// kTileSlots stages, three of them in flight while one is multiplied.
//
// Waves: wave w owns the 32-row strip sm = w % WM (WM = TM / 32) and the
// 64-column half h = (w / WM) % H of the tile (H = TN / 64) for K part
// kp = w / (WM H) (KP = 8 / (WM H) parts): PAIRS block pairs from block
// 2 PAIRS kp of every SB-block stage (SB = 8 / H for 64-row tiles, 4 for
// 128 x 128, whose waves take both pairs of a stage: twice the blocks between
// barriers, and half the operand bytes per output of 64 x 128).  A stage holds
// RB = 32 SB bytes of each operand row.  The K parts are added in order
// through LDS at the end.
//
// Per block a wave issues two v_mfma_i32_32x32x32_i8 (its 32 x 64 integer
// block sums) and one two-block f16 outer product (the 2 x 32 x 32 scale
// products d_x[m] d_w[n], exact in fp32: scale_outer_f16; against the fp32
// outer product of the converted scales it frees 48 of the 128 matrix-core
// cycles a wave spends per block, which the VALU work does not fully hide:
// gate/up at M = 512 55.6 -> 50.8 us, the 512-token prefill 4.11 -> 3.82 ms),
// then converts and accumulates:
// acc += float(sum) * scale.  The MFMAs of the next block are always issued
// before the conversion of the current one, so the matrix core runs under
// the VALU work and no result is waited for.
//
// Scales: the weight scales come from the tile-blocked copy dt (groups of 64
// rows x 4 blocks, 512 contiguous bytes; rows past N hold zeros), so a
// stage's TN x SB scales are one DMA instruction.  The activation scales of
// the tile's 64 rows over the split's K range are one LDS panel loaded with
// the first stages (rows of 2 (b1 - b0) bytes + 16 bytes of padding, which
// spreads the 32 rows a wave reads over the banks).  Operand rows past M or
// N load the clamped last row; past-N columns have zero scales and past-M
// rows are never stored.
//
// Operand rows are RB bytes in LDS with the 16-byte piece p of row r stored
// at p ^ swz(r) (R16 = RB / 16 pieces per row), so the 32 rows of an MFMA operand
// read fall on distinct banks; each DMA lane simply loads the piece its LDS
// position holds.  Each wave issues the same number of stage loads (wave 0
// one more: the weight scales), so its own in-order load counter tells when
// its part of a stage has landed; a barrier then publishes all parts and
// frees the slot of the stage before.
//
// K splits (blockIdx.y) end as in gemm_finish: tagged partial words, the last
// workgroup of a tile adds them in split order.  DOTS = true writes the int32
// block sums to dots[(m*N + n)*nb + b] instead (no scaling, no split fix-up).
// ---------------------------------------------------------------------------
// 1: the tile GEMM's scale products on the fp32 outer product of the converted
// scales (the former form, kept for comparison builds)
#ifndef VXM_TILE_F32_SCALES
#define VXM_TILE_F32_SCALES 0
#endif
constexpr int kTileSlots = 4;
constexpr int kTileThreads = 512;

#ifdef VXM_TILE_TRACE
// per-stage timestamps (s_memtime) of every wave of the first 256 workgroups:
// [workgroup][wave][stage < 62][top, compute done, loads landed, barrier passed];
// stage 62: entry, loop end, stores done
__device__ uint64_t vxm_tile_trace[256 * 8 * 64 * 4];
#define VXM_TILE_TS(st, k)                                                                         \
    do {                                                                                           \
        if (lane == 0 && blockIdx.x < 256 && blockIdx.y == 0 && (st) < 64)                         \
            vxm_tile_trace[((blockIdx.x * 8 + wave) * 64 + (st)) * 4 + (k)] = __builtin_amdgcn_s_memtime(); \
    } while (0)
#else
#define VXM_TILE_TS(st, k) \
    do {                   \
    } while (0)
#endif

template <int TM, int TN>
struct TileCfg {
    static constexpr int WM = TM / 32;                 // 32-row strips
    static constexpr int H = TN / 64;                  // 64-column halves
    static constexpr int KP = 8 / (WM * H);            // K parts
    static constexpr int SB = TM == 64 ? 8 / H : 4;    // blocks per stage
    static constexpr int PAIRS = SB / (2 * KP);        // block pairs of a wave per stage
    static constexpr int RB = SB * 32;                 // operand row bytes per stage
    static constexpr int R16 = RB / 16;                // 16-byte pieces per row
    // LDS position of piece p of row r: p ^ swz(r).  An operand read of 16 bytes per
    // lane is served 16 lanes (16 consecutive rows, one piece each) per 256 bytes of
    // banks; 128-byte rows (TN = 128) put two rows in that span, so the even rows and
    // the odd rows of any 16 must each take 8 distinct pieces, and any 8 consecutive
    // rows too (the same reads served 8 lanes per 128 bytes)
    static __device__ __forceinline__ int swz(int r) { return R16 == 8 ? (r & 7) ^ ((r >> 3) & 1) : r & 15; }
    static constexpr int ABytes = TM * RB, BBytes = TN * RB;
    static constexpr int Slot = ABytes + BBytes + 1024;   // + TN x SB weight scales
    static constexpr int LoadsAB = (ABytes + BBytes) / 1024 / 8;   // operand loads per wave and stage
    static constexpr int Red = KP * WM * H * 32 * 64;  // floats of the K-part reduction
    static constexpr int MaxBps = TM == 64 ? 192 : 96;  // K blocks per split (activation scale panel)
    static_assert((TM == 64 || TM == 128) && (TN == 64 || TN == 128) && WM * H * KP == 8, "eight waves");
    static_assert(PAIRS >= 1 && SB == 2 * KP * PAIRS, "every wave takes whole block pairs of a stage");
    static_assert((ABytes + BBytes) % 8192 == 0, "operand loads must split evenly over the waves");
    static_assert(Red * 4 <= kTileSlots * Slot, "the reduction reuses the ring");
};

static size_t tile_lds_bytes(int tm, int tn, int bps) {
    const int slot = tm == 128 ? TileCfg<128, 128>::Slot : tn == 128 ? TileCfg<64, 128>::Slot : TileCfg<64, 64>::Slot;
    return (size_t)kTileSlots * slot + 1024 * (size_t)(tm / 64) * (size_t)(bps / 8 + 1);
}

static int tile_max_bps(int tm) { return tm == 128 ? TileCfg<128, 128>::MaxBps : TileCfg<64, 64>::MaxBps; }

// 16 bytes per lane from src into LDS at lds_base + 16 lane.
__device__ __forceinline__ void lds_dma16(uint32_t lds_base, const void *src) {
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_base);
    uint32_t saved_m0;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %2, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved_m0)
        : "s"(m0v), "v"(src)
        : "memory");
}

// 16 bytes per lane of lanes 0..7 only (exec = 0xff), into LDS at lds_base + 16 lane.
__device__ __forceinline__ void lds_dma16_8(uint32_t lds_base, const void *src) {
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(lds_base);
    uint64_t saved;
    uint32_t saved_m0;
    asm volatile(
        "s_mov_b32 %1, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_mov_b64 %0, exec\n\t"
        "s_mov_b64 exec, 0xff\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %3, off\n\t"
        "s_mov_b64 exec, %0\n\t"
        "s_mov_b32 m0, %1"
        : "=&s"(saved), "=&s"(saved_m0)
        : "s"(m0v), "v"(src)
        : "memory", "scc");
}

// Two tagged 64-bit words in one 16-byte store that bypasses the non-coherent
// caches (sc1): each 8-byte half is written as an agent-scope relaxed atomic
// store of that word would be (the same instruction's 8-byte form), so a
// reader checking each word's tag sees the old or the new word.  p is 16-byte
// aligned.  A store of more than 8 bytes reads its data registers after
// issue, and the compiler's hazard checks do not see into the asm: the s_nop
// keeps the next instructions from overwriting them first.
__device__ __forceinline__ void store_words2_sc1(uint64_t *p, uint64_t a, uint64_t b) {
    typedef unsigned v4u_t __attribute__((ext_vector_type(4)));
    const v4u_t v = {(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(p), "v"(v) : "memory");
}

template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// wait until at most `stages` later stages of this wave's loads (L per stage) are in flight
template <int L>
__device__ __forceinline__ void vm_wait_stages(int stages) {
    if (stages >= 2) vm_wait<2 * L>();
    else if (stages == 1) vm_wait<L>();
    else vm_wait<0>();
}

__device__ __forceinline__ void ring_barrier() {   // orders LDS only: loads in flight stay in flight
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int TM, int TN, bool DOTS>
__global__ __launch_bounds__(kTileThreads, 1) void k_gemm_q8_0_tile(
    const int8_t *__restrict__ xq, const uint16_t *__restrict__ xd, const int8_t *__restrict__ wq,
    const uint16_t *__restrict__ wt, float *__restrict__ y, uint64_t *__restrict__ part, int *__restrict__ cnt,
    int32_t *__restrict__ dots, int M, int N, int K, int tiles_m, int tiles_n, int bps, int splits, int n_base,
    const uint32_t *__restrict__ epoch_p, int *__restrict__ err, int8_t *__restrict__ sq, uint16_t *__restrict__ sd,
    int variant,
    const vxm_qkv_epi qe) {
    using C = TileCfg<TM, TN>;
    extern __shared__ __attribute__((aligned(16))) int8_t ring[];
    __shared__ int last_sh;
    const int id = blockIdx.x, xcd = id % 8, k8 = id / 8;
    const int tn = (k8 / tiles_m) * 8 + xcd, tm = k8 % tiles_m;
    if (tn >= tiles_n) return;
    const int m0 = tm * TM, n0 = n_base + tn * TN;   // n_base: this launch's first column (a multiple of 128)
    const int nb = K / 32, nb4 = nb / 4;
    const int z = blockIdx.y;
    const int b0 = z * bps, b1 = min(nb, b0 + bps);
    const int ns = (b1 - b0) / C::SB;   // whole stages
    const int P = (b1 - b0) / 8;        // 16-byte pieces of a panel row
    const int pitch = 16 * (P + 1);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sm = wave % C::WM, h = (wave / C::WM) % C::H, kp = wave / (C::WM * C::H);
    const int lr = lane & 31, lh = lane >> 5;
    const int j0 = 2 * C::PAIRS * kp;   // this wave's first block of a stage
    const uint32_t ring_lds = (uint32_t)(uintptr_t)ring;
    const int8_t *panel = ring + kTileSlots * C::Slot;
    VXM_TILE_TS(62, 0);

    // activation scale panel: piece f = 64 i + lane of instruction i is row f / (P + 1),
    // piece f % (P + 1) (the last piece of a row is padding and loads a valid dummy)
    for (int i = wave; i < (TM / 64) * (P + 1); i += 8) {
        const int f = 64 * i + lane, row = f / (P + 1), pc = f % (P + 1);
        const int r = min(m0 + row, M - 1), q = pc < P ? pc : 0;
        lds_dma16(ring_lds + kTileSlots * C::Slot + 1024 * i, xd + (int64_t)r * nb + b0 + 8 * q);
    }
    // this wave's loads of stage st: operand instruction i < LoadsAB is instruction
    // wave * LoadsAB + i of the stage's A | B rows; i == LoadsAB is the wave's
    // eighth (128 bytes, 8 lanes) of the TN x SB weight scales
    auto issue_one = [&](int st, int i) {
        const uint32_t base = ring_lds + (st % kTileSlots) * C::Slot;
        const int kb0 = b0 + C::SB * st;
        if (i < C::LoadsAB) {
            const int q = wave * C::LoadsAB + i;
            const int rr = q * (64 / C::R16) + lane / C::R16;   // row of A (< TM) then B
            const int pg = (lane % C::R16) ^ C::swz(rr);
            const int8_t *src = rr < TM ? xq + (int64_t)min(m0 + rr, M - 1) * K
                                        : wq + (int64_t)min(n0 + rr - TM, N - 1) * K;
            lds_dma16(base + q * 1024, src + kb0 * 32 + pg * 16);
        } else {
            // 16-byte piece p = 8 wave + lane of the stage's 1 KiB: 64-row group
            // p >> 5 (TN = 128) or 4-block step p >> 5 (TN = 64), rows 2 (p & 31) ..
            const int p = 8 * wave + (lane & 7), g = n0 / 64 + (C::H == 2 ? p >> 5 : 0),
                      c = C::H == 2 ? 0 : p >> 5;
            lds_dma16_8(base + C::ABytes + C::BBytes + 128 * wave,
                        wt + ((int64_t)g * nb4 + kb0 / 4 + c) * 256 + (p & 31) * 8);
        }
    };
    auto issue = [&](int st) {
#pragma unroll
        for (int i = 0; i <= C::LoadsAB; i++) issue_one(st, i);
    };

    float acc[2][16];
#pragma unroll
    for (int v = 0; v < 16; v++) acc[0][v] = acc[1][v] = 0.0f;
    // LDS offsets of this lane's operand rows and scales
    const int ar = 32 * sm + lr, br0 = 64 * h + lr, br1 = br0 + 32, sr = 64 * h + 32 * lh + lr;
    const int a_off = ar * C::RB, b0_off = C::ABytes + br0 * C::RB, b1_off = C::ABytes + br1 * C::RB;
    // (pair pr of the stage: blocks j0 + 2 pr, j0 + 2 pr + 1, 4 bytes further in the TN = 128 layout,
    // the only one with more than one pair)
    const int s_off = C::ABytes + C::BBytes +
                      (C::H == 2 ? (sr >> 6) * 512 + (sr & 63) * 8 + j0 * 2 : (j0 >> 2) * 512 + sr * 8 + (j0 & 3) * 2);
    static_assert(C::PAIRS == 1 || C::H == 2, "pairs past the first sit in the 4-block rows of the TN = 128 scales");
    const int8_t *pa_row = panel + ar * pitch;

    // operands of block j of a stage: this lane's 16 bytes of its A row and of its two B rows
    auto operands = [&](const int8_t *sb, int j, v4i &a, v4i &w0, v4i &w1) {
        const int pc = 2 * j + lh;
        a = *(const v4i *)(sb + a_off + ((pc ^ C::swz(ar)) * 16));
        w0 = *(const v4i *)(sb + b0_off + ((pc ^ C::swz(br0)) * 16));
        w1 = *(const v4i *)(sb + b1_off + ((pc ^ C::swz(br1)) * 16));
    };
    // conversion of values v0 <= v < v1 of a block's sums (both column halves)
    auto epi_part = [&](const v16i &c0, const v16i &c1, const v32f &sc, int v0, int v1) {
#pragma unroll
        for (int v = v0; v < v1; v++) {
            acc[0][v] = __builtin_fmaf((float)c0[v], sc[v], acc[0][v]);
            acc[1][v] = __builtin_fmaf((float)c1[v], sc[16 + v], acc[1][v]);
        }
    };
    auto dots_out = [&](const v16i &c0, const v16i &c1, int kb) {
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const int n = n0 + 64 * h + 32 * half + lr;
            const v16i &c = half ? c1 : c0;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = m0 + 32 * sm + 8 * (v >> 2) + 4 * lh + (v & 3);
                if (m < M && n < N) dots[((int64_t)m * N + n) * nb + kb] = c[v];
            }
        }
    };

    constexpr int L = C::LoadsAB + 1;   // loads per wave and stage
#pragma unroll
    for (int st = 0; st < kTileSlots - 1; st++)
        if (st < ns) issue(st);
    vm_wait_stages<L>(min(2, ns - 1));
    ring_barrier();   // the panel and stage 0 are in LDS

    // Block pipeline: X = the first block of a pair, Y = its second (a wave takes
    // PAIRS pairs of every stage).  Each MFMA is followed by a third of the
    // conversion of the other block -- Y of the pair before while X's MFMAs run, X
    // while Y's run -- so the matrix core works under the VALU and no conversion
    // waits for a product (scheduling fences keep that order).  The blocks are
    // converted in K order.  Y starts as zeros, whose conversion adds nothing.
    // The loads of stage st + 3 go out first, into the slot that stage st - 1
    // freed at the last barrier.
    v16i xc0, xc1, yc0 = {}, yc1 = {};
    v32f xs, ys = {};
#define VXM_FENCE __builtin_amdgcn_sched_barrier(0)
    for (int st = 0; st < ns; st++) {
        VXM_TILE_TS(st, 0);
        const int8_t *sb = ring + (st % kTileSlots) * C::Slot;
        uint32_t pa[C::PAIRS], pw[C::PAIRS];
#pragma unroll
        for (int pr = 0; pr < C::PAIRS; pr++) {
            pa[pr] = *(const uint32_t *)(pa_row + 2 * (C::SB * st + j0 + 2 * pr));
            pw[pr] = *(const uint32_t *)(sb + s_off + 4 * pr);
        }
        const bool more = st + kTileSlots - 1 < ns;
        if (more) issue(st + kTileSlots - 1);
        v4i xa[C::PAIRS], xw0[C::PAIRS], xw1[C::PAIRS], ya[C::PAIRS], yw0[C::PAIRS], yw1[C::PAIRS];
#pragma unroll
        for (int pr = 0; pr < C::PAIRS; pr++) {
            operands(sb, j0 + 2 * pr, xa[pr], xw0[pr], xw1[pr]);
            operands(sb, j0 + 2 * pr + 1, ya[pr], yw0[pr], yw1[pr]);
        }
#pragma unroll
        for (int pr = 0; pr < C::PAIRS; pr++) {
            if (DOTS) {
                const int kb = b0 + C::SB * st + j0 + 2 * pr;
                xc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[pr], xw0[pr], v16i{}, 0, 0, 0);
                xc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[pr], xw1[pr], v16i{}, 0, 0, 0);
                yc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(ya[pr], yw0[pr], v16i{}, 0, 0, 0);
                yc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(ya[pr], yw1[pr], v16i{}, 0, 0, 0);
                dots_out(xc0, xc1, kb);
                dots_out(yc0, yc1, kb + 1);
            } else {
#if VXM_TILE_F32_SCALES
                const float dax = vxm_h2f((uint16_t)pa[pr]), dwx = vxm_h2f((uint16_t)pw[pr]);
                const float day = vxm_h2f((uint16_t)(pa[pr] >> 16)), dwy = vxm_h2f((uint16_t)(pw[pr] >> 16));
                VXM_FENCE;
                xs = __builtin_amdgcn_mfma_f32_32x32x1f32(dax, dwx, v32f{}, 0, 0, 0);
#else
                VXM_FENCE;
                xs = scale_outer_f16(pa[pr], pw[pr]);
#endif
                VXM_FENCE;
                epi_part(yc0, yc1, ys, 0, 6);
                VXM_FENCE;
                xc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[pr], xw0[pr], v16i{}, 0, 0, 0);
                VXM_FENCE;
                epi_part(yc0, yc1, ys, 6, 11);
                VXM_FENCE;
                xc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[pr], xw1[pr], v16i{}, 0, 0, 0);
                VXM_FENCE;
                epi_part(yc0, yc1, ys, 11, 16);
                VXM_FENCE;
#if VXM_TILE_F32_SCALES
                ys = __builtin_amdgcn_mfma_f32_32x32x1f32(day, dwy, v32f{}, 0, 0, 0);
#else
                ys = scale_outer_f16(pa[pr] >> 16, pw[pr] >> 16);
#endif
                VXM_FENCE;
                epi_part(xc0, xc1, xs, 0, 6);
                VXM_FENCE;
                yc0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(ya[pr], yw0[pr], v16i{}, 0, 0, 0);
                VXM_FENCE;
                epi_part(xc0, xc1, xs, 6, 11);
                VXM_FENCE;
                yc1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(ya[pr], yw1[pr], v16i{}, 0, 0, 0);
                VXM_FENCE;
                epi_part(xc0, xc1, xs, 11, 16);
                VXM_FENCE;
                // the sums are needed here, not after the stage wait: keep the conversions
                // in this block (otherwise they sink past the barrier, behind the MFMAs)
#pragma unroll
                for (int v = 0; v < 16; v++) asm volatile("" ::"v"(acc[0][v]), "v"(acc[1][v]));
            }
        }
        VXM_TILE_TS(st, 1);
        if (st + 1 < ns) {
            // stage st + 1 has landed once at most the stages after it remain in flight
            vm_wait_stages<L>(min(2, ns - 2 - st));
            VXM_TILE_TS(st, 2);
            ring_barrier();   // every wave's part of stage st + 1 is visible; slot st is free
            VXM_TILE_TS(st, 3);
        }
    }
#undef VXM_FENCE
    if (DOTS) return;
    if (ns > 0) epi_part(yc0, yc1, ys, 0, 16);
    VXM_TILE_TS(62, 1);

    // K parts in order through LDS: red[kp][wave of the part][32 values][64 lanes]
    __syncthreads();   // every wave is done with the ring
    float *red = (float *)ring;
    constexpr int WP = C::WM * C::H;           // waves of one K part
    const int wi = wave % WP;                  // = sm + WM h
#pragma unroll
    for (int v = 0; v < 16; v++) {
        red[((kp * WP + wi) * 32 + v) * 64 + lane] = acc[0][v];
        red[((kp * WP + wi) * 32 + 16 + v) * 64 + lane] = acc[1][v];
    }
    __syncthreads();
    constexpr int PER = WP * 32 * 64;          // floats of one K part
    if (sq) {
        // gate/up with SwiGLU and Q8_0 (one split): columns 2n and 2n + 1 are gate n and
        // up n, so the 64 columns of a row in one wave half are one 32-value block of
        // p = vxm_swiglu(gate, up).  Four threads per (row, half): 16 columns each
        const int F = N / 2;
        // whole waves take the same iterations (4 TM H is a multiple of 64), so the four
        // lanes of a block always run together
        for (int tq = tid; tq < 4 * TM * C::H; tq += kTileThreads) {
            const int bi = tq >> 2, part = tq & 3, mi = bi % TM, g = bi / TM;
            const int r32 = mi & 31;
            const int v = 16 * (part >> 1) + 4 * (r32 >> 3) + (r32 & 3);
            const int f = (((mi >> 5) + C::WM * g) * 32 + v) * 64 + 32 * ((r32 >> 2) & 1) + 16 * (part & 1);
            float gu[16];
#pragma unroll
            for (int c4 = 0; c4 < 4; c4++) {
                float4 t = *(const float4 *)(red + f + 4 * c4);
#pragma unroll
                for (int q = 1; q < C::KP; q++) {
                    const float4 u = *(const float4 *)(red + q * PER + f + 4 * c4);
                    t.x = t.x + u.x; t.y = t.y + u.y; t.z = t.z + u.z; t.w = t.w + u.w;
                }
                gu[4 * c4] = t.x; gu[4 * c4 + 1] = t.y; gu[4 * c4 + 2] = t.z; gu[4 * c4 + 3] = t.w;
            }
            float pv[8];
#pragma unroll
            for (int e = 0; e < 8; e++) pv[e] = vxm_swiglu(gu[2 * e], gu[2 * e + 1]);
            const int m = m0 + mi;
            const bool live = m < M && n0 + 64 * g < N;   // N % 64 == 0: a half is in or out
            const int64_t o = live ? (int64_t)m * F + (n0 + 64 * g) / 2 + 8 * part : 0;
            // rows past M and a half past N quantize too (the amax exchange needs all four
            // lanes) but store nothing
            quant_block_4lanes(pv, variant, sq + o, sd + o / 32, part == 0, live);
        }
        return;
    }
    // four neighbouring lanes = four neighbouring columns of one row: 16-byte LDS
    // reads and (N % 4 == 0, the usual case) 16-byte stores
    const int64_t MN = (int64_t)M * N;
    // the launch's split tag (device word, advanced before every split launch)
    const uint32_t epoch = splits > 1 ? *epoch_p : 0u;
    const bool vec = (N & 3) == 0 && splits == 1 && ((uintptr_t)y & 15) == 0;
#pragma unroll 2
    for (int f = 4 * tid; f < PER; f += 4 * kTileThreads) {
        float4 s = *(const float4 *)(red + f);
#pragma unroll
        for (int q = 1; q < C::KP; q++) {
            const float4 t = *(const float4 *)(red + q * PER + f);
            s.x = s.x + t.x; s.y = s.y + t.y; s.z = s.z + t.z; s.w = s.w + t.w;
        }
        const int fw = f >> 11, v = (f >> 6) & 31, fl = f & 63;
        const int vv = v & 15;
        const int m = m0 + 32 * (fw % C::WM) + 8 * (vv >> 2) + 4 * (fl >> 5) + (vv & 3);
        const int n = n0 + 64 * (fw / C::WM) + 32 * (v >> 4) + (fl & 31);
        if (m >= M) continue;
        if (qe.q_out) {
            // k_rope_kv on columns n .. n + 3 of token m (one split, N % 4 == 0): two
            // rope pairs of q or k (rows 2i, 2i + 1 of a head are dims i, i + hd/2),
            // or four values of v
            const int qd = qe.nh * qe.hd, kvd = qe.nkv * qe.hd, half = qe.hd / 2;
            const int seg = m / qe.S, ti = m % qe.S, cpos = qe.cache_pos0 + ti;
            const float sv[4] = {s.x, s.y, s.z, s.w};
            if (n < qd + kvd) {
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                    const int c = n + e;
                    const bool isq = c < qd;
                    const int cc = isq ? c : c - qd, head = cc / qe.hd, i = (cc % qe.hd) / 2;
                    const float x0 = vxm_bf16(sv[e]), x1 = vxm_bf16(sv[e + 1]);
                    float y0 = x0, y1 = x1;
                    if (!qe.no_rope) {
                        const float2 r = qe.cs[(int64_t)(qe.pos0 + ti) * half + i];
                        y0 = vxm_bf16(x0 * r.x - x1 * r.y);
                        y1 = vxm_bf16(x0 * r.y + x1 * r.x);
                    }
                    if (isq) {
                        float *qo = qe.q_out + (int64_t)m * qd + head * qe.hd;
                        qo[i] = y0;
                        qo[i + half] = y1;
                    } else {
                        uint16_t *kd = qe.kc + seg * qe.seg_stride + ((int64_t)head * qe.cap + cpos) * qe.hd;
                        kd[i] = vxm_f2h(y0);
                        kd[i + half] = vxm_f2h(y1);
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int c = n + e - qd - kvd, kh = c / qe.hd, dd = c % qe.hd;
                    qe.vc[seg * qe.seg_stride + ((int64_t)kh * qe.cap + cpos) * qe.hd + dd] = vxm_f2h(vxm_bf16(sv[e]));
                }
            }
            continue;
        }
        const int64_t idx = (int64_t)m * N + n;
        if (vec && n + 3 < N) {
            *(float4 *)(y + idx) = s;
            continue;
        }
        if (splits > 1 && (N & 3) == 0 && n + 3 < N) {
            // four partial words as two 16-byte stores (idx and z M N are even: aligned)
            const uint64_t tag = (uint64_t)epoch << 32;
            uint64_t *dst = part + (int64_t)z * MN + idx;
            store_words2_sc1(dst, tag | __float_as_uint(s.x), tag | __float_as_uint(s.y));
            store_words2_sc1(dst + 2, tag | __float_as_uint(s.z), tag | __float_as_uint(s.w));
            continue;
        }
        const float sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if (n + e >= N) break;
            if (splits == 1) {
                y[idx + e] = sv[e];
            } else {
                const uint64_t word = ((uint64_t)epoch << 32) | __float_as_uint(sv[e]);
                __hip_atomic_store(part + (int64_t)z * MN + idx + e, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    VXM_TILE_TS(62, 2);
    if (splits == 1) return;
    // split fix-up: count arrivals; the last one adds the tagged partials in split order
    __syncthreads();
    const int tile = tm * tiles_n + tn;
    if (tid == 0) {
        const int prev = __hip_atomic_fetch_add(cnt + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_sh = prev == splits - 1;
        if (last_sh) __hip_atomic_store(cnt + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last_sh) return;
    // thread t adds elements t + 512 j, EPR at a time: every word of a round (EPR x splits)
    // is requested before any tag is checked, so a round costs one memory round trip
    constexpr int EPT = TM * TN / kTileThreads, EPR = 8;
    static_assert(EPT % EPR == 0, "whole rounds");
    bool stale = false;
    for (int j0 = 0; j0 < EPT; j0 += EPR) {
        uint64_t w[EPR][kGemmMaxSplits];
#pragma unroll
        for (int j = 0; j < EPR; j++) {
            const int e = tid + kTileThreads * (j0 + j), m = m0 + e / TN, n = n0 + e % TN;
            const bool live = m < M && n < N;
            const int64_t i = live ? (int64_t)m * N + n : 0;
#pragma unroll
            for (int zz = 0; zz < kGemmMaxSplits; zz++)
                w[j][zz] = (live && zz < splits)
                               ? __hip_atomic_load(part + zz * MN + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                               : ((uint64_t)epoch << 32);
        }
#pragma unroll
        for (int j = 0; j < EPR; j++) {
            const int e = tid + kTileThreads * (j0 + j), m = m0 + e / TN, n = n0 + e % TN;
            if (m >= M || n >= N) continue;
            const int64_t i = (int64_t)m * N + n;
            float s = 0.0f;
            bool st_e = false;
#pragma unroll
            for (int zz = 0; zz < kGemmMaxSplits; zz++) {
                if (zz >= splits) break;
                uint64_t v = w[j][zz];
                for (int spin = 0; (uint32_t)(v >> 32) != epoch && spin < kGemmSpin; spin++) {
                    __builtin_amdgcn_s_sleep(1);
                    v = __hip_atomic_load(part + zz * MN + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                st_e |= (uint32_t)(v >> 32) != epoch;
                const float p = __uint_as_float((uint32_t)v);
                s = zz ? s + p : p;
            }
            // a partial that never arrived: a visible NaN and the context's error word
            y[i] = st_e ? __builtin_nanf("") : s;
            stale |= st_e;
        }
    }
    if (stale) __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Small-M MFMA GEMM (M <= 64: the CFM batch of both CFG branches, LocEnc
// patches, short prompts).  Each weight byte feeds at most 64 products here,
// so the weight stream sets the time: every weight byte is loaded once, with
// 16-byte loads, straight into MFMA operand registers; the activations (a few
// KiB per K stage) are staged once per workgroup in LDS and shared by its
// waves.
//
// v_mfma_i32_16x16x32_i8 takes one Q8_0 block: A = 16 weight rows x 32 bytes,
// B = 32 x 16 activation rows; lane group q = l / 16 supplies 8 bytes of the
// block for row r = l % 16 and receives the sums D[4q + v][r], v < 4.  The
// products only need A and B to give a lane group the same 8 bytes of the
// block.  Weights: lane (q, r) loads 16 bytes at byte 16q of a block pair of
// row r (q < 2: first block, halves q; q >= 2: second block, halves q - 2);
// one permlane32 swap per dword exchanges the high 8 bytes of lanes 0-31 with
// the low 8 bytes of lanes 32-63, after which the low 8 bytes of lane group
// q hold bytes off(q) = 16 (q & 1) + 8 (q >> 1) of the first block and the
// high 8 bytes the same bytes of the second block.  Activations are written
// to LDS with the 8-byte pieces of each block in off(q) order, so lane group
// q reads its piece at 8q; the LDS row pitch is 16 mod 256 bytes, which maps
// each half-wave's 8-byte reads onto distinct banks.
//
// Workgroup = 4 waves, wave w owning weight rows n0 + 16w .. +15, over the K
// blocks [z*bps, (z+1)*bps) in stages of kSmallStage blocks; split z writes
// its partial product to y + z*M*N (the consumer adds the slices in order).
// Rows past M read as zeros (outside the buffer range) and are not written.
// DOTS = true writes the int32 block sums of the MFMAs to dots[(m*N + n)*nb + b]
// instead (every split its own blocks; no scaling, no epilogue).
// ---------------------------------------------------------------------------
constexpr int kSmallStage = 8;                        // K blocks per LDS stage
constexpr int kSmallPitch = kSmallStage * 32 + 16;    // LDS bytes per activation row
constexpr int kSmallRG = 4;                           // 16-row groups (waves) per workgroup

__device__ __forceinline__ float half_at(const v4i &v, int j) {
    const uint32_t w = (uint32_t)v[j >> 1];
    return vxm_h2f((uint16_t)((j & 1) ? (w >> 16) : (w & 0xffffu)));
}

__device__ __forceinline__ long pack64(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

template <int MT, int KG, bool DOTS>
__global__ __launch_bounds__(64 * kSmallRG * KG) void k_gemm_q8_0_small(const int8_t *__restrict__ xq,
                                                                   const uint16_t *__restrict__ xd,
                                                                   const int8_t *__restrict__ wq,
                                                                   const uint16_t *__restrict__ wd,
                                                                   float *__restrict__ y, int M, int N, int K,
                                                                   int bps, int8_t *__restrict__ sq,
                                                                   uint16_t *__restrict__ sd, int variant,
                                                                   int32_t *__restrict__ dots) {
    // KG groups of kSmallRG waves split the workgroup's K range in halves (KG = 2) and add
    // their partial products through LDS at the end; NT = threads per group
    constexpr int SB = kSmallStage, ROWS = 16 * MT, NT = 64 * kSmallRG;
    __shared__ __align__(16) int8_t xs_all[KG][ROWS * kSmallPitch];
    __shared__ float xds_all[KG][ROWS][SB + 1];
    const int nb = K / 32;
    const int g = blockIdx.x, z = blockIdx.y;
    // row tile of x: rows m0 .. m0 + Mt - 1 (one tile unless M > 16 MT)
    const int m0 = blockIdx.z * ROWS, Mt = min(ROWS, M - m0);
    xq += (int64_t)m0 * K;
    xd += (int64_t)m0 * nb;
    const int tid_all = threadIdx.x, lane = tid_all & 63, q = lane >> 4, r = lane & 15;
    const int wave_all = __builtin_amdgcn_readfirstlane(tid_all >> 6);
    const int kg = wave_all / kSmallRG, wave = wave_all % kSmallRG, tid = tid_all % NT;
    int8_t *const xs = xs_all[kg];
    float(*const xds)[SB + 1] = xds_all[kg];
    const int nw = g * 16 * kSmallRG + 16 * wave;
    // this group's share of the split's K blocks (the plan makes both shares equal)
    const int zs0 = z * bps, zs1 = min(nb, zs0 + bps), share = (zs1 - zs0) / KG;
    const int zb0 = zs0 + kg * share, zb1 = zb0 + share;
    const __amdgpu_buffer_rsrc_t w_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)wq, (short)0, N * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t x_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)xq, (short)0, Mt * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t wd_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)wd, (short)0, N * nb * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t xd_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)xd, (short)0, Mt * nb * 2, 0x00020000);

    float acc[MT][4];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) acc[t][v] = 0.0f;
    // One stage's operands in registers: weight pairs and scales (HBM), activation
    // pieces and scales (L2).  The next stage's loads are issued before this stage's
    // products, two register sets alternating.
    constexpr int PIECES = ROWS * SB * 2, PPT = (PIECES + NT - 1) / NT, SPT = (ROWS * SB + NT - 1) / NT;
    struct Stage {
        v4i wv[SB / 2], dwv[4], xv[PPT];
        uint16_t xh[SPT];
    };
    auto issue = [&](Stage &st, int kb0) {
#pragma unroll
        for (int p = 0; p < SB / 2; p++)
            st.wv[p] = __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, (nw + r) * K + (kb0 + 2 * p) * 32 + 16 * q, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; v++)
            st.dwv[v] = __builtin_amdgcn_raw_buffer_load_b128(wd_rsrc, ((nw + 4 * q + v) * nb + kb0) * 2, 0, 0);
        // activation piece c = (row, block, half); threads past the end reload the last piece
#pragma unroll
        for (int k = 0; k < PPT; k++) {
            const int c = min(k * NT + tid, PIECES - 1);
            const int row = c / (2 * SB), b = (c / 2) % SB, h = c & 1;
            st.xv[k] = __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, row * K + (kb0 + b) * 32 + 16 * h, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < SPT; k++) {
            const int c = min(k * NT + tid, ROWS * SB - 1);
            st.xh[k] = __builtin_amdgcn_raw_buffer_load_b16(xd_rsrc, ((c / SB) * nb + kb0 + c % SB) * 2, 0, 0);
        }
    };
    auto run = [&](const Stage &st, int kb0) {
        __syncthreads();   // the previous stage's LDS reads are done
#pragma unroll
        for (int k = 0; k < PPT; k++) {
            const int c = k * NT + tid;
            if (PIECES % NT == 0 || c < PIECES) {
                const int row = c / (2 * SB), b = (c / 2) % SB, h = c & 1;
                int8_t *dst = xs + row * kSmallPitch + b * 32;
                *(long *)(dst + 8 * h) = pack64((uint32_t)st.xv[k].x, (uint32_t)st.xv[k].y);
                *(long *)(dst + 8 * h + 16) = pack64((uint32_t)st.xv[k].z, (uint32_t)st.xv[k].w);
            }
        }
#pragma unroll
        for (int k = 0; k < SPT; k++) {
            const int c = k * NT + tid;
            if ((ROWS * SB) % NT == 0 || c < ROWS * SB) xds[c / SB][c % SB] = kb0 + c % SB < zb1 ? vxm_h2f(st.xh[k]) : 0.0f;
        }
        __syncthreads();
        // per block pair: the pair's operands, then all 2 MT products, then their scaling
#pragma unroll
        for (int p = 0; p < SB / 2; p++) {
            // lanes 0-31 trade their high halves for the low halves of lanes 32-63
            const auto s0 = __builtin_amdgcn_permlane32_swap((uint32_t)st.wv[p].x, (uint32_t)st.wv[p].z, false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap((uint32_t)st.wv[p].y, (uint32_t)st.wv[p].w, false, false);
            const long a[2] = {pack64(s0[0], s1[0]), pack64(s0[1], s1[1])};
            long bx[2][MT];
            float dx[2][MT];
#pragma unroll
            for (int e = 0; e < 2; e++)
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    bx[e][t] = *(const long *)(xs + (16 * t + r) * kSmallPitch + (2 * p + e) * 32 + 8 * q);
                    dx[e][t] = xds[16 * t + r][2 * p + e];
                }
            v4i c[2][MT];
#pragma unroll
            for (int e = 0; e < 2; e++)
#pragma unroll
                for (int t = 0; t < MT; t++) c[e][t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[e], bx[e][t], v4i{}, 0, 0, 0);
            if (DOTS) {
                // lane (q, r) holds the sums of weight rows nw + 4q + v with activation row 16t + r
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const int b = kb0 + 2 * p + e;
#pragma unroll
                    for (int t = 0; t < MT; t++) {
                        const int m = 16 * t + r;
                        if (b >= zb1 || m >= Mt) continue;
#pragma unroll
                        for (int v = 0; v < 4; v++)
                            dots[((int64_t)(m0 + m) * N + nw + 4 * q + v) * nb + b] = c[e][t][v];
                    }
                }
                continue;
            }
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int b = 2 * p + e;
                float dw[4];
#pragma unroll
                for (int v = 0; v < 4; v++) dw[v] = half_at(st.dwv[v], b);
#pragma unroll
                for (int t = 0; t < MT; t++)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        acc[t][v] = __builtin_fmaf((float)c[e][t][v], dw[v] * dx[e][t], acc[t][v]);
            }
        }
    };
    Stage sa, sb;
    if (zb0 < zb1) issue(sa, zb0);
    for (int kb0 = zb0; kb0 < zb1; kb0 += 2 * SB) {
        const bool b_live = kb0 + SB < zb1;
        if (b_live) issue(sb, kb0 + SB);
        run(sa, kb0);
        if (!b_live) break;
        if (kb0 + 2 * SB < zb1) issue(sa, kb0 + 2 * SB);
        run(sb, kb0 + SB);
    }
    if (DOTS) return;
    if (KG > 1) {
        // group 1 hands its partial products to group 0 (added as group 0 + group 1)
        __shared__ float kred[kSmallRG][MT * 4][64];
        if (kg == 1) {
#pragma unroll
            for (int t = 0; t < MT; t++)
#pragma unroll
                for (int v = 0; v < 4; v++) kred[wave][t * 4 + v][lane] = acc[t][v];
        }
        __syncthreads();
        if (kg == 0) {
#pragma unroll
            for (int t = 0; t < MT; t++)
#pragma unroll
                for (int v = 0; v < 4; v++) acc[t][v] = acc[t][v] + kred[wave][t * 4 + v][lane];
        }
    }
    if (sq) {
        // SwiGLU + Q8_0 epilogue (one split): the workgroup's 64 weight rows are 32 (gate,
        // up) pairs, rows 4q + v with v even (gate) and v + 1 (up) in the same lane, so each
        // activation row gets one Q8_0 block of p = bf16(bf16(silu(bf16(g))) * bf16(u)) (as in
        // k_swiglu_quant), gathered through LDS and quantized by four threads per row with
        // the activation rule of quant_block_4lanes.
        __shared__ float ps[ROWS][33];
        if (kg == 0) {
#pragma unroll
            for (int t = 0; t < MT; t++)
#pragma unroll
                for (int vp = 0; vp < 2; vp++) {
                    const float gb = vxm_bf16(acc[t][2 * vp]);
                    const float sl = vxm_bf16(__fdiv_rn(gb, 1.0f + expf(-gb)));
                    ps[16 * t + r][8 * wave + 2 * q + vp] = vxm_bf16(sl * vxm_bf16(acc[t][2 * vp + 1]));
                }
        }
        __syncthreads();
        const int F = N / 2, row = tid_all >> 2, part = tid_all & 3;
        if (row < ROWS) {   // group 0's threads, four per row; idle threads leave whole 4-lane groups
            float pv[8], amax = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                pv[e] = ps[row][8 * part + e];
                amax = fmaxf(amax, fabsf(pv[e]));
            }
            amax = vxm_quad_max(amax);
            const float d = __fdiv_rn(amax, 127.0f);
            float id;
            if (variant == VXM_QUANT_X86) id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
            else id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
            if (row < Mt) {
                uint32_t lo = 0, hi = 0;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float qv = variant == VXM_QUANT_X86 ? rintf(pv[e] * id) : roundf(pv[e] * id);
                    qv = fminf(fmaxf(qv, -128.0f), 127.0f);
                    const uint32_t b = (uint32_t)(uint8_t)(int8_t)(int)qv;
                    if (e < 4) lo |= b << (8 * e);
                    else hi |= b << (8 * (e - 4));
                }
                const int64_t base = (int64_t)(m0 + row) * F + g * 32 + 8 * part;
                *(uint2 *)(sq + base) = make_uint2(lo, hi);
                if (part == 0) sd[base / 32] = vxm_f2h(d);
            }
        }
        return;
    }
    if (kg != 0) return;
    float *yz = y + (int64_t)z * M * N + (int64_t)m0 * N;
#pragma unroll
    for (int t = 0; t < MT; t++) {
        const int m = 16 * t + r;
        if (m >= Mt) continue;
#pragma unroll
        for (int v = 0; v < 4; v++) yz[(int64_t)m * N + nw + 4 * q + v] = acc[t][v];
    }
}

// y[i] = sum of the n slices in slice order (the public entry's K-split fix-up).
__global__ void k_sum_parts(const float *__restrict__ p, int n, int64_t stride, float *__restrict__ y,
                            int64_t count) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i >= count) return;   // count % 4 == 0
    float4 s = *(const float4 *)(p + i);
    for (int z = 1; z < n; z++) {
        const float4 v = *(const float4 *)(p + z * stride + i);
        s.x = s.x + v.x; s.y = s.y + v.y; s.z = s.z + v.z; s.w = s.w + v.w;
    }
    *(float4 *)(y + i) = s;
}

// Tile grid, stage depth and K split of the register-staged GEMM
// (k_gemm_q8_0_mfma).  Single-row-tile GEMMs (M <= 64) take 16-block stages,
// the others 8-block stages (two workgroups per CU); the K split (at most 4
// ways, each part at least 2 stages) brings the grid towards one workgroup per
// CU.  tile_n > 0: k_gemm_q8_0_tile with 64 x tile_n tiles instead.
struct GemmPlan {
    int tiles_m, tiles_n, splits, bps, ks;
    int tile_n, tile_m;
    // two-part tile plans (unsplit): columns [0, n_split) on tile_m x tile_n tiles,
    // [n_split, N) on a second launch of tile_m1 x tile_n1 tiles; n_split = 0: one part
    int n_split, tile_m1, tile_n1, tiles_m1, tiles_n1;
};

static GemmPlan gemm_plan(vxm_ctx *ctx, int64_t M, int N, int nb) {
    GemmPlan p;
    p.tiles_m = (int)((M + GM - 1) / GM);
    p.tiles_n = (N + GN - 1) / GN;
    p.tile_n = p.tile_m = 0;
    p.n_split = 0;
    p.ks = p.tiles_m == 1 ? 16 : 8;
    int s = 1;
    while (s < kGemmMaxSplits && (int64_t)p.tiles_m * p.tiles_n * s < ctx->n_cu &&
           nb / (s * 2) >= 2 * p.ks)
        s *= 2;
    p.bps = (nb + s - 1) / s;
    p.splits = (nb + p.bps - 1) / p.bps;   // every split then owns at least one block
    return p;
}

#ifndef VXM_GEMM_TILE
#define VXM_GEMM_TILE 1
#endif

// Relative cost of a 128 x 128 block step per output against a 64-row tile's:
// twice the blocks per wave between barriers and half the operand bytes per
// output.  Percent (measured: a 128 x 128 tile of 64 blocks takes 1.57x the time
// of a 64 x 128 one).
#ifndef VXM_TILE128_COST
#define VXM_TILE128_COST 79
#endif
#ifndef VXM_TILE128_SPLITS
#define VXM_TILE128_SPLITS 0
#endif
// Charge of a second launch in a two-part plan, in 64 x 128 block steps (the
// gap between two dependent launches, ~1.5 us).
#ifndef VXM_TILE_PART_CHARGE
#define VXM_TILE_PART_CHARGE 5
#endif
// Charge of a K split, in block steps per round (the tagged partial words and
// the last workgroup's fix-up).
#ifndef VXM_TILE_SPLIT_CHARGE
#define VXM_TILE_SPLIT_CHARGE 24
#endif

// k_gemm_q8_0_tile plan: the tile (64 x 64, 64 x 128 or 128 x 128) and K split
// with the fewest block steps on the busiest CU, one workgroup per CU: rounds of
// the grid x blocks per split x tile outputs (the per-block conversion work is
// per output; a 128 x 128 step is charged VXM_TILE128_COST percent of four
// 64 x 64 steps), plus a fix-up charge per round when the K is split.  Ties go
// to the larger tile (fewer operand bytes per output).  Splits keep whole
// 8-block steps and at most the tile's MaxBps blocks (the activation scale
// panel); their partial words must fit max_split_bytes.  Returns false when the
// shape is not the tile kernel's (K % 256, alignment).
static bool tile_plan(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                      size_t max_split_bytes, GemmPlan &best) {
    const int N = (int)w->n, nb = (int)(w->k / 32);
    if (!VXM_GEMM_TILE || !w->dt || nb % 8 != 0 || ((uintptr_t)xq & 15) || ((uintptr_t)xd & 15)) return false;
    int64_t best_cost = -1;
    const int shapes[3][2] = {{128, 128}, {64, 128}, {64, 64}};
    for (const auto &sh : shapes) {
        const int tm = sh[0], tn = sh[1];
        for (int s = 1; s <= kGemmMaxSplits; s++) {
            const int bps = ((nb + s - 1) / s + 7) / 8 * 8;
            const int splits = (nb + bps - 1) / bps;
            if (bps > tile_max_bps(tm) || splits != s) continue;
            // 128 x 128 tiles unsplit only: split, they measured far slower than the 64-row
            // plans (O 2048 x 2048 at M = 512, 4 splits: 42 against 12.7 us)
            if (tm == 128 && splits > 1 && !VXM_TILE128_SPLITS) continue;
            if (splits > 1 && (size_t)splits * M * N * sizeof(uint64_t) > max_split_bytes)
                continue;
            const int tiles_m = (int)((M + tm - 1) / tm), tiles_n = (N + tn - 1) / tn;
            const int64_t wgs = (int64_t)tiles_m * tiles_n * splits, rounds = (wgs + ctx->n_cu - 1) / ctx->n_cu;
            int64_t cost = rounds * (bps + (splits > 1 ? VXM_TILE_SPLIT_CHARGE : 0)) * tn * (tm / 64) * 100;
            if (tm == 128) cost = cost * VXM_TILE128_COST / 100;
            if (best_cost < 0 || cost < best_cost) {
                best_cost = cost;
                best.tiles_m = tiles_m;
                best.tiles_n = tiles_n;
                best.splits = splits;
                best.bps = bps;
                best.ks = 0;
                best.tile_n = tn;
                best.tile_m = tm;
                best.n_split = 0;
            }
        }
    }
    // two launches: whole rounds of 128 x 128 tiles over the first columns, the rest
    // on 64-row tiles (a grid of 128 x 128 tiles that would leave its last round
    // part-empty, e.g. 384 tiles for 512 x 12288)
    const int tm128 = (int)((M + 127) / 128);
    if (nb <= tile_max_bps(128) && tm128 <= ctx->n_cu && ctx->n_cu % tm128 == 0) {
        const int cols = ctx->n_cu / tm128 * 128;   // columns of one full round
        for (int r = 1; (int64_t)r * cols < N; r++) {
            const int na = r * cols, rest = N - na;
            for (int tn : {128, 64}) {
                const int64_t tiles_b = (int64_t)((M + 63) / 64) * ((rest + tn - 1) / tn),
                              rounds_b = (tiles_b + ctx->n_cu - 1) / ctx->n_cu;
                const int64_t cost = (int64_t)r * nb * 256 * VXM_TILE128_COST + rounds_b * nb * tn * 100 +
                                     (int64_t)VXM_TILE_PART_CHARGE * 128 * 100;
                if (cost < best_cost) {
                    best_cost = cost;
                    best.tiles_m = tm128;
                    best.tiles_n = na / 128;
                    best.splits = 1;
                    best.bps = ((nb + 7) / 8) * 8;
                    best.ks = 0;
                    best.tile_n = 128;
                    best.tile_m = 128;
                    best.n_split = na;
                    best.tile_m1 = 64;
                    best.tile_n1 = tn;
                    best.tiles_m1 = (int)((M + 63) / 64);
                    best.tiles_n1 = (rest + tn - 1) / tn;
                }
            }
        }
    }
    return best_cost >= 0;
}

// The tile kernel's dynamic LDS (4 stages + the scale panel, up to 157 KiB) is
// above the default limit: raise it once per device for each instantiation.
template <int TM, int TN, bool DOTS>
static int launch_gemm_tile_t(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                              float *y, int32_t *dots, const GemmPlan &p, int tiles_m, int tiles_n, int n_base,
                              uint64_t *part, int *cnt, const uint32_t *epoch,
                              int8_t *sq, uint16_t *sd, int variant, const vxm_qkv_epi &qe) {
    static std::atomic<uint64_t> attr_done{0};
    const uint64_t bit = 1ull << (ctx->device & 63);
    if (!(attr_done.load() & bit)) {
        VXM_HIP(ctx, hipFuncSetAttribute((const void *)k_gemm_q8_0_tile<TM, TN, DOTS>,
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)tile_lds_bytes(TM, TN, tile_max_bps(TM))));
        attr_done.fetch_or(bit);
    }
    const int grid_x = 8 * tiles_m * ((tiles_n + 7) / 8);
    hipLaunchKernelGGL((k_gemm_q8_0_tile<TM, TN, DOTS>), dim3(grid_x, p.splits), dim3(kTileThreads),
                       (unsigned)tile_lds_bytes(TM, TN, p.bps), ctx->stream, xq, xd, w->qs, w->dt, y, part, cnt, dots,
                       (int)M, (int)w->n, (int)w->k, tiles_m, tiles_n, p.bps, p.splits, n_base, epoch, ctx->dev_err,
                       sq, sd, variant, qe);
    return VXM_OK;
}

template <bool DOTS>
static int launch_gemm_tile_part(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                                 float *y, int32_t *dots, const GemmPlan &p, int tm, int tn, int tiles_m, int tiles_n,
                                 int n_base, uint64_t *part, int *cnt, const uint32_t *epoch, int8_t *sq,
                                 uint16_t *sd, int variant, const vxm_qkv_epi &qe) {
    if (tm == 128)
        return launch_gemm_tile_t<128, 128, DOTS>(ctx, w, xq, xd, M, y, dots, p, tiles_m, tiles_n, n_base, part, cnt,
                                                  epoch, sq, sd, variant, qe);
    return tn == 128 ? launch_gemm_tile_t<64, 128, DOTS>(ctx, w, xq, xd, M, y, dots, p, tiles_m, tiles_n, n_base, part,
                                                         cnt, epoch, sq, sd, variant, qe)
                     : launch_gemm_tile_t<64, 64, DOTS>(ctx, w, xq, xd, M, y, dots, p, tiles_m, tiles_n, n_base, part,
                                                        cnt, epoch, sq, sd, variant, qe);
}

// sq != nullptr: SwiGLU + Q8_0 epilogue (gate/up weight with interleaved rows, one
// split, N % 64 == 0) into sq [M][N/2], sd [M][N/64] instead of y
// qe.q_out != nullptr: the QKV epilogue (k_rope_kv's work, one split) instead of y
template <bool DOTS>
static int launch_gemm_tile(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                            float *y, int32_t *dots, const GemmPlan &p, uint64_t *part, int *cnt, const uint32_t *epoch,
                            int8_t *sq = nullptr, uint16_t *sd = nullptr, int variant = 0,
                            const vxm_qkv_epi &qe = vxm_qkv_epi{}) {
    int rc = launch_gemm_tile_part<DOTS>(ctx, w, xq, xd, M, y, dots, p, p.tile_m, p.tile_n, p.tiles_m, p.tiles_n, 0,
                                         part, cnt, epoch, sq, sd, variant, qe);
    if (rc || !p.n_split) return rc;
    return launch_gemm_tile_part<DOTS>(ctx, w, xq, xd, M, y, dots, p, p.tile_m1, p.tile_n1, p.tiles_m1, p.tiles_n1,
                                       p.n_split, part, cnt, epoch, sq, sd, variant, qe);
}

template <int KS>
static void launch_gemm_ks(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                           float *y, const GemmPlan &p, uint64_t *part, int *cnt, const uint32_t *epoch) {
    const int grid_x = 8 * p.tiles_m * ((p.tiles_n + 7) / 8);
    hipLaunchKernelGGL((k_gemm_q8_0_mfma<KS, false>), dim3(grid_x, p.splits), dim3(kGemmThreads), 0, ctx->stream,
                       xq, xd, w->qs, w->d, y, part, cnt, nullptr, (int)M, (int)w->n, (int)w->k, p.tiles_m,
                       p.tiles_n, p.bps, p.splits, epoch, ctx->dev_err);
}

template <int KS>
static void launch_gemm_dots_ks(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                                int32_t *dots, const GemmPlan &p) {
    const int grid_x = 8 * p.tiles_m * ((p.tiles_n + 7) / 8);
    hipLaunchKernelGGL((k_gemm_q8_0_mfma<KS, true>), dim3(grid_x, p.splits), dim3(kGemmThreads), 0, ctx->stream,
                       xq, xd, w->qs, w->d, nullptr, nullptr, nullptr, dots, (int)M, (int)w->n, (int)w->k,
                       p.tiles_m, p.tiles_n, p.bps, p.splits, nullptr, ctx->dev_err);
}

// Buffer-load offsets are 32-bit: every row tile of A and W must lie below 2 GiB.
static bool gemm_fits(int64_t M, int64_t N, int64_t K) {
    const int64_t lim = (int64_t)1 << 31;
    return (M + 128) * K < lim && (N + 128) * K < lim;
}

// Buffers of the public matmul entries' K splits when the caller brings them
// (the allocation-free entry); null: the context's own scratch.
struct MmWork {
    uint64_t *words;     // tagged partial words of the tiled GEMM's splits
    size_t words_bytes;
    int *cnt;            // its per-tile arrival counters, zero on entry
    size_t ncnt;
    float *parts;        // the small-M GEMM's K-split slices
    size_t parts_bytes;
    uint32_t *epoch;     // device word: the tag of the last split launch on these words
};

__global__ void k_fill_zero(uint4 *__restrict__ p, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0, 0, 0, 0);
}

// Before every split launch: the next split tag into the device word *ep (0 is
// skipped: the partial words start zeroed), and n16 16-byte words of arrival
// counters cleared.  The tag lives in device memory, so a launch recorded into
// a HIP graph reads a new tag on every replay: a replay can never take a word
// that an earlier replay left for its own tag.
__global__ void k_split_prepare(uint32_t *__restrict__ ep, uint4 *__restrict__ cnt, int64_t n16) {
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        const uint32_t e = *ep + 1u;
        *ep = e ? e : 1u;
    }
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
        cnt[i] = make_uint4(0, 0, 0, 0);
}

static int launch_gemm(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                       float *y, const MmWork *wk = nullptr) {
    const int N = (int)w->n, K = (int)w->k, nb = K / 32;
    if (!gemm_fits(M, N, K))
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "mul_mat: %lld x %d x %d exceeds the GEMM's 2 GiB operand range",
                        (long long)M, N, K);
    // the same plan with or without a caller's workspace: a workspace too small
    // for it is an error, never a silently different (unsplit) summation order
    GemmPlan p;
    if (!tile_plan(ctx, w, xq, xd, M, SIZE_MAX, p)) p = gemm_plan(ctx, M, N, nb);
    uint64_t *part = nullptr;
    int *cnt = nullptr;
    uint32_t *epoch = nullptr;
    if (p.splits > 1) {
        const size_t wbytes = (size_t)p.splits * M * N * sizeof(uint64_t), ncnt = (size_t)p.tiles_m * p.tiles_n;
        int64_t n16 = 0;
        if (wk) {
            if (wbytes > wk->words_bytes || ncnt > wk->ncnt)
                return vxm_fail(ctx, VXM_ERR_INVALID_ARG,
                                "mul_mat: %lld x %d x %d needs %zu B of split partials and %zu counters; the "
                                "workspace holds %zu B and %zu",
                                (long long)M, N, K, wbytes, ncnt, wk->words_bytes, wk->ncnt);
            part = wk->words;
            cnt = wk->cnt;
            epoch = wk->epoch;
            // the counters start this launch at zero whatever an earlier call left
            n16 = (int64_t)((ncnt * sizeof(int) + 15) / 16);
        } else {
            int rc = vxm_ensure_split(ctx, wbytes, ncnt);
            if (rc) return rc;
            part = (uint64_t *)ctx->split_buf;
            cnt = ctx->split_cnt;   // zero between launches: the last workgroup of a tile resets its counter
            epoch = ctx->split_epoch_dev;
        }
        hipLaunchKernelGGL(k_split_prepare, dim3((unsigned)(n16 > 0 ? (n16 + 255) / 256 : 1)), dim3(256), 0,
                           ctx->stream, epoch, (uint4 *)cnt, n16);
        ctx->split_launched = true;
    }
    if (p.tile_n) {
        int rc = launch_gemm_tile<false>(ctx, w, xq, xd, M, y, nullptr, p, part, cnt, epoch);
        if (rc) return rc;
    } else if (p.ks == 16) {
        launch_gemm_ks<16>(ctx, w, xq, xd, M, y, p, part, cnt, epoch);
    } else {
        launch_gemm_ks<8>(ctx, w, xq, xd, M, y, p, part, cnt, epoch);
    }
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

// Rows of activations from which the MFMA GEMM replaces the weight-streaming
// GEMV (which re-reads each activation row per weight row group).
constexpr int kMfmaMinRows = 8;
// Inside the block pipeline (no fix-up launch for K splits, SwiGLU fused into
// gate/up) the small-M kernel already beats the GEMV from 2 rows.
constexpr int kSmallPartsMinRows = 2;

// Small-M plan: K splits in whole stages, doubling while the grid leaves CUs
// idle (at most max_parts).  Shapes outside the kernel's layout (N % 64,
// K % 256, M > 64, operands of 2 GiB) take the tiled GEMM.
struct SmallPlan {
    int mt, bps, splits, groups, mtiles, kg;
};

static bool small_plan(vxm_ctx *ctx, int64_t M, int64_t N, int64_t K, int max_parts, SmallPlan &p) {
    if (M < 1 || M > VXM_SMALL_MAX_ROWS || N % (16 * kSmallRG) || K % (32 * kSmallStage)) return false;
    // 32-bit buffer offsets: the weights, and the activation rows
    if (N * K >= ((int64_t)1 << 31) || VXM_SMALL_MAX_ROWS * K >= ((int64_t)1 << 31)) return false;
    const int nb = (int)(K / 32), stages = nb / kSmallStage;
    p.mt = (int)((M + 15) / 16);
    p.mtiles = 1;   // the kernel takes row tiles of 16 MT (blockIdx.z); M <= 64 is one tile
    p.groups = (int)(N / (16 * kSmallRG));
    int s = 1;
    while (s * 2 <= max_parts && s * 2 <= stages && (int64_t)p.groups * p.mtiles * s < ctx->n_cu) s *= 2;
    const int per = (stages + s - 1) / s;   // stages per split
    p.bps = per * kSmallStage;
    p.splits = (nb + p.bps - 1) / p.bps;
    // two wave groups per workgroup halve each split's serial stage chain when every
    // split (the last one included) holds an even number of stages
    p.kg = (per % 2 == 0 && stages % 2 == 0) ? 2 : 1;
    return true;
}

static void launch_small(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                         float *y, const SmallPlan &p, int8_t *sq = nullptr, uint16_t *sd = nullptr,
                         int variant = 0, int32_t *dots = nullptr) {
    const dim3 grid(p.groups, p.splits, p.mtiles), block(64 * kSmallRG * p.kg);
    const int N = (int)w->n, K = (int)w->k;
#define VXM_SMALL_ARGS xq, xd, w->qs, w->d, y, (int)M, N, K, p.bps, sq, sd, variant, dots
#define VXM_SMALL_KG(MT, D)                                                                                \
    do {                                                                                                   \
        if (p.kg == 2)                                                                                     \
            hipLaunchKernelGGL((k_gemm_q8_0_small<MT, 2, D>), grid, block, 0, ctx->stream, VXM_SMALL_ARGS); \
        else                                                                                               \
            hipLaunchKernelGGL((k_gemm_q8_0_small<MT, 1, D>), grid, block, 0, ctx->stream, VXM_SMALL_ARGS); \
    } while (0)
#define VXM_SMALL_MT(MT)                    \
    do {                                    \
        if (dots) VXM_SMALL_KG(MT, true);   \
        else VXM_SMALL_KG(MT, false);       \
    } while (0)
    switch (p.mt) {
        case 1: VXM_SMALL_MT(1); break;
        case 2: VXM_SMALL_MT(2); break;
        case 3: VXM_SMALL_MT(3); break;
        default: VXM_SMALL_MT(4); break;
    }
#undef VXM_SMALL_MT
#undef VXM_SMALL_KG
#undef VXM_SMALL_ARGS
}

// Public entry: a split product goes through the context's scratch and one
// fix-up launch that adds the slices in order.
static int launch_gemm_small(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                             float *y, const SmallPlan &p, const MmWork *wk = nullptr) {
    if (p.splits == 1) {
        launch_small(ctx, w, xq, xd, M, y, p);
        VXM_CHECK_LAUNCH(ctx);
        return VXM_OK;
    }
    const int64_t count = M * w->n;
    const size_t pbytes = (size_t)p.splits * count * sizeof(float);
    float *scratch;
    if (wk) {
        if (pbytes > wk->parts_bytes)
            return vxm_fail(ctx, VXM_ERR_INVALID_ARG,
                            "mul_mat: %lld x %lld x %lld needs %zu B of K-split slices; the workspace holds %zu B",
                            (long long)M, (long long)w->n, (long long)w->k, pbytes, wk->parts_bytes);
        scratch = wk->parts;
    } else {
        int rc = vxm_ensure_parts(ctx, pbytes);
        if (rc) return rc;
        scratch = (float *)ctx->parts_buf;
    }
    launch_small(ctx, w, xq, xd, M, scratch, p);
    VXM_CHECK_LAUNCH(ctx);
    const int64_t threads = count / 4;   // N % 64 == 0
    hipLaunchKernelGGL(k_sum_parts, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, ctx->stream, scratch,
                       p.splits, count, y, count);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

int vxm_launch_mul_mat_parts(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                             float *y, int max_parts, int *parts) {
    *parts = 1;
    if (M <= 0) return VXM_OK;
    SmallPlan sp;
    const bool small = (ctx->path == VXM_PATH_MFMA || (ctx->path == VXM_PATH_AUTO && M >= kSmallPartsMinRows)) &&
                       small_plan(ctx, M, w->n, w->k, max_parts < VXM_MAX_PARTS ? max_parts : VXM_MAX_PARTS, sp);
    if (!small) return vxm_launch_mul_mat(ctx, w, xq, xd, M, y);
    launch_small(ctx, w, xq, xd, M, y, sp);
    VXM_CHECK_LAUNCH(ctx);
    *parts = sp.splits;
    return VXM_OK;
}

// The gate/up projection with SwiGLU and the Q8_0 of its output fused into the
// GEMM's epilogue (rows of w interleave gate n = row 2n and up n = row 2n+1): sq
// [M][N/2] and sd [M][N/64] are the down projection's input.  The small-M kernel
// takes M <= 64, the tile GEMM larger M when its plan needs no K split.  Returns
// false without launching otherwise (and under PATH_MFMA_TILED, which keeps the
// unfused GEMM + k_swiglu_quant as the reference of the fused epilogue).
bool vxm_launch_gate_up_swiglu(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                               int8_t *sq, uint16_t *sd, int variant, int *rc) {
    *rc = VXM_OK;
    const int64_t N = w->n, K = w->k;
    const bool mfma = ctx->path == VXM_PATH_MFMA || (ctx->path == VXM_PATH_AUTO && M >= kSmallPartsMinRows);
    if (!mfma || M <= 0 || N % 64) return false;
    SmallPlan sp;
    if (small_plan(ctx, M, N, K, 1, sp)) {
        // unsplit: each workgroup holds whole 32-pair blocks over all of K
        launch_small(ctx, w, xq, xd, M, nullptr, sp, sq, sd, variant);
    } else {
        GemmPlan p;
        if (!tile_plan(ctx, w, xq, xd, M, 0, p) || p.splits != 1) return false;
        if ((*rc = launch_gemm_tile<false>(ctx, w, xq, xd, M, nullptr, nullptr, p, nullptr, nullptr, nullptr, sq, sd,
                                           variant)))
            return true;
    }
    if (hipGetLastError() != hipSuccess) *rc = vxm_fail(ctx, VXM_ERR_BACKEND, "gate/up + SwiGLU launch failed");
    return true;
}

// The QKV projection with k_rope_kv's work in the tile GEMM's epilogue (qe):
// taken where vxm_launch_mul_mat_parts would run the tile GEMM without a K
// split (M > 64 and a plan of one split), so the products are the same.
// Returns false without launching otherwise, and under PATH_MFMA_TILED (which
// keeps the GEMM + k_rope_kv pair as the reference of the fused epilogue).
static bool use_mfma(const vxm_ctx *ctx, int64_t M);

bool vxm_launch_qkv_rope(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                         const vxm_qkv_epi &qe, int cs_rows, int *rc) {
    *rc = VXM_OK;
    if (M <= VXM_SMALL_MAX_ROWS || !use_mfma(ctx, M) || ctx->path == VXM_PATH_MFMA_TILED || !qe.q_out) return false;
    const int64_t N = w->n;
    if (qe.hd % 4 || N != (int64_t)(qe.nh + 2 * qe.nkv) * qe.hd || qe.S <= 0) return false;
    if (!gemm_fits(M, (int)N, (int)w->k)) return false;
    GemmPlan p;
    if (!tile_plan(ctx, w, xq, xd, M, SIZE_MAX, p) || p.splits != 1) return false;
    if (!qe.no_rope && (!qe.cs || qe.pos0 + std::min<int64_t>(M, qe.S) > cs_rows)) {
        *rc = vxm_fail(ctx, VXM_ERR_BACKEND, "rope: table holds %d positions, %lld needed", cs_rows,
                       (long long)(qe.pos0 + std::min<int64_t>(M, qe.S)));
        return true;
    }
    if ((*rc = launch_gemm_tile<false>(ctx, w, xq, xd, M, nullptr, nullptr, p, nullptr, nullptr, nullptr, nullptr, nullptr,
                                       0, qe)))
        return true;
    if (hipGetLastError() != hipSuccess) *rc = vxm_fail(ctx, VXM_ERR_BACKEND, "QKV + rope launch failed");
    return true;
}

template <int C, int R>
static void launch_gemv_c(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd,
                          int64_t M, float *y, int32_t *dots) {
    const int waves = (int)((w->n + R - 1) / R);
    const int grid = (waves + 3) / 4;
    if (dots)
        hipLaunchKernelGGL((k_gemv_q8_0<C, R, true>), dim3(grid), dim3(256), 0, ctx->stream, w->qs, w->dg, xq, xd,
                           nullptr, (int)w->n, (int)M, dots);
    else
        hipLaunchKernelGGL((k_gemv_q8_0<C, R, false>), dim3(grid), dim3(256), 0, ctx->stream, w->qs, w->dg, xq, xd,
                           y, (int)w->n, (int)M, nullptr);
}

// The GEMV family: the chunked kernel where K / 1024 has a build, else the
// generic one.  dots != nullptr: the same kernel's int32 block sums instead of y.
static void launch_gemv(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                        float *y, int32_t *dots) {
    const int64_t K = w->k;
    if (w->dg) {
        switch (K / 1024) {
            case 1: launch_gemv_c<1, 4>(ctx, w, xq, xd, M, y, dots); return;
            case 2: launch_gemv_c<2, 2>(ctx, w, xq, xd, M, y, dots); return;
            case 4: launch_gemv_c<4, 1>(ctx, w, xq, xd, M, y, dots); return;
            case 6: launch_gemv_c<6, 1>(ctx, w, xq, xd, M, y, dots); return;
            default: break;
        }
    }
    const int grid = (int)((w->n + 3) / 4);
    if (dots)
        hipLaunchKernelGGL(k_gemv_q8_0_generic<true>, dim3(grid), dim3(256), 0, ctx->stream, w->qs, w->d, xq, xd,
                           nullptr, (int)w->n, (int)K, (int)M, dots);
    else
        hipLaunchKernelGGL(k_gemv_q8_0_generic<false>, dim3(grid), dim3(256), 0, ctx->stream, w->qs, w->d, xq, xd,
                           y, (int)w->n, (int)K, (int)M, nullptr);
}

static bool use_mfma(const vxm_ctx *ctx, int64_t M) {
    return ctx->path == VXM_PATH_MFMA || ctx->path == VXM_PATH_MFMA_TILED ||
           (ctx->path == VXM_PATH_AUTO && M >= kMfmaMinRows);
}

static int launch_mul_mat(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                          float *y, const MmWork *wk) {
    if (M <= 0) return VXM_OK;
    if (use_mfma(ctx, M)) {
        SmallPlan sp;
        if (ctx->path != VXM_PATH_MFMA_TILED && small_plan(ctx, M, w->n, w->k, VXM_MAX_PARTS, sp))
            return launch_gemm_small(ctx, w, xq, xd, M, y, sp, wk);
        return launch_gemm(ctx, w, xq, xd, M, y, wk);
    }
    launch_gemv(ctx, w, xq, xd, M, y, nullptr);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

int vxm_launch_mul_mat(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd,
                       int64_t M, float *y) {
    return launch_mul_mat(ctx, w, xq, xd, M, y, nullptr);
}

// int32 block sums from the kernel vxm_launch_mul_mat picks for this M and path,
// with the same plan (stage depth, K splits): that kernel's own integer sums.
static int launch_block_dots(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                             int32_t *out) {
    if (use_mfma(ctx, M)) {
        SmallPlan sp;
        if (ctx->path != VXM_PATH_MFMA_TILED && small_plan(ctx, M, w->n, w->k, VXM_MAX_PARTS, sp)) {
            launch_small(ctx, w, xq, xd, M, nullptr, sp, nullptr, nullptr, 0, out);
        } else {
            const int N = (int)w->n, K = (int)w->k;
            if (!gemm_fits(M, N, K))
                return vxm_fail(ctx, VXM_ERR_INVALID_ARG,
                                "block_dots: %lld x %d x %d exceeds the GEMM's 2 GiB operand range", (long long)M, N, K);
            GemmPlan p;
            if (!tile_plan(ctx, w, xq, xd, M, SIZE_MAX, p)) p = gemm_plan(ctx, M, N, K / 32);
            if (p.tile_n) {
                int rc = launch_gemm_tile<true>(ctx, w, xq, xd, M, nullptr, out, p, nullptr, nullptr, nullptr);
                if (rc) return rc;
            } else if (p.ks == 16) {
                launch_gemm_dots_ks<16>(ctx, w, xq, xd, M, out, p);
            } else {
                launch_gemm_dots_ks<8>(ctx, w, xq, xd, M, out, p);
            }
        }
    } else {
        launch_gemv(ctx, w, xq, xd, M, nullptr, out);
    }
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

// ---- C ABI -----------------------------------------------------------------

extern "C" int vxm_quantize_q8_0(vxm_ctx *ctx, const float *x_dev, int64_t M, int64_t K, int variant,
                                 int8_t *xq_dev, uint16_t *xd_dev) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (!x_dev || !xq_dev || !xd_dev || M < 0 || K <= 0 || K % VXM_QK != 0)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "quantize: bad arguments (M=%lld K=%lld)",
                        (long long)M, (long long)K);
    if (variant != VXM_QUANT_REF && variant != VXM_QUANT_X86)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "quantize: unknown variant %d", variant);
    return vxm_launch_quantize(ctx, x_dev, M, K, variant, xq_dev, xd_dev);
}

static int check_mm(vxm_ctx *ctx, const vxm_weight *w, const void *a, const void *b, int64_t M,
                    const void *y) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (!w || !a || !b || !y || M < 0)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "mul_mat: null argument or negative M");
    if (w->n > INT32_MAX || M > INT32_MAX)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "mul_mat: size exceeds 2^31");
    return VXM_OK;
}

extern "C" int vxm_mul_mat_q8_0_q8_0(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq_dev,
                                     const uint16_t *xd_dev, int64_t M, float *y_dev) {
    int rc = check_mm(ctx, w, xq_dev, xd_dev, M, y_dev);
    if (rc) return rc;
    return vxm_launch_mul_mat(ctx, w, xq_dev, xd_dev, M, y_dev);
}

extern "C" int vxm_mul_mat_q8_0(vxm_ctx *ctx, const vxm_weight *w, const float *x_dev, int64_t M,
                                float *y_dev) {
    int rc = check_mm(ctx, w, x_dev, x_dev, M, y_dev);
    if (rc) return rc;
    const int64_t K = w->k;
    const size_t qbytes = ((size_t)M * K + 255) & ~(size_t)255;
    rc = vxm_ensure_act(ctx, qbytes + (size_t)M * (K / VXM_QK) * 2);
    if (rc) return rc;
    int8_t *xq = (int8_t *)ctx->act_buf;
    uint16_t *xd = (uint16_t *)((char *)ctx->act_buf + qbytes);
    rc = vxm_launch_quantize(ctx, x_dev, M, K, ctx->quant_variant, xq, xd);
    if (rc) return rc;
    return vxm_launch_mul_mat(ctx, w, xq, xd, M, y_dev);
}

extern "C" int vxm_block_dots_q8_0(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq_dev,
                                   const uint16_t *xd_dev, int64_t M, int32_t *out_dev) {
    int rc = check_mm(ctx, w, xq_dev, xd_dev, M, out_dev);
    if (rc) return rc;
    const int64_t total = M * w->n * (w->k / VXM_QK);
    if (total == 0) return VXM_OK;
    return launch_block_dots(ctx, w, xq_dev, xd_dev, M, out_dev);
}

// ---- the allocation-free matmul ---------------------------------------------
// vxm_mul_mat_q8_0_noalloc runs the kernels of vxm_mul_mat_q8_0, with the same
// plans, but takes every buffer beyond x and y from `scratch`, a file-scope
// device array that the code object carries: no call allocates.  Layout:
//   [0, kScrCnt - 256)           per-tile arrival counters of the tiled GEMM's
//                                K splits (zeroed by each call that splits)
//   [kScrCnt - 256, kScrCnt)     the split tag word (advanced on the device
//                                before each split launch)
//   [kScrCnt, +kScrWords)        its tagged partial words, and nothing else, so
//                                no leftover of another use can carry a live tag
//   [kScrCnt + kScrWords, end)   the quantized activation, then the small-M
//                                GEMM's K-split slices
// Every call on a device shares that device's copy of the array: calls that
// overlap on one device (two streams, two threads) race.
constexpr size_t kScrCnt = 64 << 10, kScrWords = 16 << 20, kScrGeneral = 32 << 20;
constexpr size_t kScratchBytes = kScrCnt + kScrWords + kScrGeneral;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// The device address of `scratch` on each device (the host-side name is a
// stand-in, never a device address), set once per device with that device
// current.
constexpr int kScrMaxDev = 64;
static std::mutex g_scr_mu;
static unsigned char *g_scr_ptr[kScrMaxDev];

int vxm_scratch_setup(vxm_ctx *ctx) {
    ctx->scratch = nullptr;
    if (ctx->device < 0 || ctx->device >= kScrMaxDev) {
        ctx->scratch_err = "device index beyond the scratch table";
        return VXM_OK;
    }
    std::lock_guard<std::mutex> lock(g_scr_mu);
    if (!g_scr_ptr[ctx->device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            ctx->scratch_err = std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e);
            return VXM_OK;   // only the allocation-free entry reports it
        }
        // all zero once, so the split words hold tag 0, which no launch uses
        const int64_t n16 = (int64_t)(kScratchBytes / 16);
        hipLaunchKernelGGL(k_fill_zero, dim3(1024), dim3(256), 0, ctx->stream, (uint4 *)p, n16);
        if (hipGetLastError() != hipSuccess || hipStreamSynchronize(ctx->stream) != hipSuccess) {
            (void)hipGetLastError();
            ctx->scratch_err = "clearing the scratch array failed";
            return VXM_OK;
        }
        g_scr_ptr[ctx->device] = (unsigned char *)p;
    }
    ctx->scratch = g_scr_ptr[ctx->device];
    return VXM_OK;
}

extern "C" size_t vxm_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int vxm_mul_mat_q8_0_noalloc(vxm_ctx *ctx, const vxm_weight *w, const float *x_dev, int64_t M,
                                        float *y_dev) {
    int rc = check_mm(ctx, w, x_dev, x_dev, M, y_dev);
    if (rc) return rc;
    if (!ctx->scratch) return vxm_fail(ctx, VXM_ERR_BACKEND, "mul_mat_noalloc: no scratch (%s)", ctx->scratch_err.c_str());
    const int64_t K = w->k;
    const size_t qbytes = ((size_t)M * K + 255) & ~(size_t)255;
    const size_t abytes = qbytes + (((size_t)M * (K / VXM_QK) * 2 + 255) & ~(size_t)255);
    if (abytes > kScrGeneral)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG,
                        "mul_mat_noalloc: the quantized %lld x %lld activation needs %zu B; the scratch holds %zu B",
                        (long long)M, (long long)K, abytes, kScrGeneral);
    unsigned char *base = ctx->scratch;
    unsigned char *gen = base + kScrCnt + kScrWords;
    int8_t *xq = (int8_t *)gen;
    uint16_t *xd = (uint16_t *)(gen + qbytes);
    // the last 256 bytes of the counter region hold the split tag word
    const MmWork wk{(uint64_t *)(base + kScrCnt), kScrWords, (int *)base, (kScrCnt - 256) / sizeof(int),
                    (float *)(gen + abytes), kScrGeneral - abytes, (uint32_t *)(base + kScrCnt - 256)};
    rc = vxm_launch_quantize(ctx, x_dev, M, K, ctx->quant_variant, xq, xd);
    if (rc) return rc;
    return launch_mul_mat(ctx, w, xq, xd, M, y_dev, &wk);
}

// ---- many GEMVs in one launch, and the read floor ---------------------------
template <int C, int R>
static int launch_gemv_multi(vxm_ctx *ctx, int n, const vxm_weight *const *w, const int8_t *const *xq,
                             const uint16_t *const *xd, int64_t M, float *const *y) {
    GemvBatch b;
    int wg = 0;
    for (int i = 0; i < n; i++) {
        const int waves = (int)((w[i]->n + R - 1) / R);
        b.it[i] = GemvItem{w[i]->qs, w[i]->dg, xq[i], xd[i], y[i], (int)w[i]->n, wg};
        wg += (waves + 3) / 4;
    }
    b.n_items = n;
    hipLaunchKernelGGL((k_gemv_q8_0_multi<C, R>), dim3(wg), dim3(256), 0, ctx->stream, b, (int)M);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}

extern "C" int vxm_mul_mat_q8_0_q8_0_multi(vxm_ctx *ctx, int32_t n, const vxm_weight *const *w,
                                           const int8_t *const *xq_dev, const uint16_t *const *xd_dev, int64_t M,
                                           float *const *y_dev) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (n < 0 || (n > 0 && (!w || !xq_dev || !xd_dev || !y_dev)) || M < 0)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "mul_mat_multi: bad arguments (n=%d M=%lld)", n, (long long)M);
    for (int i = 0; i < n; i++) {
        int rc = check_mm(ctx, w[i], xq_dev[i], xd_dev[i], M, y_dev[i]);
        if (rc) return rc;
        if (w[i]->k != w[0]->k)
            return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "mul_mat_multi: product %d has K %lld, product 0 has %lld", i,
                            (long long)w[i]->k, (long long)w[0]->k);
    }
    if (n == 0 || M == 0) return VXM_OK;
    // one launch per 64 products where the chunked GEMV takes the shape; else each
    // product on the kernel vxm_mul_mat_q8_0_q8_0 picks
    const int64_t K = w[0]->k;
    bool chunked = !use_mfma(ctx, M) && (K / 1024 == 1 || K / 1024 == 2 || K / 1024 == 4 || K / 1024 == 6) &&
                   K % 1024 == 0;
    for (int i = 0; chunked && i < n; i++) chunked = w[i]->dg != nullptr;
    if (!chunked) {
        for (int i = 0; i < n; i++) {
            int rc = vxm_launch_mul_mat(ctx, w[i], xq_dev[i], xd_dev[i], M, y_dev[i]);
            if (rc) return rc;
        }
        return VXM_OK;
    }
    for (int i0 = 0; i0 < n; i0 += kMultiMax) {
        const int c = n - i0 < kMultiMax ? n - i0 : kMultiMax;
        int rc = VXM_OK;
        switch (K / 1024) {
            case 1: rc = launch_gemv_multi<1, 4>(ctx, c, w + i0, xq_dev + i0, xd_dev + i0, M, y_dev + i0); break;
            case 2: rc = launch_gemv_multi<2, 2>(ctx, c, w + i0, xq_dev + i0, xd_dev + i0, M, y_dev + i0); break;
            case 4: rc = launch_gemv_multi<4, 1>(ctx, c, w + i0, xq_dev + i0, xd_dev + i0, M, y_dev + i0); break;
            default: rc = launch_gemv_multi<6, 1>(ctx, c, w + i0, xq_dev + i0, xd_dev + i0, M, y_dev + i0); break;
        }
        if (rc) return rc;
    }
    return VXM_OK;
}

extern "C" int64_t vxm_stream_read_sink_words(int32_t n, const int64_t *bytes) {
    int64_t wg = 0;
    for (int i = 0; i < n; i++) wg += (bytes[i] + kReadWgBytes - 1) / kReadWgBytes;
    return 4 * wg;
}

extern "C" int vxm_stream_read(vxm_ctx *ctx, int32_t n, const void *const *ranges_dev, const int64_t *bytes,
                               uint32_t *sink_dev) {
    if (!ctx) return VXM_ERR_INVALID_ARG;
    if (n < 0 || n > kReadMax || (n > 0 && (!ranges_dev || !bytes)) || !sink_dev)
        return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "stream_read: bad arguments (n=%d, at most %d ranges)", n, kReadMax);
    ReadBatch b;
    int64_t wg = 0;
    for (int i = 0; i < n; i++) {
        if (!ranges_dev[i] || bytes[i] < 0 || bytes[i] % 16 || ((uintptr_t)ranges_dev[i] & 15))
            return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "stream_read: range %d must be 16-byte aligned, a multiple of 16 B", i);
        b.r[i] = ReadRange{(const uint4 *)ranges_dev[i], bytes[i] / 16, (int)wg};
        // (sink: 4 words per workgroup, vxm_stream_read_sink_words)
        wg += (bytes[i] + kReadWgBytes - 1) / kReadWgBytes;
        if (wg >= INT32_MAX) return vxm_fail(ctx, VXM_ERR_INVALID_ARG, "stream_read: too many bytes in one launch");
    }
    b.n = n;
    if (wg == 0) return VXM_OK;
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)wg), dim3(256), 0, ctx->stream, b, sink_dev);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}
