// q8_matmul.hip -- activation quantization and the Q8_0 x Q8_0 matmul
// (ggml_mul_mat on GGUF Q8_0 weights) for gfx950.
//
// Semantics (ggml vec_dot_q8_0_q8_0, called from ggml_mul_mat at
// src/projections.h:24-29 and src/minicpm4.c:270-279,415,441-458):
//   y[m][n] = sum_b float(sumi[m][n][b]) * (float(d_w[n][b]) * float(d_x[m][b]))
//   sumi = sum over the 32 int8 pairs of block b (exact int32).
// Every kernel here forms exactly these per-block fp32 terms; only the order
// of the fp32 additions over b differs from ggml's (a tree over lanes).
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
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
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
// ---------------------------------------------------------------------------
template <int C, int R>
__global__ __launch_bounds__(256) void k_gemv_q8_0(const int8_t *__restrict__ qs,
                                                   const uint16_t *__restrict__ dg,
                                                   const int8_t *__restrict__ xq,
                                                   const uint16_t *__restrict__ xd, float *__restrict__ y,
                                                   int N, int M) {
    constexpr int K = C * 1024;
    constexpr int NB = K / 32;
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
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

// ---------------------------------------------------------------------------
// Generic GEMV, any K % 32 == 0: one wave per row, lanes stride over the
// row's 16-byte half blocks (the two halves of a block sit in lanes 2p, 2p+1).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_gemv_q8_0_generic(const int8_t *__restrict__ qs,
                                                           const uint16_t *__restrict__ d,
                                                           const int8_t *__restrict__ xq,
                                                           const uint16_t *__restrict__ xd,
                                                           float *__restrict__ y, int N, int K, int M) {
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
            acc += (float)s * sc;
        }
        acc = pair_sum(acc);
        if (lane == 0) y[(int64_t)m * N + row] = acc;
    }
}

// Debug: exact int32 per-block sums, one thread per (m, n, b).
__global__ void k_block_dots(const int8_t *__restrict__ qs, const int8_t *__restrict__ xq, int64_t N,
                             int64_t K, int64_t M, int32_t *__restrict__ out) {
    const int64_t nb = K / 32;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= M * N * nb) return;
    const int64_t b = i % nb, n = (i / nb) % N, m = i / (nb * N);
    const v4i *a = (const v4i *)(qs + n * K + b * 32);
    const v4i *x = (const v4i *)(xq + m * K + b * 32);
    int s = dot16v(a[0], x[0], 0);
    s = dot16v(a[1], x[1], s);
    out[i] = s;
}


// ---------------------------------------------------------------------------
// Q8_0 x Q8_0 GEMM on int8 MFMA, for M rows of activations (prefill, CFM).
// gfx950's v_mfma_i32_32x32x32_i8 contracts K = 32 -- exactly one Q8_0
// block -- so one instruction yields the exact int32 block sums of a 32 x 32
// sub-tile.  Lane l supplies A row l % 32 and B row (weight row) l % 32, k
// half l / 32; result register v of lane l is row 8(v/4) + 4(l/32) + v%4,
// column l % 32.  Each lane then adds term = (float)sumi * (d_w * d_x) to its
// fp32 accumulators block after block: ggml's generic vec_dot_q8_0_q8_0
// order, so without a K split the output is bit-exact with a sequential
// per-block fp32 sum.  (Per block and element that is four VALU operations
// against 1/1024 of an MFMA, which bounds the MFMA duty cycle.)
//
// Workgroup: 256 threads (4 waves) on a 64 (M) x 64 (N) tile, wave w on the
// 32 x 32 sub-tile (w / 2, w % 2).  K moves through LDS GKS blocks at a time,
// double-buffered through registers.  Tiles are ordered so that the M tiles
// sharing one weight tile run on one XCD (workgroups are dispatched round
// robin over the 8 XCDs): the weight tile is fetched into that XCD's L2 once.
// blockIdx.y = K split: split z adds blocks [z*bps, (z+1)*bps) and writes its
// partial tile to part[z] (the caller reduces), or y directly when splits = 1.
// ---------------------------------------------------------------------------
typedef int v16i __attribute__((ext_vector_type(16)));
constexpr int GM = 64, GN = 64, GKS = 4;     // tile M, N; blocks per LDS stage
constexpr int GROW = GKS * 32 + 16;          // padded LDS row (bytes) against bank conflicts

__global__ __launch_bounds__(256) void k_gemm_q8_0_mfma(const int8_t *__restrict__ xq, const uint16_t *__restrict__ xd,
                                                        const int8_t *__restrict__ wq, const uint16_t *__restrict__ wd,
                                                        float *__restrict__ y, int M, int N, int K, int tiles_m,
                                                        int tiles_n, int bps) {
    __shared__ __align__(16) int8_t As[2][GM * GROW];
    __shared__ __align__(16) int8_t Bs[2][GN * GROW];
    __shared__ __align__(16) float Ad[2][GKS][GM];
    __shared__ __align__(16) float Bd[2][GKS][GN];
    const int id = blockIdx.x, xcd = id % 8, k8 = id / 8;
    const int tn = (k8 / tiles_m) * 8 + xcd, tm = k8 % tiles_m;
    if (tn >= tiles_n) return;
    const int m0 = tm * GM, n0 = tn * GN;
    const int nb = K / 32;
    const int b0 = blockIdx.y * bps, b1 = min(nb, b0 + bps);
    if (b0 >= b1) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // stage loader: thread t moves 16-byte chunks c = t, t + 256 of each 64 x 128-byte tile
    // (row c / 8, chunk c % 8) and one scale (block t / 64, row t % 64) of each side
    auto load = [&](int kb0, v4i (&ra)[2], v4i (&rb)[2], float &sa, float &sb) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int c = tid + 256 * h, r = c >> 3, ch = c & 7, kb = kb0 + (ch >> 1);
            const bool okk = kb < b1;
            const int m = m0 + r, n = n0 + r;
            ra[h] = (okk && m < M) ? *(const v4i *)(xq + (int64_t)m * K + kb * 32 + (ch & 1) * 16) : v4i{0, 0, 0, 0};
            rb[h] = (okk && n < N) ? *(const v4i *)(wq + (int64_t)n * K + kb * 32 + (ch & 1) * 16) : v4i{0, 0, 0, 0};
        }
        const int kb = kb0 + (tid >> 6), r = tid & 63;
        sa = (kb < b1 && m0 + r < M) ? vxm_h2f(xd[(int64_t)(m0 + r) * nb + kb]) : 0.0f;
        sb = (kb < b1 && n0 + r < N) ? vxm_h2f(wd[(int64_t)(n0 + r) * nb + kb]) : 0.0f;
    };
    auto store = [&](int buf, const v4i (&ra)[2], const v4i (&rb)[2], float sa, float sb) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int c = tid + 256 * h, r = c >> 3, ch = c & 7;
            *(v4i *)(As[buf] + r * GROW + ch * 16) = ra[h];
            *(v4i *)(Bs[buf] + r * GROW + ch * 16) = rb[h];
        }
        Ad[buf][tid >> 6][tid & 63] = sa;
        Bd[buf][tid >> 6][tid & 63] = sb;
    };

    float acc[16];
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = 0.0f;
    v4i ra[2], rb[2];
    float sa, sb;
    load(b0, ra, rb, sa, sb);
    store(0, ra, rb, sa, sb);
    __syncthreads();
    int buf = 0;
    for (int kb0 = b0; kb0 < b1; kb0 += GKS) {
        const bool more = kb0 + GKS < b1;
        if (more) load(kb0 + GKS, ra, rb, sa, sb);
        const int8_t *arow = As[buf] + (wm * 32 + (lane & 31)) * GROW + (lane >> 5) * 16;
        const int8_t *brow = Bs[buf] + (wn * 32 + (lane & 31)) * GROW + (lane >> 5) * 16;
#pragma unroll
        for (int kb = 0; kb < GKS; kb++) {
            if (kb0 + kb >= b1) break;
            const v4i a = *(const v4i *)(arow + kb * 32);
            const v4i b = *(const v4i *)(brow + kb * 32);
            const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, v16i{}, 0, 0, 0);
            const float dw = Bd[buf][kb][wn * 32 + (lane & 31)];
            const float *dxr = Ad[buf][kb] + wm * 32 + 4 * (lane >> 5);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 dx = *(const float4 *)(dxr + 8 * g);
                const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int v = 4 * g + e;
                    acc[v] = acc[v] + (float)c[v] * (dw * dxv[e]);
                }
            }
        }
        if (more) {
            store(buf ^ 1, ra, rb, sa, sb);
            buf ^= 1;
        }
        __syncthreads();
    }
    float *out = y + (int64_t)blockIdx.y * M * N;
    const int n = n0 + wn * 32 + (lane & 31);
    if (n < N) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = m0 + wm * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
            if (m < M) out[(int64_t)m * N + n] = acc[v];
        }
    }
}

// y = sum over the K splits of part[z], added in split order.
__global__ void k_split_reduce(const float *__restrict__ part, int splits, int64_t mn, float *__restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= mn) return;
    float s = part[i];
    for (int z = 1; z < splits; z++) s = s + part[(int64_t)z * mn + i];
    y[i] = s;
}

static int launch_gemm(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd, int64_t M,
                       float *y) {
    const int N = (int)w->n, K = (int)w->k, nb = K / 32;
    const int tiles_m = (int)((M + GM - 1) / GM), tiles_n = (N + GN - 1) / GN;
    const int grid_x = 8 * tiles_m * ((tiles_n + 7) / 8);
    // split K until the grid covers the CUs (each split at least one LDS stage)
    int splits = 1;
    while ((int64_t)tiles_m * tiles_n * splits < ctx->n_cu && nb / (splits * 2) >= GKS) splits *= 2;
    const int bps = (nb + splits - 1) / splits;
    splits = (nb + bps - 1) / bps;   // every split then owns at least one block
    float *dst = y;
    if (splits > 1) {
        int rc = vxm_ensure_split(ctx, (size_t)splits * M * N * sizeof(float));
        if (rc) return rc;
        dst = (float *)ctx->split_buf;
    }
    hipLaunchKernelGGL(k_gemm_q8_0_mfma, dim3(grid_x, splits), dim3(256), 0, ctx->stream, xq, xd, w->qs, w->d, dst,
                       (int)M, N, K, tiles_m, tiles_n, bps);
    VXM_CHECK_LAUNCH(ctx);
    if (splits > 1) {
        const int64_t mn = M * N;
        hipLaunchKernelGGL(k_split_reduce, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, ctx->stream, dst, splits,
                           mn, y);
        VXM_CHECK_LAUNCH(ctx);
    }
    return VXM_OK;
}

template <int C, int R>
static void launch_gemv_c(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd,
                          int64_t M, float *y) {
    const int waves = (int)((w->n + R - 1) / R);
    const int grid = (waves + 3) / 4;
    hipLaunchKernelGGL((k_gemv_q8_0<C, R>), dim3(grid), dim3(256), 0, ctx->stream, w->qs, w->dg, xq, xd,
                       y, (int)w->n, (int)M);
}

// Rows of activations from which the MFMA GEMM replaces the weight-streaming
// GEMV (which re-reads each activation row per weight row group).
constexpr int kMfmaMinRows = 8;

int vxm_launch_mul_mat(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd,
                       int64_t M, float *y) {
    if (M <= 0) return VXM_OK;
    const int64_t K = w->k;
    const bool mfma = ctx->path == VXM_PATH_MFMA || (ctx->path == VXM_PATH_AUTO && M >= kMfmaMinRows);
    if (mfma) return launch_gemm(ctx, w, xq, xd, M, y);
    bool done = false;
    if (w->dg) {
        switch (K / 1024) {
            case 1: launch_gemv_c<1, 4>(ctx, w, xq, xd, M, y); done = true; break;
            case 2: launch_gemv_c<2, 2>(ctx, w, xq, xd, M, y); done = true; break;
            case 4: launch_gemv_c<4, 1>(ctx, w, xq, xd, M, y); done = true; break;
            case 6: launch_gemv_c<6, 1>(ctx, w, xq, xd, M, y); done = true; break;
            default: break;
        }
    }
    if (!done) {
        const int grid = (int)((w->n + 3) / 4);
        hipLaunchKernelGGL(k_gemv_q8_0_generic, dim3(grid), dim3(256), 0, ctx->stream, w->qs, w->d, xq, xd,
                           y, (int)w->n, (int)K, (int)M);
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
    const int64_t grid = (total + 255) / 256;
    hipLaunchKernelGGL(k_block_dots, dim3((unsigned)grid), dim3(256), 0, ctx->stream, w->qs, xq_dev, w->n,
                       w->k, M, out_dev);
    VXM_CHECK_LAUNCH(ctx);
    return VXM_OK;
}
