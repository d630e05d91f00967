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

template <int C, int R>
static void launch_gemv_c(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd,
                          int64_t M, float *y) {
    const int waves = (int)((w->n + R - 1) / R);
    const int grid = (waves + 3) / 4;
    hipLaunchKernelGGL((k_gemv_q8_0<C, R>), dim3(grid), dim3(256), 0, ctx->stream, w->qs, w->dg, xq, xd,
                       y, (int)w->n, (int)M);
}

int vxm_launch_mul_mat(vxm_ctx *ctx, const vxm_weight *w, const int8_t *xq, const uint16_t *xd,
                       int64_t M, float *y) {
    if (M <= 0) return VXM_OK;
    const int64_t K = w->k;
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
