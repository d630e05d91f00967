// vxm_ops.h -- launchers of the MiniCPM4 block kernels (ops.hip).
#pragma once
#include "vxm_internal.h"

// rows output rows; with seg_rows > 0 the h / delta rows are seg_rows of every seg_stride
int vxm_launch_rmsnorm(vxm_ctx *ctx, float *h, vxm_parts delta, float res_scale, const float *gain,
                       int64_t rows, int64_t n, float eps, float *y, int8_t *xq, uint16_t *xd, int variant,
                       int seg_rows = 0, int seg_stride = 0);
int vxm_launch_rope_kv(vxm_ctx *ctx, vxm_parts qkv, int64_t M, int nh, int nkv, int hd, int pos0, int S,
                       const float2 *cs, int cs_rows, int no_rope, float *q_out, uint16_t *kc,
                       uint16_t *vc, int cap, int64_t seg_stride, int cache_pos0);
// xq != nullptr: the output goes out as Q8_0 rows (xq, xd; quantization variant)
// instead, fused into the MFMA kernel; out is then scratch for the other kernel
int vxm_launch_attention(vxm_ctx *ctx, const float *q, const uint16_t *kc, const uint16_t *vc, float *out,
                         int64_t M, int nh, int nkv, int hd, int cap, int64_t seg_stride, int S, int kv_base,
                         int causal, int8_t *xq = nullptr, uint16_t *xd = nullptr, int variant = 0);
int vxm_launch_swiglu_quant(vxm_ctx *ctx, vxm_parts gu, int64_t M, int64_t F, int64_t ld, int8_t *xq,
                            uint16_t *xd, float *p_out, int variant);
int vxm_launch_residual(vxm_ctx *ctx, float *h, vxm_parts delta, float scale, int64_t n);
int vxm_launch_bias_bf16(vxm_ctx *ctx, const float *x, const float *bias, float *y, int64_t rows, int64_t n);
bool vxm_attention_local_fits(int S, int hd);
int vxm_launch_attention_local(vxm_ctx *ctx, vxm_parts qkv, int64_t M, int nh, int nkv, int hd, int S, int pos0,
                               const float2 *cs, int cs_rows, int no_rope, int8_t *xq, uint16_t *xd, int variant);
