// host_cfm.cpp -- host-side scalar math of the LocDiT / CFM driver: the
// sinusoidal timestep embedding, the CFM time schedules and the zero-init
// step count.  These run on the host in the reference as well (scalars and
// tables fed to the graph), so they are computed here with the C library's
// expf / sinf / cosf in the reference's operation order and BF16 roundings.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../../include/vxm_q8.h"

namespace {

// float -> bf16 -> float, round to nearest even; NaN stays a (quiet) NaN.
inline float bf16r(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) {
        x = (x | 0x00400000u) & 0xffff0000u;
    } else {
        const uint32_t lsb = (x >> 16) & 1u;
        x = (x + 0x7fffu + lsb) & 0xffff0000u;
    }
    float r;
    memcpy(&r, &x, 4);
    return r;
}

}  // namespace

// dit_sinusoidal_t_embed (src/locdit.c:163-188): freq_i = bf16(expf(bf16(bf16(i) *
// (-ln 10000 / (half - 1))))), angle_i = bf16(freq_i * bf16(t * 1000)),
// out = [bf16(sin(angle)), bf16(cos(angle))].
extern "C" int vxm_host_sinusoid_embed(float t, int32_t dim, float *out) {
    if (!out || dim <= 0 || dim % 2) return VXM_ERR_INVALID_ARG;
    const int32_t half = dim / 2;
    const float log_max_period = logf(10000.0f);
    const float denom = half > 1 ? (float)(half - 1) : 1.0f;
    const float scaled_t = bf16r(t * 1000.0f);
    for (int32_t i = 0; i < half; i++) {
        const float exponent = bf16r(bf16r((float)i) * (-log_max_period / denom));
        const float freq = bf16r(expf(exponent));
        const float angle = bf16r(freq * scaled_t);
        out[i] = bf16r(sinf(angle));
        out[half + i] = bf16r(cosf(angle));
    }
    return VXM_OK;
}

// vcpm_cfm_sway_t_bf16 (src/cfm_solver.c:27-37) for schedule VXM_CFM_SWAY:
// base = bf16(1 - step/n), t = bf16(base + bf16(bf16(bf16(cos(bf16(bf16(pi/2) *
// base))) - 1) + base)); VXM_CFM_UNIFORM: t = bf16(1 - step/n).
extern "C" float vxm_host_cfm_t(int32_t step, int32_t n_steps, int32_t schedule) {
    if (n_steps <= 0 || step < 0 || step > n_steps) return 0.0f;
    const float base = bf16r(1.0f - (float)step / (float)n_steps);
    if (schedule == VXM_CFM_UNIFORM) return base;
    const float half_pi = bf16r(1.57079632679489661923f);
    const float angle = bf16r(half_pi * base);
    const float cosine = bf16r(cosf(angle));
    const float inner = bf16r(bf16r(cosine - 1.0f) + base);
    return bf16r(base + inner);
}

// vcpm_cfm_zero_star_steps (src/gen_step.c:50-54): the first steps whose
// velocity is zero (skipped) under CFG-Zero*.
extern "C" int32_t vxm_host_cfm_zero_star_steps(int32_t n_steps) {
    if (n_steps <= 1) return 0;
    const int32_t z = (int32_t)(((float)n_steps + 1.0f) * 0.04f);
    return z > 1 ? z : 1;
}

// The NEOX rope cache of ggml_rope_ext as the reference's CPU backend builds it
// (src/minicpm4.c:165-223 calling ggml_rope_ext; ggml-cpu's rope cache):
// theta_scale = powf(base, -2 / head_dim); for position p, theta_0 = p,
// theta_{i+1} = theta_i * theta_scale, angle_i = theta_i / ff_i (ff NULL: no
// factors); out[(p - pos0) * head_dim + 2i] = cosf(angle_i), [.. + 2i + 1] = sinf.
extern "C" int vxm_host_rope_cache(float base, int32_t head_dim, const float *ff, int32_t pos0, int32_t n_pos,
                                   float *out) {
    if (!out || head_dim <= 0 || head_dim % 2 || n_pos < 0 || pos0 < 0) return VXM_ERR_INVALID_ARG;
    const int32_t half = head_dim / 2;
    const float theta_scale = powf(base, -2.0f / (float)head_dim);
    for (int32_t p = 0; p < n_pos; p++) {
        float theta = (float)(pos0 + p);
        float *o = out + (int64_t)p * head_dim;
        for (int32_t i = 0; i < half; i++) {
            const float f = ff ? ff[i] : 1.0f;
            const float th = theta / f;
            o[2 * i] = cosf(th);
            o[2 * i + 1] = sinf(th);
            theta *= theta_scale;
        }
    }
    return VXM_OK;
}
