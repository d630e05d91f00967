// host_q8.cpp -- host-side helpers of the library: the GGUF Q8_0 weight
// quantizer (the rule ggml_quantize_chunk applies in tools/quantize.c:292)
// and the seeded synthetic normal generator used to build benchmark inputs.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../../include/vxm_q8.h"

namespace {

inline uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    uint32_t e = ax >> 23, man = (ax & 0x7fffffu) | 0x800000u;
    if (e < 113) {
        if (e == 0) return (uint16_t)sign;
        uint32_t sh = 126 - e;
        if (sh > 24) return (uint16_t)sign;
        uint32_t q = man >> sh, rem = man & ((1u << sh) - 1u), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = ((e - 112) << 10) | ((ax & 0x7fffffu) >> 13), rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

inline uint64_t splitmix_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

}  // namespace

// Q8_0 weight rule: per 32 values d = amax/127 (fp16, RNE), id = d ? 1/d : 0,
// qs = roundf(x * id).  Output: GGUF rows of k/32 34-byte blocks.
extern "C" int vxm_host_quantize_q8_0(const float *x, int64_t rows, int64_t k, void *gguf_rows) {
    if (!x || !gguf_rows || rows < 0 || k <= 0 || k % 32) return VXM_ERR_INVALID_ARG;
    const int64_t nb = k / 32, total = rows * nb;
    uint8_t *out = (uint8_t *)gguf_rows;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; i++) {
        const float *xb = x + i * 32;
        uint8_t *blk = out + i * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(xb[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t dh = f32_to_f16_rne(d);
        memcpy(blk, &dh, 2);
        int8_t *qs = (int8_t *)(blk + 2);
        for (int j = 0; j < 32; j++) qs[j] = (int8_t)roundf(xb[j] * id);
    }
    return VXM_OK;
}

// Seeded N(mean, std^2) floats.  SplitMix64 (the generator the reference uses
// for CFM noise, src/gen_step.c:409-431) in counter form: output t of the
// stream seeded with s is mix(s + t * 0x9E3779B97F4A7C15), t = 1, 2, ...;
// values 2j and 2j+1 are the Box-Muller pair (in double) of outputs 2j+1 and
// 2j+2.  Element i of the returned array is stream element offset + i, so any
// slice can be generated independently (and in parallel).
extern "C" int vxm_host_randn(uint64_t seed, uint64_t offset, int64_t n, float mean, float std,
                              float *out) {
    if (!out || n < 0) return VXM_ERR_INVALID_ARG;
    const uint64_t G = 0x9E3779B97F4A7C15ULL;
    const double two_pi = 6.283185307179586476925286766559;
    const double inv53 = 1.0 / 9007199254740992.0;
#pragma omp parallel for schedule(static, 4096)
    for (int64_t i = 0; i < n; i++) {
        const uint64_t e = offset + (uint64_t)i, j = e >> 1;
        const uint64_t z1 = splitmix_mix(seed + (2 * j + 1) * G);
        const uint64_t z2 = splitmix_mix(seed + (2 * j + 2) * G);
        const double u1 = (double)((z1 >> 11) + 1) * inv53;
        const double u2 = (double)(z2 >> 11) * inv53;
        const double r = sqrt(-2.0 * log(u1));
        const double v = (e & 1) ? r * sin(two_pi * u2) : r * cos(two_pi * u2);
        out[i] = (float)((double)mean + (double)std * v);
    }
    return VXM_OK;
}
