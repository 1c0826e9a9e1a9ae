// qwm_q80.h -- the x86 Q8_0 activation quantizer by waves, the input of the
// Q8_0 expert GEMVs (q80_dot8 in qwm_exact.h).
//
// Q8_0 (ggml-common.h:251-256) is a fp16 scale and 32 int8 values, 34 bytes.
#pragma once

#include "qwm_q4k.h"

namespace qwm {

// One wave quantizes 256 floats (8 blocks) with ggml's x86 activation
// quantizer (ggml-cpu/arch/x86/quants.c:302-345): d = amax / 127 stored as
// fp16, multiplier 127 / amax, round half to even.  Lane l owns elements
// 4l..4l+3; qs gets the int8 values, d_out the 8 scales (as floats).
template <bool SRC_AGENT = false>
QWM_DEV void quantize_q80_256(const float * __restrict__ src, int8_t * __restrict__ qs, float * __restrict__ d_out,
                              int lane) {
    float4 v;
    if constexpr (SRC_AGENT) {
        const uint64_t * s64 = reinterpret_cast<const uint64_t *>(src) + 2 * lane;
        const uint64_t lo = ld_agent(s64), hi = ld_agent(s64 + 1);
        v = make_float4(__uint_as_float((uint32_t)lo), __uint_as_float((uint32_t)(lo >> 32)),
                        __uint_as_float((uint32_t)hi), __uint_as_float((uint32_t)(hi >> 32)));
    } else {
        v = reinterpret_cast<const float4 *>(src)[lane];
    }
    float amax = fmaxf(fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)), fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, WAVE));
    amax = fmaxf(amax, __shfl_xor(amax, 2, WAVE));
    amax = fmaxf(amax, __shfl_xor(amax, 4, WAVE));
    const float d = amax / 127.f;
    const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
    const uint32_t b0 = (uint32_t)((int)__builtin_rintf(v.x * id) & 0xff);
    const uint32_t b1 = (uint32_t)((int)__builtin_rintf(v.y * id) & 0xff);
    const uint32_t b2 = (uint32_t)((int)__builtin_rintf(v.z * id) & 0xff);
    const uint32_t b3 = (uint32_t)((int)__builtin_rintf(v.w * id) & 0xff);
    reinterpret_cast<uint32_t *>(qs)[lane] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
    if ((lane & 7) == 0) d_out[lane >> 3] = fp16_to_f32(f32_to_fp16(d));
}

}  // namespace qwm
