// qwm_q4k.h -- the wave-level Q8_K activation quantizer in its plain layout
// (qs [256] int8, d, bsums [16] as int32), used by the prefill path; the
// GEMVs' own layout and the Q4_K dots in ggml's float order are in
// qwm_exact.h.
#pragma once

#include "qwm_device.h"

namespace qwm {

// Q8_K quantization of one 256-value block by one wave (ggml-quants.c:2769-2806):
// lane L owns values 4L..4L+3.  max = the signed value of the first largest
// |x|; iscale = -127/max; q = min(127, nearest_int(iscale*x)); bsums per 16;
// d = 1/iscale.  Writes qs (256 B), d, and the 16 bsums (as int32); with
// AGENT the writes are agent-scope stores (read by other workgroups of the
// same launch); with SRC_AGENT the block is read with agent-scope loads
// (written by other workgroups of the same launch).
template <bool AGENT = false, bool SRC_AGENT = false>
QWM_DEV void quantize_block_q8K(const float * __restrict__ src, int8_t * __restrict__ qs, float * __restrict__ d_out,
                                int32_t * __restrict__ bs_out, int lane) {
    float4 v4;
    if constexpr (SRC_AGENT) {
        const uint64_t * s64 = reinterpret_cast<const uint64_t *>(src) + 2 * lane;
        const uint64_t lo = ld_agent(s64), hi = ld_agent(s64 + 1);
        v4 = make_float4(__uint_as_float((uint32_t)lo), __uint_as_float((uint32_t)(lo >> 32)),
                         __uint_as_float((uint32_t)hi), __uint_as_float((uint32_t)(hi >> 32)));
    } else {
        v4 = reinterpret_cast<const float4 *>(src)[lane];
    }
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    float a = __builtin_fabsf(v[0]);
    int ii = 0;
#pragma unroll
    for (int i = 1; i < 4; ++i)
        if (__builtin_fabsf(v[i]) > a) { a = __builtin_fabsf(v[i]); ii = i; }
    int idx = 4 * lane + ii;
    wave_best_first(a, idx);
    idx = __builtin_amdgcn_readfirstlane(idx);
    const int c = idx & 3;
    const float mine = c == 0 ? v[0] : c == 1 ? v[1] : c == 2 ? v[2] : v[3];
    const float mx = readlane_f(mine, idx >> 2);
    int q[4] = {0, 0, 0, 0};
    float d = 0.f;
    if (a != 0.f) {
        const float iscale = -127.f / mx;
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = min(127, nearest_int_mul(iscale, v[i]));
        d = 1.f / iscale;
    }
    const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                            ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
    int sm = q[0] + q[1] + q[2] + q[3];
    sm += dpp_i<0xB1>(sm);
    sm += dpp_i<0x4E>(sm);
    if constexpr (AGENT) {
        st_agent(reinterpret_cast<uint32_t *>(qs) + lane, packed);
        if ((lane & 3) == 0) st_agent(bs_out + (lane >> 2), sm);
        if (lane == 0) st_agent(d_out, d);
    } else {
        reinterpret_cast<uint32_t *>(qs)[lane] = packed;
        if ((lane & 3) == 0) bs_out[lane >> 2] = sm;
        if (lane == 0) *d_out = d;
    }
}

}  // namespace qwm
