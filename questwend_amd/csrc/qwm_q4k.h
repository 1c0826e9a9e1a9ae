// qwm_q4k.h -- device building blocks of the Q4_K x Q8_K expert GEMVs, shared
// by the per-op kernels (qwm_moe.hip) and the fused verify step (qwm_step.hip):
// the wave-level Q8_K activation quantizer and the 16-byte-chunk dot of one
// Q4_K row against one token's Q8_K activations.
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

// ======================================================================
// Q4_K x Q8_K GEMV machinery
// ======================================================================

// Activation bytes of one token for one 16-byte quant chunk (sub-blocks 2j
// and 2j+1 of super-block sb, half h): 16 q8 values for the low nibbles,
// 16 for the high nibbles, the block scale and the two 16-value bsums.
struct ActChunk {
    uint4 lo, hi;
    float d;
    int32_t bs_lo, bs_hi;
};

// dd[sb * DS] is block sb's scale and bs[sb * BS + i] its i-th bsum (the
// padded layouts give every block's scale and bsums a cache line of their own).
template <int DS = 1, int BS = 16>
QWM_DEV void load_act_chunk(ActChunk & A, const int8_t * qs, const float * dd, const int32_t * bs, int c) {
    const int sb = c >> 3, p = c & 7, j = p >> 1, h = p & 1;
    const int8_t * q = qs + sb * QK_K + 64 * j + 16 * h;
    A.lo = *reinterpret_cast<const uint4 *>(q);
    A.hi = *reinterpret_cast<const uint4 *>(q + 32);
    A.d = dd[sb * DS];
    A.bs_lo = bs[sb * BS + 4 * j + h];
    A.bs_hi = bs[sb * BS + 4 * j + 2 + h];
}

// Weight data of one chunk: the 16 quant bytes and the block header.
struct WChunk {
    uint4 q, hd;
};

QWM_DEV void load_w_chunk(WChunk & W, const uint8_t * row, int c) {
    const int sb = c >> 3, p = c & 7;
    const uint8_t * blk = row + sb * 144;
    W.hd = *reinterpret_cast<const uint4 *>(blk);
    W.q = *reinterpret_cast<const uint4 *>(blk + 16 + 16 * p);
}

// Contribution of one chunk to d*sum(sc*q4*q8) - dmin*sum(m*bsum).
QWM_DEV float chunk_dot(const WChunk & W, const ActChunk & A, int c, float acc) {
    const int p = c & 7, j = p >> 1;
    int sc_lo, m_lo, sc_hi, m_hi;
    q4k_scale_min_reg(2 * j, W.hd.y, W.hd.z, W.hd.w, sc_lo, m_lo);
    q4k_scale_min_reg(2 * j + 1, W.hd.y, W.hd.z, W.hd.w, sc_hi, m_hi);
    const uint32_t m4 = 0x0F0F0F0Fu;
    int s_lo = 0, s_hi = 0;
    s_lo = dot4(W.q.x & m4, A.lo.x, s_lo);
    s_lo = dot4(W.q.y & m4, A.lo.y, s_lo);
    s_lo = dot4(W.q.z & m4, A.lo.z, s_lo);
    s_lo = dot4(W.q.w & m4, A.lo.w, s_lo);
    s_hi = dot4((W.q.x >> 4) & m4, A.hi.x, s_hi);
    s_hi = dot4((W.q.y >> 4) & m4, A.hi.y, s_hi);
    s_hi = dot4((W.q.z >> 4) & m4, A.hi.z, s_hi);
    s_hi = dot4((W.q.w >> 4) & m4, A.hi.w, s_hi);
    const int isum = sc_lo * s_lo + sc_hi * s_hi;
    const int imin = m_lo * A.bs_lo + m_hi * A.bs_hi;
    const float d = A.d * fp16_to_f32((uint16_t)(W.hd.x & 0xffff));
    const float dmin = A.d * fp16_to_f32((uint16_t)(W.hd.x >> 16));
    acc = __builtin_fmaf(d, (float)isum, acc);
    return __builtin_fmaf(-dmin, (float)imin, acc);
}

// The same chunk with the block header shared across lanes: lane c loads its
// 16 quant bytes and dword (c & 3) of its block's 16-byte header (8 lanes per
// block, so every quad holds the whole header); chunk_dot_s rebuilds the
// header with quad broadcasts.  Five registers per lane instead of eight.
// All four lanes of a quad must be active in chunk_dot_s.
struct WChunkS {
    uint4 q;
    uint32_t h;
};

QWM_DEV void load_w_chunk_s(WChunkS & W, const uint8_t * row, int c) {
    const int sb = c >> 3, p = c & 7;
    const uint8_t * blk = row + sb * 144;
    W.h = reinterpret_cast<const uint32_t *>(blk)[c & 3];
    W.q = *reinterpret_cast<const uint4 *>(blk + 16 + 16 * p);
}

// One lane's chunk of one row decoded once for every token: the unpacked
// nibbles, both sub-blocks' scales and mins, and the block's d and dmin.
struct RowChunk {
    uint32_t lo[4], hi[4];
    int sc_lo, m_lo, sc_hi, m_hi;
    float d, dmin;
};

QWM_DEV void decode_chunk_s(const WChunkS & W, int c, RowChunk & R) {
    const int h = (int)W.h;
    const uint32_t h0 = (uint32_t)dpp_i<0x00>(h), h1 = (uint32_t)dpp_i<0x55>(h);
    const uint32_t h2 = (uint32_t)dpp_i<0xAA>(h), h3 = (uint32_t)dpp_i<0xFF>(h);
    const int j = 2 * ((c & 7) >> 1);
    q4k_scale_min_reg(j, h1, h2, h3, R.sc_lo, R.m_lo);
    q4k_scale_min_reg(j + 1, h1, h2, h3, R.sc_hi, R.m_hi);
    const uint32_t m4 = 0x0F0F0F0Fu;
    const uint32_t q[4] = {W.q.x, W.q.y, W.q.z, W.q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) { R.lo[i] = q[i] & m4; R.hi[i] = (q[i] >> 4) & m4; }
    R.d = fp16_to_f32((uint16_t)(h0 & 0xffff));
    R.dmin = fp16_to_f32((uint16_t)(h0 >> 16));
}

// The same arithmetic as chunk_dot (identical operations and order).
QWM_DEV float token_dot_acc(const RowChunk & R, const ActChunk & A, float acc) {
    int s_lo = 0, s_hi = 0;
    s_lo = dot4(R.lo[0], A.lo.x, s_lo);
    s_lo = dot4(R.lo[1], A.lo.y, s_lo);
    s_lo = dot4(R.lo[2], A.lo.z, s_lo);
    s_lo = dot4(R.lo[3], A.lo.w, s_lo);
    s_hi = dot4(R.hi[0], A.hi.x, s_hi);
    s_hi = dot4(R.hi[1], A.hi.y, s_hi);
    s_hi = dot4(R.hi[2], A.hi.z, s_hi);
    s_hi = dot4(R.hi[3], A.hi.w, s_hi);
    const int isum = R.sc_lo * s_lo + R.sc_hi * s_hi;
    const int imin = R.m_lo * A.bs_lo + R.m_hi * A.bs_hi;
    const float d = A.d * R.d;
    const float dmin = A.d * R.dmin;
    acc = __builtin_fmaf(d, (float)isum, acc);
    return __builtin_fmaf(-dmin, (float)imin, acc);
}
QWM_DEV float token_dot(const RowChunk & R, const ActChunk & A) { return token_dot_acc(R, A, 0.f); }

QWM_DEV float chunk_dot_s(const WChunkS & W, const ActChunk & A, int c, float acc) {
    WChunk w;
    w.q = W.q;
    const int h = (int)W.h;
    w.hd.x = (uint32_t)dpp_i<0x00>(h);
    w.hd.y = (uint32_t)dpp_i<0x55>(h);
    w.hd.z = (uint32_t)dpp_i<0xAA>(h);
    w.hd.w = (uint32_t)dpp_i<0xFF>(h);
    return chunk_dot(w, A, c, acc);
}

// Down-projection rows with 8 lanes per row: lane c8 of a row takes chunk c8
// of each of the row's NB Q4_K blocks (every lane works for any FFN width
// that is a multiple of 256) and accumulates them in block order; row8_sum
// adds the row's 8 partial sums by quad butterflies and a row rotation that
// brings lane i + 4 to lane i, which leaves the row's sum in the first four
// lanes of its group.
template <int NB>
QWM_DEV void load_row8(WChunkS (&W)[NB], const uint8_t * row, int c8) {
#pragma unroll
    for (int q = 0; q < NB; ++q) load_w_chunk_s(W[q], row, 8 * q + c8);
}

// acc[i] = this lane's partial dot of the row with the Q8_K activations of
// token slot i (i < n) held in LDS at qs + i * QS, dd + i * QS / 256,
// bs + i * QS / 16.
template <int NB, int MAXP, int QS>
QWM_DEV void row8_dots(float (&acc)[MAXP], const WChunkS (&W)[NB], int n, const int8_t * qs, const float * dd,
                       const int32_t * bs, int c8) {
#pragma unroll
    for (int i = 0; i < MAXP; ++i) acc[i] = 0.f;
#pragma unroll
    for (int q = 0; q < NB; ++q) {
        RowChunk R;
        decode_chunk_s(W[q], 8 * q + c8, R);
#pragma unroll
        for (int i = 0; i < MAXP; ++i)
            if (i < n) {
                ActChunk A;
                load_act_chunk(A, qs + i * QS, dd + i * (QS / QK_K), bs + i * (QS / 16), 8 * q + c8);
                acc[i] = token_dot_acc(R, A, acc[i]);
            }
    }
}

QWM_DEV float row8_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    return v + dpp_f<0x12C>(v);                  // row_ror:12: lane i receives lane i + 4 of its row
}

}  // namespace qwm
