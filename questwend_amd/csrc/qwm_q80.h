// qwm_q80.h -- Q8_0 expert slabs on gfx950: per-lane block dots against
// Q8_0 activations, and the x86 Q8_0 activation quantizer by waves.
//
// Q8_0 (ggml-common.h:251-256) is a fp16 scale and 32 int8 weights, 34 bytes,
// so every other block starts 2 bytes off dword alignment.  A lane owns one
// block and loads the 9 aligned dwords around it (start 34c - 2 (c & 1));
// the block's activations are shifted into the same window once, with zero
// bytes facing the scale bytes, so nine v_dot4_i32_i8 give the exact
// 32-element integer dot with no byte shuffling of the weights.  A row of K
// weights needs K / 32 even (K a multiple of 64): then the last block is odd
// and its window ends at the row's end.
#pragma once

#include "qwm_q4k.h"

namespace qwm {

constexpr int QK8_0_ = 32;

struct W80 {
    uint32_t w[9];
};

// Block c of a row.
QWM_DEV void load_w80(W80 & W, const uint8_t * row, int c) {
    typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
    const uint32_t * p = reinterpret_cast<const uint32_t *>(row + 34 * c - 2 * (c & 1));
    const u32x4_a4 v0 = *reinterpret_cast<const u32x4_a4 *>(p);
    const u32x4_a4 v1 = *reinterpret_cast<const u32x4_a4 *>(p + 4);
    W.w[0] = v0.x; W.w[1] = v0.y; W.w[2] = v0.z; W.w[3] = v0.w;
    W.w[4] = v1.x; W.w[5] = v1.y; W.w[6] = v1.z; W.w[7] = v1.w;
    W.w[8] = p[8];
}

// Activation block c: 32 int8 at qs + 32 c (16-byte aligned) and its scale,
// shifted into the window of weight block c.
struct A80 {
    uint32_t a[9];
    float d;
};

QWM_DEV void load_a80(A80 & A, const int8_t * qs, const float * d, int c) {
    const uint4 q0 = *reinterpret_cast<const uint4 *>(qs + 32 * c);
    const uint4 q1 = *reinterpret_cast<const uint4 *>(qs + 32 * c + 16);
    const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    if (c & 1) {
        A.a[0] = 0;
#pragma unroll
        for (int i = 1; i < 9; ++i) A.a[i] = q[i - 1];
    } else {
        A.a[0] = q[0] << 16;
#pragma unroll
        for (int i = 1; i < 8; ++i) A.a[i] = __builtin_amdgcn_alignbit(q[i], q[i - 1], 16);
        A.a[8] = q[7] >> 16;
    }
    A.d = d[c];
}

// acc + d_w * d_x * (exact block dot)
QWM_DEV float dot80(const W80 & W, const A80 & A, int c, float acc) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 9; ++i) s = dot4(W.w[i], A.a[i], s);
    const float dw = fp16_to_f32((uint16_t)(W.w[0] >> ((c & 1) ? 16 : 0)));
    return __builtin_fmaf(dw * A.d, (float)s, acc);
}

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

// Format policies of the expert GEMVs.  Activation rows: qs [K] int8 plus,
// for Q4_K (Q8_K activations), d [K / 256] and bsums [K / 16]; for Q8_0, d
// [K / 32].  A "chunk" c is one lane's share of a row: 16 quant bytes of a
// Q4_K block, or one Q8_0 block.
struct FmtQ4K {
    using W = WChunk;
    using A = ActChunk;
    static constexpr int CHUNK = 32;        // weights per chunk
    static QWM_DEV size_t row_bytes(int K) { return (size_t)(K / QK_K) * 144; }
    static QWM_DEV void load_w(W & w, const uint8_t * row, int c) { load_w_chunk(w, row, c); }
    static QWM_DEV void load_a(A & x, const int8_t * qs, const float * d, const int32_t * bs, int K, int c) {
        load_act_chunk(x, qs, d, bs, c);
        (void)K;
    }
    static QWM_DEV size_t d_per_row(int K) { return (size_t)(K / QK_K); }
    static QWM_DEV float dot(const W & w, const A & x, int c) { return chunk_dot(w, x, c, 0.f); }
};

struct FmtQ80 {
    using W = W80;
    using A = A80;
    static constexpr int CHUNK = 32;
    static QWM_DEV size_t row_bytes(int K) { return (size_t)(K / QK8_0_) * 34; }
    static QWM_DEV void load_w(W & w, const uint8_t * row, int c) { load_w80(w, row, c); }
    static QWM_DEV void load_a(A & x, const int8_t * qs, const float * d, const int32_t * bs, int K, int c) {
        load_a80(x, qs, d, c);
        (void)bs; (void)K;
    }
    static QWM_DEV size_t d_per_row(int K) { return (size_t)(K / QK8_0_); }
    static QWM_DEV float dot(const W & w, const A & x, int c) { return dot80(w, x, c, 0.f); }
};

}  // namespace qwm
