// qwm_exact.h -- Q4_K x Q8_K row dots in ggml-CPU's exact float order.
//
// ggml's x86 ggml_vec_dot_q4_K_q8_K (ggml-cpu/arch/x86/quants.c:2102-2185)
// keeps eight fp32 lanes: lane m accumulates, block after block,
//   acc[m] = fma(y.d * fp16(x.d), (float) sumi[m], acc[m]),
//   sumi[m] = sum_j sc_j * (dot of elements 4m .. 4m+3 of sub-block j),
// and four lanes of mins, acc_m[l] = fma(-y.d * fp16(x.dmin), (float)
// (mn_2l * q8s_2l + mn_2l+1 * q8s_2l+1), acc_m[l]) with q8s_j = bsums_2j +
// bsums_2j+1; the row's value is hsum8(acc) + hsum4(acc_m) (pairs (m, m+4),
// then (0, 2) and (1, 3), then the two halves).  The integer sums are exact
// in any order; only the float steps have an order, and here eight GPU lanes
// play the eight CPU lanes: lane m of a row's 8-lane group walks the row's
// blocks in order with the same fused multiply-adds, so the result is the
// CPU's bit for bit.  Then the SwiGLU activations, their Q8_K levels, and the
// down projection's integer sums are the CPU's too: no quantization-boundary
// flips between the two.
//
// Weights: lane m loads the 16-byte block header (d, dmin, 12 scale bytes,
// shared by the group) and the 4 dwords of qs it needs (bytes 32p + 4m).
// Activations (Q8_K) sit in LDS in a per-lane order: per block XS dwords,
// lane m's 8 qs dwords contiguous (sub-block 2p+h at slot 2p+h), then the
// block scale and the eight 32-element sums q8s.
#pragma once

#include "qwm_q4k.h"

namespace qwm {

constexpr int XS = 76;       // LDS dwords per Q8_K block in the exact layout (64 qs + d + 8 q8s + pad)

// One wave quantizes 256 floats to Q8_K (quantize_block_q8K's arithmetic)
// into the exact layout at `dst` (XS dwords).  Lane l owns elements 4l..4l+3,
// i.e. qs dword l = 16p + 8h + m.
// quantize_q8K_x_reg: the same from the lane's four elements already in
// registers (so a wave can request several blocks before quantizing any).
template <bool AGENT = false>
QWM_DEV void quantize_q8K_x_reg(const float4 v4, uint32_t * __restrict__ dst, int lane);

template <bool SRC_AGENT = false, bool AGENT = false>
QWM_DEV void quantize_block_q8K_x(const float * __restrict__ src, uint32_t * __restrict__ dst, int lane) {
    float4 v4;
    if constexpr (SRC_AGENT) {
        const uint64_t * s64 = reinterpret_cast<const uint64_t *>(src) + 2 * lane;
        const uint64_t lo = ld_agent(s64), hi = ld_agent(s64 + 1);
        v4 = make_float4(__uint_as_float((uint32_t)lo), __uint_as_float((uint32_t)(lo >> 32)),
                         __uint_as_float((uint32_t)hi), __uint_as_float((uint32_t)(hi >> 32)));
    } else {
        v4 = reinterpret_cast<const float4 *>(src)[lane];
    }
    quantize_q8K_x_reg<AGENT>(v4, dst, lane);
}

template <bool AGENT>
QWM_DEV void quantize_q8K_x_reg(const float4 v4, uint32_t * __restrict__ dst, int lane) {
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
    const int m = lane & 7, h = (lane >> 3) & 1, p = lane >> 4;
    // sums over 32 elements (8 lanes): quads by DPP, then quad + quad + 4
    int sm = q[0] + q[1] + q[2] + q[3];
    sm += dpp_i<0xB1>(sm);
    sm += dpp_i<0x4E>(sm);
    sm += dpp_i<0x124>(sm);                   // lane i receives lane i - 4 (same 16-lane row)
    const uint32_t q8s = (uint32_t)(int32_t)(int16_t)sm;
    if constexpr (AGENT) {
        st_agent(dst + 8 * m + 2 * p + h, packed);
        if ((lane & 7) == 4) st_agent(dst + 65 + (lane >> 3), q8s);
        if (lane == 0) st_agent(dst + 64, __float_as_uint(d));
    } else {
        dst[8 * m + 2 * p + h] = packed;
        if ((lane & 7) == 4) dst[65 + (lane >> 3)] = q8s;
        if (lane == 0) dst[64] = __float_as_uint(d);
    }
}

// One Q4_K block as lane m of its row's 8-lane group holds it.
struct XBlk {
    uint4 h;         // d, dmin (fp16 x 2), scales[0..11]
    uint32_t q[4];   // qs bytes 32p + 4m .. +3, p = 0..3
};

QWM_DEV void load_xblk(XBlk & B, const uint8_t * blk, int m) {
    B.h = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
    for (int p = 0; p < 4; ++p) B.q[p] = *reinterpret_cast<const uint32_t *>(blk + 16 + 32 * p + 4 * m);
}

// The integer products below run on the 24-bit multiplier (full rate; a
// 32-bit v_mul_lo is quarter rate): every operand fits 24 signed bits, e.g.
// |dot4| <= 4 * 63 * 128 (Q6_K), scales and mins <= 63 (Q4_K/Q5_K) or 128
// (Q6_K), |q8s| <= 32 * 128, so the products and sums are the exact integers.

// The block loop of a Q4_K row dot: the NB blocks in W against n <= MAXP
// activation rows at xt[i] (NB consecutive blocks of XS dwords each in LDS),
// added to each lane's 8-lane accumulators acc (scales) and accm (mins) in
// block order.  A row of more blocks than a lane's registers hold runs as
// several calls on consecutive chunks, the accumulators carried between them:
// the same sums in the same order.  FIXN as in q4k_dot8_off.
template <int NB, int MAXP, int FIXN = 0>
QWM_DEV void q4k_acc8(float (&acc)[MAXP], float (&accm)[MAXP], const XBlk (&W)[NB], const uint32_t * const (&xt)[MAXP],
                      int n, int m) {
    const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u, m4 = 0x0f0f0f0fu;
    const int l = m & 3;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const XBlk & B = W[b];
        // scales and mins as ggml unpacks them (quants.c:2133-2138)
        const uint32_t u0 = B.h.y, u1 = B.h.z, u2 = B.h.w;
        uint32_t mn_hi = ((u2 >> 4) & k2) | (((u1 >> 6) & k3) << 4);
        uint32_t mn_lo = u1 & k1;
        uint32_t sc_hi = (u2 & k2) | (((u0 >> 6) & k3) << 4);
        uint32_t sc_lo = u0 & k1;
        // opaque to the optimizer, so that each scale below is a byte select
        // of these words inside the multiply (no separate bit-field extract)
        asm("" : "+v"(sc_lo), "+v"(sc_hi), "+v"(mn_lo), "+v"(mn_hi));
        int sc[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) { sc[j] = (sc_lo >> (8 * j)) & 0xff; sc[4 + j] = (sc_hi >> (8 * j)) & 0xff; }
        const uint32_t mw = l < 2 ? mn_lo : mn_hi;
        const int sh = 16 * (l & 1);
        const int mnA = (mw >> sh) & 0xff, mnB = (mw >> (sh + 8)) & 0xff;
        const float dw = fp16_to_f32((uint16_t)(B.h.x & 0xffff));
        const float dmw = fp16_to_f32((uint16_t)(B.h.x >> 16));
        uint32_t wl[4], wh[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) { wl[p] = B.q[p] & m4; wh[p] = (B.q[p] >> 4) & m4; }
#pragma unroll
        for (int i = 0; i < MAXP; ++i) {
            if (i < n) {
                const uint32_t * xb = xt[i] + b * XS;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(xb + 8 * m);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(xb + 8 * m + 4);
                const float yd = __uint_as_float(xb[64]);
                const int qa = (int)xb[65 + 2 * l], qb = (int)xb[66 + 2 * l];
                int s = __mul24(sc[0], dot4(wl[0], x0.x, 0));
                s += __mul24(sc[1], dot4(wh[0], x0.y, 0));
                s += __mul24(sc[2], dot4(wl[1], x0.z, 0));
                s += __mul24(sc[3], dot4(wh[1], x0.w, 0));
                s += __mul24(sc[4], dot4(wl[2], x1.x, 0));
                s += __mul24(sc[5], dot4(wh[2], x1.y, 0));
                s += __mul24(sc[6], dot4(wl[3], x1.z, 0));
                s += __mul24(sc[7], dot4(wh[3], x1.w, 0));
                acc[i] = __builtin_fmaf(yd * dw, (float)s, acc[i]);
                const int prod = __mul24(mnA, qa) + __mul24(mnB, qb);
                accm[i] = __builtin_fmaf(-yd * dmw, (float)prod, accm[i]);
            }
        }
    }
}

// hsum_float_8(acc) + hsum_float_4(acc_m) (quants.c:43-49, 2181-2184): the
// row's dot in lane m == 0 of each 8-lane group.
template <int MAXP>
QWM_DEV void q4k_fin8(float (&out)[MAXP], const float (&acc)[MAXP], const float (&accm)[MAXP], int n) {
#pragma unroll
    for (int i = 0; i < MAXP; ++i) {
        if (i < n) {
            const float t = acc[i] + dpp_f<0x12C>(acc[i]);        // lanes 0-3: a[m] + a[m + 4]
            const float u = t + dpp_f<0x12E>(t);                   // lanes 0-1: t[m] + t[m + 2]
            const float h8 = u + dpp_f<0x12F>(u);                  // lane 0: u[0] + u[1]
            const float v = accm[i] + dpp_f<0x12E>(accm[i]);       // lanes 0-1: am[l] + am[l + 2]
            const float h4 = v + dpp_f<0x12F>(v);                  // lane 0
            out[i] = h8 + h4;
        } else {
            out[i] = 0.f;
        }
    }
}

// Row dots of one weight row (NB blocks in W) with n <= MAXP activation rows
// at sx + off[i] in LDS (NB consecutive blocks of XS dwords each).  out[i] is
// valid in lane m == 0 of the group.
// FIXN > 0: exactly FIXN tokens (a compile-time count, so that no branch
// splits the unrolled block loop and the scheduler can request later blocks'
// activations early); 0: n at run time.
template <int NB, int MAXP, int FIXN = 0>
QWM_DEV void q4k_dot8_off(float (&out)[MAXP], const XBlk (&W)[NB], const uint32_t * sx, const int (&off)[MAXP], int n_,
                          int m) {
    // the token count and offsets are uniform: scalar loop control, and each
    // token's activation rows at one scalar base (block offsets immediate)
    const int n = FIXN > 0 ? FIXN : __builtin_amdgcn_readfirstlane(n_);
    const uint32_t * xt[MAXP];
#pragma unroll
    for (int i = 0; i < MAXP; ++i) xt[i] = sx + __builtin_amdgcn_readfirstlane(off[i]);
    float acc[MAXP], accm[MAXP];
#pragma unroll
    for (int i = 0; i < MAXP; ++i) { acc[i] = 0.f; accm[i] = 0.f; }
    q4k_acc8<NB, MAXP, FIXN>(acc, accm, W, xt, n, m);
    q4k_fin8<MAXP>(out, acc, accm, n);
}

// One chunk step of q4k_dot8_chunked: the loads of chunk C + 1 into the other
// buffer, then chunk C's arithmetic, then the next step (a compile-time
// recursion, so every buffer index is a constant and the buffers stay in
// registers).
template <int NB, int CB, int NR, int MAXP, int C>
QWM_DEV void q4k_chunk_step(float (&acc)[NR][MAXP], float (&accm)[NR][MAXP], XBlk (&W)[2][NR][CB],
                            const uint8_t * const (&row)[NR], const uint32_t * sx, int n, int m) {
    constexpr int NC = NB / CB;
    if constexpr (C < NC) {
        if constexpr (C + 1 < NC) {
#pragma unroll
            for (int q = 0; q < NR; ++q)
#pragma unroll
                for (int b = 0; b < CB; ++b) load_xblk(W[(C + 1) & 1][q][b], row[q] + ((C + 1) * CB + b) * 144, m);
        }
        const uint32_t * xt[MAXP];
#pragma unroll
        for (int i = 0; i < MAXP; ++i) xt[i] = sx + i * NB * XS + C * CB * XS;
#pragma unroll
        for (int q = 0; q < NR; ++q) q4k_acc8<CB, MAXP>(acc[q], accm[q], W[C & 1][q], xt, n, m);
        q4k_chunk_step<NB, CB, NR, MAXP, C + 1>(acc, accm, W, row, sx, n, m);
    }
}

// NR rows of NB > 8 blocks (hidden sizes above 2048), each against the same
// n <= MAXP activation rows packed at sx + i * NB * XS: the blocks are
// requested CB at a time into two register buffers, the next chunk's loads
// issued before the current chunk's arithmetic, and each chunk runs through
// q4k_acc8 with the accumulators carried over.  CB divides NB.
template <int NB, int CB, int NR, int MAXP>
QWM_DEV void q4k_dot8_chunked(float (&out)[NR][MAXP], const uint8_t * const (&row)[NR], const uint32_t * sx, int n_,
                              int m) {
    static_assert(NB % CB == 0, "the chunk must divide the row");
    const int n = __builtin_amdgcn_readfirstlane(n_);
    float acc[NR][MAXP], accm[NR][MAXP];
#pragma unroll
    for (int q = 0; q < NR; ++q)
#pragma unroll
        for (int i = 0; i < MAXP; ++i) { acc[q][i] = 0.f; accm[q][i] = 0.f; }
    XBlk W[2][NR][CB];
#pragma unroll
    for (int q = 0; q < NR; ++q)
#pragma unroll
        for (int b = 0; b < CB; ++b) load_xblk(W[0][q][b], row[q] + b * 144, m);
    q4k_chunk_step<NB, CB, NR, MAXP, 0>(acc, accm, W, row, sx, n, m);
#pragma unroll
    for (int q = 0; q < NR; ++q) q4k_fin8<MAXP>(out[q], acc[q], accm[q], n);
}

// q4k_dot8_off with the common token counts (1 and 2, most expert units of a
// verify batch) as branch-free instances.
template <int NB, int MAXP>
QWM_DEV void q4k_dot8_auto(float (&out)[MAXP], const XBlk (&W)[NB], const uint32_t * sx, const int (&off)[MAXP], int n_,
                           int m) {
    const int n = __builtin_amdgcn_readfirstlane(n_);
    if (n == 1) q4k_dot8_off<NB, MAXP, 1>(out, W, sx, off, 1, m);
    else if (MAXP >= 2 && n == 2) q4k_dot8_off<NB, MAXP, (MAXP >= 2 ? 2 : 1)>(out, W, sx, off, 2, m);
    else q4k_dot8_off<NB, MAXP>(out, W, sx, off, n, m);
}

// The same with the activation rows packed at sx + i * NB * XS.
template <int NB, int MAXP>
QWM_DEV void q4k_dot8(float (&out)[MAXP], const XBlk (&W)[NB], const uint32_t * sx, int n, int m) {
    int off[MAXP];
#pragma unroll
    for (int i = 0; i < MAXP; ++i) off[i] = i * NB * XS;
    q4k_dot8_auto<NB, MAXP>(out, W, sx, off, n, m);
}

}  // namespace qwm

namespace qwm {

// Q8_0 x Q8_0 row dots in ggml-CPU's exact float order: the x86
// ggml_vec_dot_q8_0_q8_0 (ggml-cpu/arch/x86/quants.c:1389-1406) keeps eight
// fp32 lanes, lane m adding fma(fp16(x.d) * fp16(y.d), (float)(dot of
// elements 4m .. 4m+3 of the block), acc[m]) block after block, then
// hsum8.  Lane m of a row's 8-lane group plays CPU lane m.
//
// A pair of 34-byte blocks is 17 dwords: lane m takes dwords m, m+1 (the even
// block's qs bytes 4m..4m+3 sit 2 bytes into dword m), 9+m (the odd block's),
// and the scale dwords 0 (low half) and 8 (high half).  Activations (Q8_0) in
// LDS: xq [MAXP][kq dwords], xd [MAXP][kd] (natural layout: lane m reads dword
// 8b + m of block b).
template <int NPAIR, int MAXP>
QWM_DEV void q80_dot8(float (&out)[MAXP], const uint8_t * row, const uint32_t * xq, const float * xd, int kq, int kd,
                      int n, int m) {
    float acc[MAXP];
#pragma unroll
    for (int i = 0; i < MAXP; ++i) acc[i] = 0.f;
    const uint32_t * rw = reinterpret_cast<const uint32_t *>(row);
    constexpr int CH = NPAIR % 8 == 0 ? 8 : NPAIR % 4 == 0 ? 4 : NPAIR;   // pairs per chunk, dividing NPAIR
    static_assert(NPAIR % CH == 0, "chunk must divide the row");
#pragma unroll
    for (int c0 = 0; c0 < NPAIR; c0 += CH) {
        uint32_t w0[CH], w1[CH], w2[CH], s0[CH], s1[CH];
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const uint32_t * pr = rw + 17 * (c0 + k);
            w0[k] = pr[m]; w1[k] = pr[m + 1]; w2[k] = pr[9 + m]; s0[k] = pr[0]; s1[k] = pr[8];
        }
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int b = 2 * (c0 + k);
            const uint32_t we = __builtin_amdgcn_alignbit(w1[k], w0[k], 16);
            const float de = fp16_to_f32((uint16_t)(s0[k] & 0xffff));
            const float dd = fp16_to_f32((uint16_t)(s1[k] >> 16));
#pragma unroll
            for (int i = 0; i < MAXP; ++i) {
                if (i < n) {
                    const uint32_t xe = xq[i * kq + 8 * b + m], xo = xq[i * kq + 8 * b + 8 + m];
                    const float dxe = xd[i * kd + b], dxo = xd[i * kd + b + 1];
                    acc[i] = __builtin_fmaf(de * dxe, (float)dot4(we, xe, 0), acc[i]);
                    acc[i] = __builtin_fmaf(dd * dxo, (float)dot4(w2[k], xo, 0), acc[i]);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < MAXP; ++i) {
        if (i < n) {
            const float t = acc[i] + dpp_f<0x12C>(acc[i]);
            const float u = t + dpp_f<0x12E>(t);
            out[i] = u + dpp_f<0x12F>(u);
        } else {
            out[i] = 0.f;
        }
    }
}

// Q6_K x Q8_K row dots in ggml-CPU's exact float order: the x86
// ggml_vec_dot_q6_K_q8_K (ggml-cpu/arch/x86/quants.c:2490-2566) keeps eight
// int32 lanes per block, lane m gathering over the eight 32-value chunks c
// scale[2c + (m >= 4)] times the dot of chunk values 4m..4m+3 (6-bit values
// 0..63), minus 32 * (bsums[2m] * scale[2m] + bsums[2m+1] * scale[2m+1]),
// then acc[m] = fma(y.d * fp16(x.d), (float)lane, acc[m]) block after block,
// and hsum8.  Lane m of a row's 8-lane group plays CPU lane m.
//
// Q6_K blocks are 210 bytes (ql [128], qh [64], int8 scales [16], fp16 d), so
// a block starts 2 bytes off dword alignment when its byte offset does: then
// each needed dword is joined from the two aligned dwords around it
// (v_alignbit) and d is a 16-bit load; no access leaves the block's bytes
// and the 2 before it.  Lane m needs ql dwords 64j + 32h + 4m (j, h in 0..1:
// chunk 4j + k takes the low (k < 2) or high nibbles of half h = k & 1) and
// qh dwords 128 + 32j + 4m (bits 2k, 2k+1 are the values' top bits).  The
// chunk bsums come from the activations in LDS: chunk m's values 0..15 are
// dwords 8m' + m of lanes m' = 0..3, values 16..31 those of m' = 4..7.
template <int NB, int MAXP>
QWM_DEV void q6k_dot8(float (&out)[MAXP], const uint8_t * row, const uint32_t * sx, int n, int m) {
    float acc[MAXP];
#pragma unroll
    for (int i = 0; i < MAXP; ++i) acc[i] = 0.f;
    const int hm = m >= 4 ? 8 : 0;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const uint8_t * bp = row + 210 * b;
        const int s = (int)((uintptr_t)bp & 2);
        const uint32_t * A = reinterpret_cast<const uint32_t *>(bp - s);
        auto get = [&](int r) -> uint32_t {        // the 4 bytes at bp + r, r % 4 == 0
            const uint32_t lo = A[r >> 2];
            if (!s) return lo;
            return __builtin_amdgcn_alignbit(A[(r >> 2) + 1], lo, 16);
        };
        uint32_t ql[2][2], qh[2], sc[4];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            ql[j][0] = get(64 * j + 4 * m);
            ql[j][1] = get(64 * j + 32 + 4 * m);
            qh[j] = get(128 + 32 * j + 4 * m);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) sc[q] = get(192 + 4 * q);
        const float dw = fp16_to_f32(*reinterpret_cast<const uint16_t *>(bp + 208));
        int scc[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) scc[c] = (int)(int8_t)(uint8_t)(sc[c >> 1] >> (16 * (c & 1) + hm));
        const int mq = m >> 1;
        const uint32_t wm = mq == 0 ? sc[0] : mq == 1 ? sc[1] : mq == 2 ? sc[2] : sc[3];
        const int sA = (int)(int8_t)(uint8_t)(wm >> (16 * (m & 1))), sB = (int)(int8_t)(uint8_t)(wm >> (16 * (m & 1) + 8));
        uint32_t q6[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int j = c >> 2, k = c & 3;
            const uint32_t w = ql[j][k & 1];
            q6[c] = ((k < 2 ? w : w >> 4) & 0x0f0f0f0fu) | (((qh[j] >> (2 * k)) & 0x03030303u) << 4);
        }
#pragma unroll
        for (int i = 0; i < MAXP; ++i) {
            if (i < n) {
                const uint32_t * xb = sx + (i * NB + b) * XS;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(xb + 8 * m);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(xb + 8 * m + 4);
                const float yd = __uint_as_float(xb[64]);
                int isum = 0;
                isum += __mul24(scc[0], dot4(q6[0], x0.x, 0));
                isum += __mul24(scc[1], dot4(q6[1], x0.y, 0));
                isum += __mul24(scc[2], dot4(q6[2], x0.z, 0));
                isum += __mul24(scc[3], dot4(q6[3], x0.w, 0));
                isum += __mul24(scc[4], dot4(q6[4], x1.x, 0));
                isum += __mul24(scc[5], dot4(q6[5], x1.y, 0));
                isum += __mul24(scc[6], dot4(q6[6], x1.z, 0));
                isum += __mul24(scc[7], dot4(q6[7], x1.w, 0));
                int bA = 0, bB = 0;
#pragma unroll
                for (int mm = 0; mm < 4; ++mm) {
                    bA = dot4(xb[8 * mm + m], 0x01010101u, bA);
                    bB = dot4(xb[8 * (mm + 4) + m], 0x01010101u, bB);
                }
                isum -= 32 * (__mul24(bA, sA) + __mul24(bB, sB));
                acc[i] = __builtin_fmaf(yd * dw, (float)isum, acc[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < MAXP; ++i) {
        if (i < n) {
            const float t = acc[i] + dpp_f<0x12C>(acc[i]);
            const float u = t + dpp_f<0x12E>(t);
            out[i] = u + dpp_f<0x12F>(u);
        } else {
            out[i] = 0.f;
        }
    }
}

// Q5_K x Q8_K row dots in ggml-CPU's exact float order: the x86
// ggml_vec_dot_q5_K_q8_K (ggml-cpu/arch/x86/quants.c:1958-2046) keeps eight
// int32 lanes per block, lane m gathering scale[s] times the dot of values
// 4m..4m+3 of each 32-value sub-block s (5-bit values: the Q4_K nibble plus
// bit s of qh byte 4m..4m+3), then acc[m] = fma(y.d * fp16(x.d), (float)lane,
// acc[m]); the mins go to one float per row, summs = fma(-y.d * fp16(x.dmin),
// (float)sum_j(min[j] * (bsums[2j] + bsums[2j+1])), summs) (gcc contracts
// that statement), and the result is hsum8(acc) + summs.  Lane m of a row's
// 8-lane group plays CPU lane m; every lane keeps summs.  176-byte blocks
// keep dword alignment.
template <int NB, int MAXP>
QWM_DEV void q5k_dot8(float (&out)[MAXP], const uint8_t * row, const uint32_t * sx, int n, int m) {
    float acc[MAXP], summs[MAXP];
#pragma unroll
    for (int i = 0; i < MAXP; ++i) { acc[i] = 0.f; summs[i] = 0.f; }
    const uint32_t k1 = 0x3f3f3f3fu, k2 = 0x0f0f0f0fu, k3 = 0x03030303u;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const uint8_t * bp = row + 176 * b;
        const uint4 h = *reinterpret_cast<const uint4 *>(bp);
        const uint32_t qh = *reinterpret_cast<const uint32_t *>(bp + 16 + 4 * m);
        uint32_t q[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) q[p] = *reinterpret_cast<const uint32_t *>(bp + 48 + 32 * p + 4 * m);
        const uint32_t u0 = h.y, u1 = h.z, u2 = h.w;
        const uint32_t sc_lo = u0 & k1, sc_hi = (u2 & k2) | (((u0 >> 6) & k3) << 4);
        const uint32_t mn_lo = u1 & k1, mn_hi = ((u2 >> 4) & k2) | (((u1 >> 6) & k3) << 4);
        int sc[8], mn[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            sc[j] = (sc_lo >> (8 * j)) & 0xff; sc[4 + j] = (sc_hi >> (8 * j)) & 0xff;
            mn[j] = (mn_lo >> (8 * j)) & 0xff; mn[4 + j] = (mn_hi >> (8 * j)) & 0xff;
        }
        const float dw = fp16_to_f32((uint16_t)(h.x & 0xffff));
        const float dmw = fp16_to_f32((uint16_t)(h.x >> 16));
        uint32_t wl[4], wh[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            wl[p] = (q[p] & 0x0f0f0f0fu) | (((qh >> (2 * p)) & 0x01010101u) << 4);
            wh[p] = ((q[p] >> 4) & 0x0f0f0f0fu) | (((qh >> (2 * p + 1)) & 0x01010101u) << 4);
        }
#pragma unroll
        for (int i = 0; i < MAXP; ++i) {
            if (i < n) {
                const uint32_t * xb = sx + (i * NB + b) * XS;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(xb + 8 * m);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(xb + 8 * m + 4);
                const float yd = __uint_as_float(xb[64]);
                int s = 0;
                s += __mul24(sc[0], dot4(wl[0], x0.x, 0));
                s += __mul24(sc[1], dot4(wh[0], x0.y, 0));
                s += __mul24(sc[2], dot4(wl[1], x0.z, 0));
                s += __mul24(sc[3], dot4(wh[1], x0.w, 0));
                s += __mul24(sc[4], dot4(wl[2], x1.x, 0));
                s += __mul24(sc[5], dot4(wh[2], x1.y, 0));
                s += __mul24(sc[6], dot4(wl[3], x1.z, 0));
                s += __mul24(sc[7], dot4(wh[3], x1.w, 0));
                acc[i] = __builtin_fmaf(yd * dw, (float)s, acc[i]);
                int ms = 0;
#pragma unroll
                for (int j = 0; j < 8; ++j) ms += __mul24(mn[j], (int)xb[65 + j]);
                summs[i] = __builtin_fmaf(-yd * dmw, (float)ms, summs[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < MAXP; ++i) {
        if (i < n) {
            const float t = acc[i] + dpp_f<0x12C>(acc[i]);
            const float u = t + dpp_f<0x12E>(t);
            out[i] = (u + dpp_f<0x12F>(u)) + summs[i];
        } else {
            out[i] = 0.f;
        }
    }
}

}  // namespace qwm
