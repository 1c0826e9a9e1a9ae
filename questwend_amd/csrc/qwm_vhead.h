// qwm_vhead.h -- the MTP verify head on gfx950 in one kernel: rms_norm +
// x86 Q8_0 activation quantization, the Q8_0 lm_head GEMV with a running
// argmax, and (in the last block to finish) the cross-block argmax and the
// greedy acceptance check.
//
// The Q8_0 block dots run on the matrix cores: v_mfma_i32_4x4x4_16b_i8 holds
// 16 independent 4x4x4 int8 products, which here are 16 Q8_0 blocks x 4 tokens
// x 4 vocabulary rows.  A wave owns a tile of 4 rows; lane l = 4*b + j loads
// row j's blocks b, b+16, b+32, b+48 (one "set" each) and the MFMA of set s
// gives it the exact int32 block sums of its row for all four tokens.  Only
// the per-block fp32 scaling, one per (row, block, token), is vector work.
//
// A 34-byte block is 2 bytes off dword alignment in every other position.
// Each lane loads the 9 aligned dwords around its block and the block's
// activations are shifted by the same 2 bytes once, up front (zeros facing
// the fp16 scale bytes), so the 9 MFMA steps over the raw window give exactly
// the 32-element block dot with no byte shuffling in the loop.
//
// Per tile, the 16 lanes of a row hold partial sums over their blocks for four
// tokens: two DPP rotate stages reduce-scatter the tokens (each lane keeps one
// token), two cross-row shuffles finish the sum.  Each lane then keeps a
// running argmax for its (row slot, token).
#pragma once

#include "qwm_device.h"

namespace qwm {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int VH_MAX_T = MAX_T;
constexpr int VH_WIN = 9;      // dwords in the aligned window around one block

struct VerifyArgs {
    const uint8_t * W; int H, V;
    const float * x; const float * norm_w; float eps;
    const int32_t * drafts; int32_t * result;
    float * pv; int32_t * pi; int32_t * counter;
};

// The set windows of one lane: row + lane_off + 544*s (16 blocks of 34 B per set).
template <int NS>
QWM_DEV void load_tile(uint32_t (&w)[NS][VH_WIN], const uint8_t * p0) {
    typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const uint32_t * p = reinterpret_cast<const uint32_t *>(p0 + 544 * s);
        const u32x4_a4 v0 = *reinterpret_cast<const u32x4_a4 *>(p);
        const u32x4_a4 v1 = *reinterpret_cast<const u32x4_a4 *>(p + 4);
        w[s][0] = v0.x; w[s][1] = v0.y; w[s][2] = v0.z; w[s][3] = v0.w;
        w[s][4] = v1.x; w[s][5] = v1.y; w[s][6] = v1.z; w[s][7] = v1.w;
        w[s][8] = p[8];
    }
}

// LDS bytes of the quantized activations for NT tokens of 512 NS values
// (s_q, s_d, s_sq: 16 NS Q8_0 blocks per token).
template <int NT, int NS = 4> struct VhSmem {
    static constexpr size_t nb = (size_t)16 * NS;
    static constexpr size_t q = (size_t)NT * nb * 32, d = (size_t)NT * nb * 4, sq = (size_t)NT * nb * 8;
    static constexpr size_t bytes = q + d + sq;
};

// The whole verify head for one workgroup `wg` of `n_wg` (grid-stride over
// vocabulary rows), with `smem` holding VhSmem<NT, NS>::bytes of LDS.  Returns
// true in the workgroup that finished last (it wrote the result).
// NS = H / 512 block sets per lane (H = 512 * NS), PF tiles in flight.
// ISSUE: when the first weight tiles are requested.  VH_EARLY: before the
// rms_norm and quantization prep; VH_LATE: after it; VH_BEFORE_WAIT: first of
// all, then the workgroup waits until `*ready` counts `ready_target`
// completions (the producers of x inside the same launch), so the tiles'
// latency hides under the wait.
enum { VH_LATE = 0, VH_EARLY = 1, VH_BEFORE_WAIT = 2 };
template <int NT, int NS, int PF, int ISSUE = VH_EARLY>
QWM_DEV bool verify_body(const VerifyArgs & a, int wg, int n_wg, uint8_t * smem, const int32_t * ready = nullptr,
                         int32_t ready_target = 0, int32_t * err = nullptr, uint32_t spin_limit = 0) {
    constexpr int NG = (NT + 3) / 4;                  // token groups (MFMA A rows)
    __shared__ float s_scale[NT];
    using Sm = VhSmem<NT, NS>;
    uint4 (*s_q)[16 * NS][2] = reinterpret_cast<uint4 (*)[16 * NS][2]>(smem);
    float (*s_d)[16 * NS] = reinterpret_cast<float (*)[16 * NS]>(smem + Sm::q);
    double * s_sq = reinterpret_cast<double *>(smem + Sm::q + Sm::d);
    __shared__ float s_bv[4][NT];
    __shared__ int32_t s_bi[4][NT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 3, b = lane >> 2;
    constexpr int H = 512 * NS, nblk = 16 * NS;
    const int V = a.V;
    const size_t row_bytes = (size_t)nblk * 34;
    const int odd = b & 1;                            // parity of every block this lane owns
    const int lane_off = 34 * b - 2 * odd;            // dword-aligned window start of block b

    const int64_t rb = (int64_t)wg * V / n_wg, re = (int64_t)(wg + 1) * V / n_wg;
    const int n_steps = (int)((re - rb + 15) / 16);   // 4 waves x 4 rows per step
    auto row_of = [&](int s) { return rb + (int64_t)s * 16 + wave * 4 + j; };
    auto lane_ptr = [&](int s) {
        int64_t r = row_of(s);
        r = r < re ? r : re - 1;                      // clamped: loads stay in bounds
        return a.W + r * row_bytes + lane_off;
    };

    uint32_t win[PF][NS][VH_WIN];
    if constexpr (ISSUE == VH_BEFORE_WAIT) {
#pragma unroll
        for (int p = 0; p < PF; ++p) load_tile<NS>(win[p], lane_ptr(min(p, n_steps - 1)));
        wait_count(ready, ready_target, err, spin_limit);
    }

    // ---- h = rms_norm(x) * norm_w (ggml-cpu/ops.cpp:4120-4160), then the x86
    // Q8_0 quantizer (ggml-cpu/arch/x86/quants.c:302-345) per (token, block)
    // item, into LDS.  Vector-memory waits complete in issue order, so every
    // activation load goes out before the weight prefetch: the prep then waits
    // on one round trip instead of queueing behind the weight stream.
    constexpr int NI = (NT * nblk + 255) / 256;       // items per thread
    float4 xv[NI][8], nv[NI][8];
#pragma unroll
    for (int k = 0; k < NI; ++k) {
        const int it = min(tid + 256 * k, NT * nblk - 1);
        const float4 * src = reinterpret_cast<const float4 *>(a.x + (size_t)it * QK8_0);   // token-major [T][H]
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[k][i] = src[i];
        if (a.norm_w) {
            const float4 * nw = reinterpret_cast<const float4 *>(a.norm_w + (it % nblk) * QK8_0);
#pragma unroll
            for (int i = 0; i < 8; ++i) nv[k][i] = nw[i];
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // weight loads for the first steps
    if constexpr (ISSUE == VH_EARLY) {
#pragma unroll
        for (int p = 0; p < PF; ++p) load_tile<NS>(win[p], lane_ptr(min(p, n_steps - 1)));
    }

#pragma unroll
    for (int k = 0; k < NI; ++k) {
        const int it = tid + 256 * k;
        double acc = 0.0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = xv[k][i];
            acc += (double)(v.x * v.x); acc += (double)(v.y * v.y);
            acc += (double)(v.z * v.z); acc += (double)(v.w * v.w);
        }
        if (it < NT * nblk) s_sq[it] = acc;
    }
    __syncthreads();
    if (tid < NT) {
        double sum = 0.0;
        for (int blk = 0; blk < nblk; ++blk) sum += s_sq[tid * nblk + blk];
        const float mean = (float)(sum / (double)H);
        s_scale[tid] = 1.0f / sqrtf(mean + a.eps);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NI; ++k) {
        const int it = tid + 256 * k;
        if (it >= NT * nblk) break;
        const int t = it / nblk, blk = it % nblk;
        const float sc = s_scale[t];
        float y[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = xv[k][i];
            y[4 * i + 0] = v.x * sc; y[4 * i + 1] = v.y * sc; y[4 * i + 2] = v.z * sc; y[4 * i + 3] = v.w * sc;
        }
        if (a.norm_w) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 g = nv[k][i];
                y[4 * i + 0] = y[4 * i + 0] * g.x; y[4 * i + 1] = y[4 * i + 1] * g.y;
                y[4 * i + 2] = y[4 * i + 2] * g.z; y[4 * i + 3] = y[4 * i + 3] * g.w;
            }
        }
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, __builtin_fabsf(y[i]));
        const float d = amax / 127.f;
        const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
        uint32_t pk[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t packed = 0;
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) packed |= (uint32_t)((int)__builtin_rintf(y[4 * i + k2] * id) & 0xff) << (8 * k2);
            pk[i] = packed;
        }
        s_q[t][blk][0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        s_q[t][blk][1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
        s_d[t][blk] = fp16_to_f32(f32_to_fp16(d));
    }
    __syncthreads();
    if constexpr (ISSUE == VH_LATE) {
#pragma unroll
        for (int p = 0; p < PF; ++p) load_tile<NS>(win[p], lane_ptr(min(p, n_steps - 1)));
    }

    // MFMA A operands: token 4g + j of block b + 16s, shifted to this lane's
    // window (even blocks: 2 zero bytes under the fp16 scale, qs from byte 2;
    // odd blocks: a zero dword under the previous block's tail and the scale).
    // Tokens past NT contribute zeros.  dx[g][s][i]: scale of token 4g + i.
    uint32_t act[NG][NS][VH_WIN];
    float dx[NG][NS][4];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int blk = b + 16 * s;
            const int t = 4 * g + j;
            uint32_t q[8];
            if (t < NT) {
                const uint4 q0 = s_q[t < NT ? t : 0][blk][0], q1 = s_q[t < NT ? t : 0][blk][1];
                q[0] = q0.x; q[1] = q0.y; q[2] = q0.z; q[3] = q0.w; q[4] = q1.x; q[5] = q1.y; q[6] = q1.z; q[7] = q1.w;
            } else {
#pragma unroll
                for (int c = 0; c < 8; ++c) q[c] = 0;
            }
            if (odd) {
                act[g][s][0] = 0;
#pragma unroll
                for (int c = 1; c < 9; ++c) act[g][s][c] = q[c - 1];
            } else {
                act[g][s][0] = q[0] << 16;
#pragma unroll
                for (int c = 1; c < 8; ++c) act[g][s][c] = __builtin_amdgcn_alignbit(q[c], q[c - 1], 16);
                act[g][s][8] = q[7] >> 16;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) dx[g][s][i] = (4 * g + i < NT) ? s_d[(4 * g + i < NT) ? 4 * g + i : 0][blk] : 0.f;
        }

    // running argmax per (row slot j, token of this lane); rows are visited in
    // increasing order, so ">=" keeps the last maximum (ggml-cpu/vec.h:1618-1626)
    const bool b2 = lane & 4, b3 = lane & 8;
    float best[NG];
    int32_t besti[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) { best[g] = -__builtin_inff(); besti[g] = -1; }

    auto consume = [&](const uint32_t (&w)[NS][VH_WIN], int step) {
        float f[NG][4];
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) f[g][i] = 0.f;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const float dw = fp16_to_f32((uint16_t)(w[s][0] >> (odd ? 16 : 0)));
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                v4i acc = {0, 0, 0, 0};
#pragma unroll
                for (int c = 0; c < VH_WIN; ++c)
                    acc = __builtin_amdgcn_mfma_i32_4x4x4i8((int)act[g][s][c], (int)w[s][c], acc, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (4 * g + i < NT) f[g][i] = __builtin_fmaf(dw * dx[g][s][i], (float)acc[i], f[g][i]);
            }
        }
        const int64_t r = row_of(step);
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            // reduce-scatter over lane bits 2 and 3 (rotations within 16-lane rows),
            // then sum over bits 4 and 5
            const float k0 = b2 ? f[g][2] : f[g][0], k1 = b2 ? f[g][3] : f[g][1];
            const float s0 = b2 ? f[g][0] : f[g][2], s1 = b2 ? f[g][1] : f[g][3];
            const float m0 = k0 + dpp_f<0x124>(s0);          // row_ror:4
            const float m1 = k1 + dpp_f<0x124>(s1);
            const float kk = b3 ? m1 : m0, ss = b3 ? m0 : m1;
            float tot = kk + dpp_f<0x128>(ss);               // row_ror:8
            tot += __shfl_xor(tot, 16, WAVE);
            tot += __shfl_xor(tot, 32, WAVE);
            const bool take = (r < re) & (tot >= best[g]);
            best[g] = take ? tot : best[g];
            besti[g] = take ? (int32_t)r : besti[g];
        }
    };

    int s = 0;
    for (; s + PF <= n_steps; s += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            consume(win[p], s + p);
            load_tile<NS>(win[p], lane_ptr(min(s + p + PF, n_steps - 1)));
        }
    }
#pragma unroll
    for (int p = 0; p < PF; ++p)
        if (s + p < n_steps) consume(win[p], s + p);

    // ---- wave argmax per token (lane bits 0, 1 = row slot; 4, 5 hold copies),
    // block argmax -> partials; the last block reduces them and accepts
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        float v = best[g];
        int idx = besti[g];
#pragma unroll
        for (int o = 1; o <= 32; o <<= 1) {
            if (o == 4 || o == 8) continue;
            const float ov = __shfl_xor(v, o, WAVE);
            const int oi = __shfl_xor(idx, o, WAVE);
            if (ov > v || (ov == v && oi > idx)) { v = ov; idx = oi; }
        }
        const int t = 4 * g + (b2 ? 2 : 0) + (b3 ? 1 : 0);
        if ((lane & 0x33) == 0 && t < NT) { s_bv[wave][t] = v; s_bi[wave][t] = idx; }
    }
    __syncthreads();
    if (tid < NT) {
        float v = s_bv[0][tid];
        int i = s_bi[0][tid];
        for (int w = 1; w < 4; ++w)
            if (s_bv[w][tid] > v || (s_bv[w][tid] == v && s_bi[w][tid] > i)) { v = s_bv[w][tid]; i = s_bi[w][tid]; }
        st_agent(a.pv + (size_t)wg * NT + tid, v);
        st_agent(a.pi + (size_t)wg * NT + tid, i);
    }
    if (!last_workgroup(a.counter, n_wg)) return false;
    __shared__ int32_t vA[NT];
    for (int t = wave; t < NT; t += 4) {
        float v = -__builtin_inff();
        int idx = -1;
        for (int g = lane; g < n_wg; g += 64) {
            const float ov = ld_agent(a.pv + (size_t)g * NT + t);
            const int oi = ld_agent(a.pi + (size_t)g * NT + t);
            if (ov > v || (ov == v && oi > idx)) { v = ov; idx = oi; }
        }
        wave_argmax_last(v, idx);
        if (lane == 0) vA[t] = idx < 0 ? 0 : idx;
    }
    __syncthreads();
    if (tid == 0) {
        int acc = 0;
        while (acc < NT - 1 && vA[acc] == a.drafts[acc]) ++acc;   // runtime.cpp:3648-3652
        for (int i = 0; i < NT; ++i) a.result[i] = vA[i];
        a.result[NT] = acc;
        a.result[NT + 1] = vA[acc];
    }
    return true;
}

}  // namespace qwm
