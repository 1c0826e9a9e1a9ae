// qwm_select.h -- the expert selection of Impl::route_experts
// (core/runtime.cpp:2693-2734) for one token in one wave, shared by the
// routing kernel and the fused step:
//   probs = soft_max(logits)            (gating_func 1, or 0: the default)
//         | sigmoid(logits)             (gating_func 2, unary-ops.cpp:31-33)
//   rank  = probs [+ exp_probs_b [+ rm]]   (the mask again after the bias)
//   sel   = top-k of rank (larger first; equal ranks: lower expert index)
//   w     = probs[sel]; if norm: w /= clamp(sum(w), 6.103515625e-5, inf)
//   if scale not in {0, 1}: w *= scale
// The logits arrive with rm already added (runtime.cpp:2700).
#pragma once

#include "qwm_device.h"

namespace qwm {

struct SelectCfg {
    int E, k, norm, sigm;       // sigm: gating_func == 2
    float scale;
    const float * bias;         // exp_probs_b [E] or null
};

// v[r]: the logit of expert 64 r + lane (any value past E).  Lane j < k
// returns the j-th selection in myid / myw.
template <int R>
QWM_DEV void select_token(const float (&v)[R], const SelectCfg & c, const float * rm_t, int lane, int & myid,
                          float & myw) {
    const int E = c.E, k = c.k;
    const int nr = (E + 63) / 64;
    const int nfull = E & ~15;
    float pr[R];
    if (!c.sigm) {
        // soft_max (ggml-cpu/ops.cpp:5813-5920, vec.cpp:531 AVX-512): v_expf
        // over 16-lane chunks, each chunk's 16-lane tree added to a double sum
        // in order, the scalar tail through libm expf, then x (1 / sum)
        float m = -__builtin_inff();
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (r < nr && 64 * r + lane < E) m = fmaxf(m, v[r]);
        m = wave_max(m);
        double sum = 0.0;
        float tailv = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            pr[r] = 0.f;
            if (r < nr) {
                const int i = 64 * r + lane;
                float ev = 0.f;
                if (i < nfull) ev = v_expf(v[r] - m);
                else if (i < E) ev = libm_expf(v[r] - m);
                const float cs = tree16_dpp(i < nfull ? ev : 0.f);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (64 * r + 16 * q < nfull) sum += (double)readlane_f(cs, 16 * q);
                if (r == (nfull >> 6)) tailv = ev;
                pr[r] = ev;
            }
        }
        for (int i = nfull; i < E; ++i) sum += (double)readlane_f(tailv, i & 63);
        const float sc = (float)(1.0 / sum);
#pragma unroll
        for (int r = 0; r < R; ++r) pr[r] = pr[r] * sc;
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) pr[r] = (r < nr && 64 * r + lane < E) ? libm_sigmoid(v[r]) : 0.f;
    }
    float rk[R];
    bool alive[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = 64 * r + lane;
        alive[r] = r < nr && i < E;
        rk[r] = pr[r];
        if (alive[r] && c.bias) {
            rk[r] = rk[r] + c.bias[i];
            if (rm_t) rk[r] = rk[r] + rm_t[i];
        }
    }
    // top-k: k rounds of the wave maximum over the experts not yet taken; a tie
    // goes to the lower index (the first r, then the first lane).  A round in
    // which only NaN ranks are left takes the lowest remaining index.  Lane j
    // keeps the j-th selection; the weight sum runs in selection order.
    myw = 0.f;
    myid = 0;
    double wsum = 0.0;
    for (int j = 0; j < k; ++j) {
        float mx = -__builtin_inff();
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (alive[r]) mx = fmaxf(mx, rk[r]);
        mx = wave_max(mx);
        int id = -1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const unsigned long long bal = __ballot(alive[r] && rk[r] == mx);
            if (id < 0 && bal) id = 64 * r + (int)__builtin_ctzll(bal);
        }
        if (id < 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const unsigned long long bal = __ballot(alive[r]);
                if (id < 0 && bal) id = 64 * r + (int)__builtin_ctzll(bal);
            }
        }
        id = __builtin_amdgcn_readfirstlane(id);
        float pv = 0.f;                                   // probs[id]
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float q = readlane_f(pr[r], id & 63);
            if ((id >> 6) == r) pv = q;
        }
        if (lane == j) { myw = pv; myid = id; }
        wsum += (double)pv;
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (64 * r + lane == id) alive[r] = false;
    }
    if (c.norm) {
        float ws = (float)wsum;
        ws = fmaxf(fminf(ws, __builtin_inff()), 6.103515625e-5f);
        myw = myw / ws;
    }
    if (c.scale != 0.0f && c.scale != 1.0f) myw = myw * c.scale;
}

}  // namespace qwm
