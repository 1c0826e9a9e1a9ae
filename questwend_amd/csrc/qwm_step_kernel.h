// qwm_step_kernel.h -- the fused verify step's device code (k_step and its
// phases) and its launch templates, shared by qwm_step.hip (T = 1..5, the
// host side), qwm_step_hi.hip (T = 6, 7) and qwm_step_t8.hip (T = 8), so the
// kernel's instantiations compile in parallel.
#pragma once

#include <hip/hip_runtime.h>

#include "qwm_internal.h"
#include "qwm_q4k.h"
#include "qwm_vhead.h"
#include "qwm_exact.h"
#include "qwm_select.h"

namespace qwm {

constexpr int SH = 2048;                 // hidden size of the fused step
constexpr int SNB = SH / QK_K;           // Q8_K blocks per token
constexpr uint32_t SPIN_LIMIT = 1u << 21;   // default bound of every wait (qwm_set_spin_limit changes it)
constexpr int MAX_NDOWN_S = 2048;        // longest down-projection input (FFN width)
constexpr int STEP_MAX_E = 512;          // experts per layer in the fused step
constexpr size_t STEP_SELECT_LDS = (size_t)3 * STEP_MAX_E * 4;   // the selection's union tables
constexpr int XSP = 96;                  // workspace dwords per exact-layout Q8_K block of x (3 whole lines)
constexpr size_t cmax(size_t x, size_t y) { return x > y ? x : y; }

struct StepArgs {
    const float * W_r; const float * x; const float * rm; const float * sgi;   // router [E][H], x [T][H]
    int E, k, norm, sigm; float scale;
    const float * bias;                                                         // exp_probs_b [E] or null
    int N, N_sh, shared;
    const uint8_t * gate; const uint8_t * up; const uint8_t * down;
    size_t gate_slab, up_slab, down_slab;
    int n_slots[3];                                                             // slots per pool (gate, up, down)
    const uint8_t * sh_gate; const uint8_t * sh_up; const uint8_t * sh_down;
    const int32_t * slot_tables; int64_t table_stride; int layer;
    const float * resid; float * out;                                           // [T][H]
    int32_t * ids_out; int64_t ids_ld; float * w_out; int64_t w_ld;
    float * lg;                                                                 // [E + 1][32]: logits of row e (row E: shared gate)
    float * act; float * act_sh; float * ex; float * ex_sh;
    int32_t * rows_done;                                                        // P0 workgroups finished
    uint32_t * xq_x;                                                            // Q8_K of x, exact layout, XSP dwords per block
    int32_t * tile_counters; int32_t * err;
    int d6;                                                                     // down slabs are Q6_K
    int32_t * gu_done;                                                          // per unit, one 32-word line each
    int32_t * tiles_done;                                                       // combined down tiles
    uint32_t spin;                                                              // bound of every wait, in sleeps
    VerifyArgs v;                                                               // v.x = out
};

// Per-workgroup copy of the expert schedule (phase P1).
struct StepShared {
    int32_t ids[MAX_PAIRS];
    float w[MAX_PAIRS];
    float shg[MAX_T];
    Unit units[MAX_PAIRS + 1];
    int32_t uslot[MAX_PAIRS + 1][3];
    int32_t nu;
    int32_t slot_of[3 * STEP_MAX_E];   // this layer's slot tables, [role][expert]
};

// ---------------------------------------------------------------- P0 ----
// Router rows e = g, g + G, ... (row E: the shared-expert gate row), and the
// Q8_K of x: NT * SNB / 4 quantizer workgroups, one 256-block per wave, into
// the workspace (the workgroups after the router rows when the grid has them,
// else the first router workgroups).  Every workgroup with a share counts
// once in rows_done when its writes are out; step_p0_parts() is the total.
template <int NT>
QWM_DEV int step_p0_first_quantizer(int rows, int G) {
    return rows + NT * SNB / 4 <= G ? rows : 0;
}
template <int NT>
QWM_DEV int step_p0_parts(int rows, int G) {
    const int q0 = step_p0_first_quantizer<NT>(rows, G);
    return (rows < G ? rows : G) + (q0 ? NT * SNB / 4 : 0);
}
template <int NT>
QWM_DEV void step_router(const StepArgs & a, int g, int G) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E;
    const int rows = E + (a.sgi ? 1 : 0);
    const int q0 = step_p0_first_quantizer<NT>(rows, G);
    const bool quantizer = g >= q0 && g < q0 + NT * SNB / 4;
    if (quantizer) {
        const int jb = (g - q0) * 4 + wave;                   // < NT * SNB
        quantize_block_q8K_x<false, true>(a.x + (size_t)(jb / SNB) * SH + (jb % SNB) * QK_K, a.xq_x + (size_t)jb * XSP, lane);
    }
    if (g >= rows) {                             // uniform per workgroup
        if (quantizer) signal_count(a.rows_done);
        return;
    }
    // ggml_vec_dot_f32's AVX-512 order (vec.cpp:11-135), which ggml-CPU runs
    // per (row, token) at every token count (ggml-cpu.c:1165-1244; llamafile
    // is not built), one token per wave pass
    for (int e = g; e < rows; e += G) {
        const bool sh_row = e == E;
        const float * w = sh_row ? a.sgi : a.W_r + (size_t)e * SH;
        float wv[SH / 64];
#pragma unroll
        for (int s = 0; s < SH / 64; ++s) wv[s] = w[64 * s + lane];
        for (int t = wave; t < NT; t += 4) {
            const float * xr = a.x + (size_t)t * SH;
            float xv[SH / 64];
#pragma unroll
            for (int s = 0; s < SH / 64; ++s) xv[s] = xr[64 * s + lane];
            float acc = 0.f;
#pragma unroll
            for (int s = 0; s < SH / 64; ++s) acc = __builtin_fmaf(wv[s], xv[s], acc);
            acc += lane_xor32_f(acc);
            acc += lane_xor16_f(acc);
            acc = tree16_dpp(acc);
            if (lane == 0) st_agent(a.lg + (size_t)e * 32 + t, (a.rm && !sh_row) ? acc + a.rm[(size_t)t * E + e] : acc);
        }
    }
    signal_count(a.rows_done);
}

// ---------------------------------------------------------------- P1 ----
// The selection of route_experts (runtime.cpp:2693-2734) for every token, in
// every workgroup, one wave per token (select_token, qwm_select.h: soft_max
// or sigmoid, the optional ranking bias, top-k, weights); then the expert
// union in first-occurrence order and each unit's slots.
// R: logits per lane (E <= 64 * R).  LG_DENSE: the logits lie at lg[e * NT +
// t] (several writers per line, so they are read with agent-scope loads)
// instead of one 128-byte line per row (lg[e * 32 + t]).
template <int NT, int R, bool LG_DENSE = false>
QWM_DEV void step_select(const StepArgs & a, int g, StepShared & S, uint8_t * smem) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E, k = a.k;
    const int nr = (E + 63) / 64;
    const unsigned long long below = (1ull << lane) - 1ull;
    const SelectCfg sel{E, k, a.norm, a.sigm, a.scale, a.bias};
    for (int t = wave; t < NT; t += 4) {
        const float shl = !a.sgi ? 0.f : LG_DENSE ? ld_agent(a.lg + (size_t)E * NT + t) : a.lg[(size_t)E * 32 + t];
        float v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = 64 * r + lane;
            v[r] = (r < nr && i < E) ? (LG_DENSE ? ld_agent(a.lg + (size_t)i * NT + t) : a.lg[(size_t)i * 32 + t])
                                     : -__builtin_inff();
        }
        int myid;
        float myw;
        select_token<R>(v, sel, a.rm ? a.rm + (size_t)t * E : nullptr, lane, myid, myw);
        if (lane < k) {
            S.ids[t * k + lane] = myid;
            S.w[t * k + lane] = myw;
            if (g == 0) {
                if (a.ids_out) a.ids_out[(size_t)t * a.ids_ld + lane] = myid;
                if (a.w_out) a.w_out[(size_t)t * a.w_ld + lane] = myw;
            }
        }
        if (lane == 0) S.shg[t] = a.sgi ? libm_sigmoid(shl) : 1.f;   // unary-ops.cpp:31
    }
    __syncthreads();
    // expert union through per-expert LDS tables: first pair, token mask, unit
    // (STEP_SELECT_LDS bytes: three tables of STEP_MAX_E words, E <= STEP_MAX_E)
    int32_t * tab_first = reinterpret_cast<int32_t *>(smem);
    uint32_t * tab_mask = reinterpret_cast<uint32_t *>(tab_first + STEP_MAX_E);
    int32_t * tab_unit = reinterpret_cast<int32_t *>(tab_mask + STEP_MAX_E);
    __shared__ unsigned long long s_bal[2];
    const int P = NT * k;
    const int p = tid;
    const int e = p < P ? S.ids[p] : 0;
    if (p < P) { tab_first[e] = 0x7fffffff; tab_mask[e] = 0u; }
    __syncthreads();
    if (p < P) { atomicMin(&tab_first[e], p); atomicOr(&tab_mask[e], 1u << (p / k)); }
    __syncthreads();
    const bool first = p < P && tab_first[e] == p;
    const uint32_t tmask = p < P ? tab_mask[e] : 0u;
    const unsigned long long bal = __ballot(first);
    if (lane == 0 && wave < 2) s_bal[wave] = bal;
    __syncthreads();
    const int nu = __popcll(s_bal[0]) + (P > 64 ? __popcll(s_bal[1]) : 0);
    if (first) {
        const int u = (wave == 1 ? __popcll(s_bal[0]) : 0) + __popcll(bal & below);
        S.units[u].expert = e;
        S.units[u].n = __popc(tmask);
        tab_unit[e] = u;
    }
    __syncthreads();
    if (p < P) {
        const int t = p / k;
        S.units[tab_unit[e]].pair[__popc(tmask & ((1u << t) - 1u))] = p;
    }
    __syncthreads();
    for (int u = tid; u < nu; u += 256)
        for (int r = 0; r < 3; ++r)   // table entries out of [0, S) are clamped into the pool
            S.uslot[u][r] = min(max(S.slot_of[r * E + S.units[u].expert], 0), a.n_slots[r] - 1);
    if (tid == 0) {
        if (a.shared) {
            S.units[nu].expert = -1;
            S.units[nu].n = NT;
            for (int i = 0; i < NT; ++i) S.units[nu].pair[i] = i;
        }
        S.nu = nu;
    }
    __syncthreads();
}

// ---------------------------------------------------------------- P2 ----
// gate/up: items of GU_ROWS = 32 consecutive rows of one unit (one whole
// 128-byte line of activations per token); workgroup g takes items g,
// g + G, ...  Each wave owns 8 rows, 8 lanes per row, in ggml-CPU's exact
// float order (qwm_exact.h): the unit's Q8_K activations are copied into LDS,
// both rows' blocks are requested at once, and act = silu(g) * u (the
// vectorized silu except for the row tail the CPU runs through scalar expf)
// leaves as agent-scope stores.  Each finished item counts for its unit.
constexpr int GU_ROWS = 32;

template <int MAXP>
QWM_DEV void step_gateup(const StepArgs & a, int g, int G, const StepShared & S, const uint32_t * s_xq) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m = lane & 7, rsub = lane >> 3;
    const int nb_r = (a.N + GU_ROWS - 1) / GU_ROWS, nb_s = a.shared ? (a.N_sh + GU_ROWS - 1) / GU_ROWS : 0;
    const int items = S.nu * nb_r + nb_s;
    constexpr size_t row_bytes = (size_t)SNB * 144;
    (void)tid;
    for (int item = g; item < items; item += G) {
        const bool shared = item >= S.nu * nb_r;
        const int u = shared ? S.nu : item / nb_r;
        const int blk = shared ? item - S.nu * nb_r : item % nb_r;
        const int rows = shared ? a.N_sh : a.N;
        const Unit & U_ = S.units[u];
        const int n = U_.n;
        const uint8_t * gbase = shared ? a.sh_gate : a.gate + (size_t)S.uslot[u][0] * a.gate_slab;
        const uint8_t * ubase = shared ? a.sh_up : a.up + (size_t)S.uslot[u][1] * a.up_slab;
        const int r = blk * GU_ROWS + wave * 8 + rsub;
        const int rc = min(r, rows - 1);                           // rows past the unit's last re-read it; dropped
        XBlk Gw[SNB], Uw[SNB];
#pragma unroll
        for (int b = 0; b < SNB; ++b) {
            load_xblk(Gw[b], gbase + (size_t)rc * row_bytes + b * 144, m);
            load_xblk(Uw[b], ubase + (size_t)rc * row_bytes + b * 144, m);
        }
        int off[MAXP];                                             // the unit's tokens in s_xq
#pragma unroll
        for (int i = 0; i < MAXP; ++i) {
            const int pi = i < n ? U_.pair[i] : 0;
            off[i] = (shared ? pi : pi / a.k) * (SNB * XS);
        }
        float gs[MAXP], us[MAXP];
        q4k_dot8_auto<SNB, MAXP>(gs, Gw, s_xq, off, n, m);
        q4k_dot8_auto<SNB, MAXP>(us, Uw, s_xq, off, n, m);
        if (m == 0 && r < rows) {
#pragma unroll
            for (int i = 0; i < MAXP; ++i)
                if (i < n) {
                    const float v = (r < rows - (rows & 15)) ? v_silu(gs[i]) * us[i] : gs[i] / (1.0f + libm_expf(-gs[i])) * us[i];
                    if (shared) st_agent(a.act_sh + (size_t)U_.pair[i] * rows + r, v);
                    else st_agent(a.act + (size_t)U_.pair[i] * rows + r, v);
                }
        }
        signal_count(a.gu_done + 32 * u);
    }
}

// ---------------------------------------------------------------- P3 ----
// down + combine: each unit's rows are cut into the same 16 tiles of 128 rows
// (whole 32-row lines); items (unit, tile) go to workgroups g, g + G, ...
// The workgroup requests the tile's first weight rows, quantizes the unit's
// activations to Q8_K in LDS and streams the rest of the tile, 8 lanes per
// row (q4k_dot8), outputs collected in LDS and written as whole
// lines; then it takes the tile's ticket, and the last of the U units
// combines the tile for every token (runtime.cpp:3815-3817 for T == 1,
// 4544-4550 for T > 1; then the shared expert and the residual).
constexpr int DN_TR = 128;

// D6: Q6_K down slabs (Q4_K_M files keep the last layers' ffn_down_exps in
// Q6_K): rows through q6k_dot8, read after the activations are in LDS.
template <int NT, int NB, int MAXP, bool D6>
QWM_DEV void step_down_t(const StepArgs & a, int g, int G, const StepShared & S, uint8_t * smem) {
    constexpr int RPS = 8;                       // rows per wave step
    constexpr int TR = DN_TR;                    // 16 tiles of 128 rows
    constexpr int NSTEP = TR / (4 * RPS);        // wave steps per tile
    constexpr int PF = NB <= 3 ? NSTEP : NB <= 4 ? 3 : 1;   // steps in flight
    constexpr int ntiles = SH / TR;
    constexpr size_t row_bytes = (size_t)NB * (D6 ? 210 : 144);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c8 = lane & 7, rsub = lane >> 3;
    const int U = S.nu + a.shared;
    const int nb_r = (a.N + GU_ROWS - 1) / GU_ROWS, nb_s = (a.N_sh + GU_ROWS - 1) / GU_ROWS;   // gate/up items per unit
    uint32_t * s_x = reinterpret_cast<uint32_t *>(smem);                        // [MAXP][NB][XS]
    float (*s_ex)[DN_TR] = reinterpret_cast<float (*)[DN_TR]>(smem + (size_t)MAXP * NB * XS * 4);
    for (int item = g; item < U * ntiles; item += G) {
        const int u = item / ntiles, x = item % ntiles;
        const bool shared = u == S.nu;
        const Unit & U_ = S.units[u];
        const int n = U_.n;
        const uint8_t * base = shared ? a.sh_down : a.down + (size_t)S.uslot[u][2] * a.down_slab;
        const int h0 = x * TR, h1 = h0 + TR;
        const uint8_t * rp = base + (size_t)(h0 + wave * RPS + rsub) * row_bytes;   // row of step st: + 4 * RPS * st
        // weights first: vector-memory waits count in issue order, and these
        // do not depend on the activations
        XBlk Wb[D6 ? 1 : PF][NB];
        if constexpr (!D6)
#pragma unroll
            for (int p = 0; p < PF; ++p)
#pragma unroll
                for (int b = 0; b < NB; ++b) load_xblk(Wb[p][b], rp + (size_t)(4 * RPS * p) * row_bytes + b * 144, c8);
        wait_count(a.gu_done + 32 * u, shared ? nb_s : nb_r, a.err, a.spin);   // the unit's activations are out
        for (int jb = wave; jb < n * NB; jb += 4) {
            const int i = jb / NB, b = jb % NB;
            const float * src = shared ? a.act_sh + (size_t)U_.pair[i] * (NB * QK_K)
                                       : a.act + (size_t)U_.pair[i] * (NB * QK_K);
            quantize_block_q8K_x<true>(src + b * QK_K, s_x + (i * NB + b) * XS, lane);
        }
        __syncthreads();
#pragma clang loop unroll(full)
        for (int st = 0; st < NSTEP; ++st) {
            const int p = st % PF;
            float acc[MAXP];
            if constexpr (D6) {
                q6k_dot8<NB, MAXP>(acc, rp + (size_t)(4 * RPS * st) * row_bytes, s_x, n, c8);
            } else {
                q4k_dot8<NB, MAXP>(acc, Wb[p], s_x, n, c8);
                if (st + PF < NSTEP)
#pragma unroll
                    for (int b = 0; b < NB; ++b)
                        load_xblk(Wb[p][b], rp + (size_t)(4 * RPS * (st + PF)) * row_bytes + b * 144, c8);
            }
            const int r = h0 + (st * 4 + wave) * RPS + rsub;
#pragma unroll
            for (int i = 0; i < MAXP; ++i)
                if (i < n && c8 == 0) s_ex[i][r - h0] = acc[i];
        }
        __syncthreads();
        for (int q = tid; q < n * (h1 - h0); q += 256) {
            const int i = q / (h1 - h0), h = h0 + q % (h1 - h0);
            if (shared) st_agent(a.ex_sh + (size_t)U_.pair[i] * SH + h, s_ex[i][h - h0]);
            else st_agent(a.ex + (size_t)U_.pair[i] * SH + h, s_ex[i][h - h0]);
        }
        if (last_workgroup(a.tile_counters + x, U)) {
            // every expert output of the tile is in: combine it, two outputs per
            // thread per pass with all their loads issued before any arithmetic
            const int k = a.k;
            const int TRh = h1 - h0;
            for (int q0 = tid; q0 < NT * TRh; q0 += 512) {
                float ev[2][MAX_K], shv[2], rv[2];
#pragma unroll
                for (int o = 0; o < 2; ++o) {
                    const int q = min(q0 + 256 * o, NT * TRh - 1);
                    const int t = q / TRh, h = h0 + q % TRh;
                    const float * e = a.ex + (size_t)t * k * SH + h;
#pragma unroll
                    for (int j = 0; j < MAX_K; ++j) ev[o][j] = j < k ? e[(size_t)j * SH] : 0.f;
                    shv[o] = a.shared ? a.ex_sh[(size_t)t * SH + h] : 0.f;
                    rv[o] = a.resid ? a.resid[(size_t)t * SH + h] : 0.f;
                }
#pragma unroll
                for (int o = 0; o < 2; ++o) {
                    const int q = q0 + 256 * o;
                    if (q >= NT * TRh) break;
                    const int t = q / TRh, h = h0 + q % TRh;
                    const float * wt = S.w + t * k;
                    float sacc;
                    if (NT == 1) {
                        // vec_dot_f32 with n = k <= 16: a 16-group, else an
                        // 8-group, of unfused products, then fused multiply-adds
                        sacc = 0.0f;
                        if (k >= 16) {
#pragma unroll
                            for (int l = 0; l < 16; ++l) sacc = sacc + ev[o][l] * wt[l];
                        } else {
                            const int g8 = k >= 8 ? 8 : 0;
#pragma unroll
                            for (int l = 0; l < 8; ++l)
                                if (l < g8) sacc = sacc + ev[o][l] * wt[l];
#pragma unroll
                            for (int l = 0; l < 16; ++l)
                                if (l >= g8 && l < k) sacc = __builtin_fmaf(ev[o][l], wt[l], sacc);
                        }
                    } else {
                        sacc = ev[o][0] * wt[0];
#pragma unroll
                        for (int j = 1; j < MAX_K; ++j)
                            if (j < k) sacc = sacc + ev[o][j] * wt[j];
                    }
                    if (a.shared) {
                        float vv = shv[o];
                        if (a.sgi) vv = vv * S.shg[t];
                        sacc = sacc + vv;
                    }
                    if (a.resid) sacc = sacc + rv[o];
                    st_agent(a.out + (size_t)t * SH + h, sacc);
                }
            }
            signal_count(a.tiles_done);
        }
        __syncthreads();
    }
}

template <int NT, int NB, int MAXP>
QWM_DEV void step_down(const StepArgs & a, int g, int G, const StepShared & S, uint8_t * smem) {
    if (a.d6) step_down_t<NT, NB, MAXP, true>(a, g, G, S, smem);
    else step_down_t<NT, NB, MAXP, false>(a, g, G, S, smem);
}

template <int NT, int NB_D>
__global__ void __launch_bounds__(256) k_step(StepArgs a) {
    constexpr int MAXP = NT <= 1 ? 1 : NT <= 2 ? 2 : NT <= 4 ? 4 : 8;
    constexpr size_t down_bytes = (size_t)MAXP * (NB_D * XS * 4 + DN_TR * 4);
    constexpr size_t smem_bytes = cmax(cmax(STEP_SELECT_LDS, down_bytes), VhSmem<NT>::bytes);
    __shared__ __align__(16) uint8_t smem[smem_bytes];
    __shared__ __align__(16) uint32_t s_xq[NT * SNB * XS];     // Q8_K of every token's x, exact layout [t][b]
    __shared__ StepShared S;
    const int g = blockIdx.x, G = gridDim.x;

    // the layer's slot tables, requested first and kept in LDS for the selection
    constexpr int SLQ = 3 * STEP_MAX_E / 256;
    int32_t sl[SLQ];
#pragma unroll
    for (int q = 0; q < SLQ; ++q) {
        const int idx = threadIdx.x + 256 * q;
        sl[q] = idx < 3 * a.E ? a.slot_tables[(size_t)(idx / a.E) * a.table_stride + (size_t)a.layer * a.E + idx % a.E] : 0;
    }
    step_router<NT>(a, g, G);
#pragma unroll
    for (int q = 0; q < SLQ; ++q) S.slot_of[threadIdx.x + 256 * q] = sl[q];
    wait_count(a.rows_done, step_p0_parts<NT>(a.E + (a.sgi ? 1 : 0), G), a.err, a.spin);   // ends with a workgroup barrier
    // Q8_K of x into LDS for the gate/up GEMVs: requested now, stored after
    // the selection, whose round trip and arithmetic hide the loads
    constexpr int XW = (NT * SNB * XS + 255) / 256;            // dwords per thread
    uint32_t xw[XW];
#pragma unroll
    for (int i = 0; i < XW; ++i) {
        const int q = threadIdx.x + 256 * i;
        xw[i] = q < NT * SNB * XS ? a.xq_x[(size_t)(q / XS) * XSP + q % XS] : 0u;
    }
    if (a.E <= 128) step_select<NT, 2>(a, g, S, smem);
    else step_select<NT, STEP_MAX_E / 64>(a, g, S, smem);
#pragma unroll
    for (int i = 0; i < XW; ++i) {
        const int q = threadIdx.x + 256 * i;
        if (q < NT * SNB * XS) s_xq[q] = xw[i];
    }
    __syncthreads();
    step_gateup<MAXP>(a, g, G, S, s_xq);
    step_down<NT, NB_D, MAXP>(a, g, G, S, smem);
    __syncthreads();
    constexpr int PF = NT <= 4 ? 2 : 1;
    if (verify_body<NT, SH / 512, PF, VH_BEFORE_WAIT>(a.v, g, G, smem, a.tiles_done, SH / DN_TR, a.err, a.spin)) {
        // every workgroup has passed all its waits: re-arm the completion
        // counters, and the tile tickets too (they re-arm themselves when
        // exactly U units arrive, but after a wait gave up the workgroups
        // may have selected from partial logits and disagree on U)
        for (int q = threadIdx.x; q < MAX_PAIRS + 1; q += 256) st_agent(a.gu_done + 32 * q, 0);
        if (threadIdx.x < SH / DN_TR) st_agent(a.tile_counters + threadIdx.x, 0);
        if (threadIdx.x == 0) { st_agent(a.tiles_done, 0); st_agent(a.rows_done, 0); }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            if (ld_agent(a.err)) {
                a.v.result[NT] = -1;
                a.v.result[NT + 1] = -1;
                st_agent(a.err, 0);
            }
        }
    }
}

}  // namespace qwm

namespace qwm {

constexpr int MAX_STEP_WG = 1024;

template <int NT, int NB_D>
static int step_grid() {
    static int grid = 0;
    if (!grid) {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return -1;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(k_step<NT, NB_D>), 256, 0) != hipSuccess)
            return -1;
        grid = std::min(std::min(per_cu, 2) * cus, MAX_STEP_WG);
    }
    return grid;
}

template <int NT, int NB_D>
static int launch_step_t(StepArgs & a, hipStream_t s) {
    const int G = step_grid<NT, NB_D>();
    if (G <= 0) return fail(QWM_ERR_HIP, "fused step: occupancy query failed");
    const int U_max = NT * a.k + a.shared;
    if (G < U_max) return fail(QWM_ERR_UNSUPPORTED, "fused step: fewer co-resident workgroups than expert units");
    if ((int64_t)a.v.V < 8LL * G) return fail(QWM_ERR_UNSUPPORTED, "fused step: vocabulary too small for the grid");
    // An ordinary launch of exactly the co-resident grid (the occupancy query
    // above): the cooperative launch API gives the same residency but costs
    // ~20 us between consecutive launches on this stack.  If other work holds
    // CUs, the missing workgroups start as it drains; the bounded spins report
    // a = -1 rather than wait without end.
    prof_begin("step", s);
    k_step<NT, NB_D><<<dim3((unsigned)G), dim3(256), 0, s>>>(a);
    prof_end("step", s);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(QWM_ERR_HIP, std::string("fused step launch: ") + hipGetErrorString(e));
    return QWM_OK;
}

template <int NT>
static int launch_step_nt(StepArgs & a, int nb_d, hipStream_t s) {
    switch (nb_d) {
        case 2: return launch_step_t<NT, 2>(a, s);
        case 3: return launch_step_t<NT, 3>(a, s);
        case 4: return launch_step_t<NT, 4>(a, s);
        default: return launch_step_t<NT, 8>(a, s);
    }
}

// the bound of the fused launches' waits (qwm_set_spin_limit)
uint32_t spin_limit();

// qwm_step_hi.hip: launch_step_nt<T> for T = 6, 7; qwm_step_t8.hip: T = 8
int launch_step_hi(StepArgs & a, int T, int nb_d, hipStream_t s);
int launch_step_t8(StepArgs & a, int nb_d, hipStream_t s);

}  // namespace qwm
