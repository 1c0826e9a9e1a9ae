// qwm_moe.hip -- the MoE FFN block on gfx950: router GEMV + softmax + top-k,
// Q8_K activation quantization, the expert-union schedule, the Q4_K
// gate/up GEMV with fused SwiGLU, the down GEMV, and the ordered combine.
//
// Layout of one GEMV wave: a weight row is split into 16-byte chunks of the
// Q4_K super-blocks' quant bytes (8 chunks per 144-byte block); LPR lanes
// cover one row (one chunk each, CPL chunks if K > 2048), so a wave streams
// 64/LPR rows per step with coalesced 128-bit loads, plus a 16-byte load of
// each block header (d, dmin, 12 scale bytes) shared by its 8 lanes.  The
// lane keeps the matching Q8_K activation bytes of every token of the unit
// in registers for the whole row loop.  Integer block sums are exact
// (v_dot4_i32_i8), so the result differs from ggml-CPU only by the order of
// the fp32 sums across blocks.
#include "qwm_device.h"
#include "qwm_internal.h"
#include "qwm_q4k.h"
#include "qwm_q80.h"
#include "qwm_exact.h"
#include "qwm_select.h"

namespace qwm {

// ======================================================================
// Router: logits, soft_max, top-k, weights, Q8_K of x, expert schedule
// ======================================================================

struct RouteKArgs {
    const float * W; const float * x; const float * rm; const float * sgi;
    int E, H, T, k, norm, sigm; float scale;
    const float * bias;                              // exp_probs_b [E] or null
    int n_row_wg;                                    // workgroups holding router rows
    float * logits; float * sh_logit;                // hand-off to the last workgroup
    int32_t * ids_ws; float * w_ws;                  // [T][k]
    int32_t * ids_out; int64_t ids_ld; float * w_out; int64_t w_ld;  // optional user copies
    const uint32_t * res_bits; int32_t * res_flag;   // residency bitmap of the layer's experts; miss flag (or null)
    float * sh_gate;                                 // [T] or null
    int8_t * xq_qs; float * xq_d; int32_t * xq_bs;   // Q8_K of x
    int q80; float * xq_d0;                         // Q8_0 pools: x as Q8_0 (qs in xq_qs, scales per 32)
    uint32_t * xq_x;                                 // Q4_K pools: x as Q8_K in the exact-dot layout [T][H/256][XS]
    Unit * units; int32_t * n_units; int32_t * counter;
    int shared;                                      // append the shared-expert unit
    const int32_t * slot_tables; int64_t table_stride; int layer; int32_t * slots_ws;  // [3][T*k]
    int32_t * uslot;                                 // resident mode: [unit][4] slots of each unit (gate, up, down)
};

// LDS of the last workgroup's expert union: first pair, token mask and unit
// per expert, and the layer's three slot-table rows (E <= 512).
constexpr int ROUTE_LDS_INTS = 3 * MAX_E + 3 * 512;

// One kernel for the whole routing step, one router row per workgroup (the
// whole row in one round trip of coalesced loads for H <= 2048, step by step
// for 3072 and 4096).
//  * Router rows in ggml_vec_dot_f32's AVX-512 order (ggml-cpu/vec.cpp:
//    11-135), which ggml-CPU runs per (row, token) at every token count
//    (ggml-cpu.c:1165-1244; the reference builds it without llamafile): one
//    token per wave, lane L = 16j + l accumulates over 64-wide steps, then
//    (j0+j2, j1+j3, 0+1) and the 16-lane tree.  The shared-gate row likewise.
//  * Q8_K of x (Q8_0 for Q8_0 pools), one 256-block per wave across the grid.
//  * The last workgroup: per token (one wave each) the selection of
//    select_token (qwm_select.h: soft_max or sigmoid, the optional ranking
//    bias, top-k, weights); then the expert union in first-occurrence order
//    and, in resident mode, the slot ids.
// R: probabilities per lane in the selection (E <= 64 R).
template <int R>
__global__ void __launch_bounds__(256) k_route(RouteKArgs a) {
    __shared__ __align__(16) int32_t smem[ROUTE_LDS_INTS];
    __shared__ int32_t s_ids[MAX_PAIRS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E, H = a.H, T = a.T, k = a.k;
    const int g = blockIdx.x, G = gridDim.x;

    // ---- Q8_K (Q4_K pools) or Q8_0 (Q8_0 pools) of x, the inputs of the
    // expert GEMVs, spread over every wave (from the last workgroup down, so
    // that the row workgroups start their loads first)
    {
        const int nb = H / QK_K;
        for (int jb = (G - 1 - g) * 4 + wave; jb < T * nb; jb += G * 4) {
            const int t = jb / nb, b = jb % nb;
            if (a.q80)
                quantize_q80_256(a.x + (size_t)t * H + b * QK_K, a.xq_qs + (size_t)t * H + b * QK_K,
                                 a.xq_d0 + (size_t)t * (H / 32) + b * 8, lane);
            else
                quantize_block_q8K_x(a.x + (size_t)t * H + b * QK_K, a.xq_x + (size_t)(t * nb + b) * XS, lane);
        }
    }

    const int rows = E + (a.sgi ? 1 : 0);
    if (g < rows && H > 2048) {
        // hidden sizes 3072 and 4096: the same lane order over more 64-wide
        // steps, the row and x read step by step
        const bool sh_row = g == E;
        const float * w = sh_row ? a.sgi : a.W + (size_t)g * H;
        const int ns = H / 64;
        for (int t = wave; t < T; t += 4) {
            const float * xr = a.x + (size_t)t * H;
            float acc = 0.f;
#pragma unroll 8
            for (int st = 0; st < ns; ++st) acc = __builtin_fmaf(w[64 * st + lane], xr[64 * st + lane], acc);
            acc += lane_xor32_f(acc);
            acc += lane_xor16_f(acc);
            acc = tree16_dpp(acc);
            if (lane == 0) {
                if (sh_row) st_agent(a.sh_logit + t, acc);
                else st_agent(a.logits + (size_t)t * E + g, a.rm ? acc + a.rm[(size_t)t * E + g] : acc);
            }
        }
    } else if (g < rows) {
        const bool sh_row = g == E;
        const float * w = sh_row ? a.sgi : a.W + (size_t)g * H;
        {
            const int ns = H / 64;
            float wv[32];
#pragma unroll
            for (int st = 0; st < 32; ++st)
                if (st < ns) wv[st] = w[64 * st + lane];
            for (int t = wave; t < T; t += 4) {
                const float * xr = a.x + (size_t)t * H;
                float xv[32];
#pragma unroll
                for (int st = 0; st < 32; ++st)
                    if (st < ns) xv[st] = xr[64 * st + lane];
                float acc = 0.f;
#pragma unroll
                for (int st = 0; st < 32; ++st)
                    if (st < ns) acc = __builtin_fmaf(wv[st], xv[st], acc);
                acc += lane_xor32_f(acc);
                acc += lane_xor16_f(acc);
                acc = tree16_dpp(acc);
                if (lane == 0) {
                    if (sh_row) st_agent(a.sh_logit + t, acc);
                    else st_agent(a.logits + (size_t)t * E + g, a.rm ? acc + a.rm[(size_t)t * E + g] : acc);
                }
            }
        }
    }

    // ---- last workgroup: selection and the expert schedule
    if (!last_workgroup(a.counter)) return;
    // The layer's slot-table rows (resident mode, E <= 512), requested before
    // the logits: they are read only by the union at the end, so their round
    // trip overlaps the selection's.
    constexpr bool PRE = R <= 8;
    constexpr int SQ = PRE ? (3 * 64 * R + 255) / 256 : 1;
    int32_t slq[SQ];
    if (PRE && a.slot_tables) {
#pragma unroll
        for (int q = 0; q < SQ; ++q) {
            const int idx = tid + 256 * q;
            slq[q] = idx < 3 * E ? a.slot_tables[(size_t)(idx / E) * a.table_stride + (size_t)a.layer * E + idx % E] : 0;
        }
    }
    const int nr = (E + 63) / 64;
    const SelectCfg sel{E, k, a.norm, a.sigm, a.scale, a.bias};
    for (int t = wave; t < T; t += 4) {
        const float * lt = a.logits + (size_t)t * E;
        float v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = 64 * r + lane;
            v[r] = (r < nr && i < E) ? ld_agent(lt + i) : -__builtin_inff();
        }
        int myid;
        float myw;
        select_token<R>(v, sel, a.rm ? a.rm + (size_t)t * E : nullptr, lane, myid, myw);
        // the optimistic path's residency check (runtime.cpp:6155-6166): a
        // selected expert without its bit ran on the slot-0 sentinel
        if (a.res_bits && lane < k && !((a.res_bits[myid >> 5] >> (myid & 31)) & 1u)) st_agent(a.res_flag, 1);
        if (lane < k) {
            s_ids[t * k + lane] = myid;
            a.ids_ws[t * k + lane] = myid;
            a.w_ws[t * k + lane] = myw;
            if (a.ids_out) a.ids_out[(size_t)t * a.ids_ld + lane] = myid;
            if (a.w_out) a.w_out[(size_t)t * a.w_ld + lane] = myw;
        }
        if (lane == 0 && a.sh_gate) a.sh_gate[t] = libm_sigmoid(ld_agent(a.sh_logit + t));   // unary-ops.cpp:31
    }
    __syncthreads();

    // expert union through per-expert LDS tables: first pair, token mask, unit
    int32_t * tab_first = smem;
    uint32_t * tab_mask = reinterpret_cast<uint32_t *>(tab_first + MAX_E);
    int32_t * tab_unit = reinterpret_cast<int32_t *>(tab_mask + MAX_E);
    int32_t * tab_slot = tab_unit + MAX_E;                 // [3][E] when PRE
    static_assert(!PRE || 3 * MAX_E + 3 * 64 * R <= ROUTE_LDS_INTS, "slot rows fit in LDS");
    if (PRE && a.slot_tables) {
#pragma unroll
        for (int q = 0; q < SQ; ++q)
            if (tid + 256 * q < 3 * E) tab_slot[tid + 256 * q] = slq[q];
    }
    __shared__ unsigned long long s_bal[2];
    const int P = T * k;
    const int p = tid;
    const int e = p < P ? s_ids[p] : 0;
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
        const int u = (wave == 1 ? __popcll(s_bal[0]) : 0) + __popcll(bal & ((1ull << lane) - 1ull));
        a.units[u].expert = e;
        a.units[u].n = __popc(tmask);
        tab_unit[e] = u;
        if (a.slot_tables)
            for (int r = 0; r < 3; ++r)
                a.uslot[4 * u + r] = PRE ? tab_slot[r * E + e] : a.slot_tables[(size_t)r * a.table_stride + (size_t)a.layer * E + e];
    }
    __syncthreads();
    if (p < P) {
        const int t = p / k;
        a.units[tab_unit[e]].pair[__popc(tmask & ((1u << t) - 1u))] = p;
        if (a.slot_tables)
            for (int r = 0; r < 3; ++r)
                a.slots_ws[r * P + p] = PRE ? tab_slot[r * E + e] : a.slot_tables[(size_t)r * a.table_stride + (size_t)a.layer * E + e];
    }
    if (tid == 0) {
        if (a.shared) {
            Unit & u = a.units[nu];
            u.expert = -1;
            u.n = T;
            for (int i = 0; i < T; ++i) u.pair[i] = i;
        }
        *a.n_units = nu;
    }
}

// ---------------------------------------------------------------------
// gate/up + SwiGLU: act[p][r] = silu(gate_e[r] . x_t) * (up_e[r] . x_t)
// grid: (row tiles, unit slots [+1 for the shared expert]), block 256.
// ---------------------------------------------------------------------
struct GateUpArgs {
    const uint8_t * gate; const uint8_t * up; size_t gate_slab, up_slab;
    const uint8_t * sh_gate; const uint8_t * sh_up;
    const int32_t * slot_g; const int32_t * slot_u;
    const int32_t * uslot;                                        // [unit][4] or null: slots through the pairs
    int S_g, S_u;                                                 // slots per pool
    const Unit * units; const int32_t * n_units; int unit_slots;  // routed unit grid rows
    const int8_t * xq_qs; const float * xq_d; const int32_t * xq_bs;
    const uint32_t * xq_x;                                        // Q8_K of x, exact-dot layout (Q4_K pools)
    float * act; float * act_sh;
    int H, N, N_sh, k, T;
};

// The workgroup's unit: its pairs (token-major (t, j) indices; the shared
// expert's unit is every token) and slot.  The unit count, the unit and its
// resident-mode slot are requested together, before the empty-unit exit, so
// the weight loads wait for one round trip instead of three.
template <int MAXP>
struct UnitView {
    int n;
    int pair[MAXP];
    int slot[2];
};
template <int MAXP>
QWM_DEV bool load_unit(UnitView<MAXP> & V, const Unit * units, const int32_t * n_units, const int32_t * uslot,
                       const int32_t * slot_a, const int32_t * slot_b, int u, bool shared, int T, int role_a,
                       int role_b, int S_a, int S_b, int & nu) {
    nu = *n_units;
    if (shared) {
        V.n = T;
#pragma unroll
        for (int i = 0; i < MAXP; ++i) V.pair[i] = i;
        V.slot[0] = V.slot[1] = 0;
        return true;
    }
    const Unit & U = units[u];
    const int n = U.n;
    int pr[MAXP];
#pragma unroll
    for (int i = 0; i < MAXP; ++i) pr[i] = U.pair[i];
    int sa = 0, sb = 0;
    if (uslot) { sa = uslot[4 * u + role_a]; sb = uslot[4 * u + role_b]; }
    if (u >= nu) return false;
    if (!uslot) { sa = slot_a[pr[0]]; sb = slot_b ? slot_b[pr[0]] : 0; }
    // caller slot ids out of [0, S) are clamped into the pool: wrong weights,
    // but no read outside it
    sa = min(max(sa, 0), S_a - 1);
    sb = min(max(sb, 0), S_b - 1);
    V.n = n;
#pragma unroll
    for (int i = 0; i < MAXP; ++i) V.pair[i] = pr[i];
    V.slot[0] = sa; V.slot[1] = sb;
    return true;
}

// Q4_K gate/up in ggml-CPU's exact float order (qwm_exact.h): 8 lanes per
// row, a workgroup owns 32 consecutive rows (4 waves x 8 rows) of one unit.
// The unit's Q8_K activations are copied into LDS first; SwiGLU then sees the
// CPU's gate and up values bit for bit.
constexpr int GUX_ROWS = 32;

template <int NB, int MAXP>
__global__ void __launch_bounds__(256) k_gateup_x(GateUpArgs a) {
    __shared__ __align__(16) uint32_t s_x[MAXP * NB * XS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m = lane & 7, rsub = lane >> 3;
    const int u = blockIdx.y;
    const bool shared = u == a.unit_slots;
    UnitView<MAXP> U;
    int nu;
    if (!load_unit<MAXP>(U, a.units, a.n_units, a.uslot, a.slot_g, a.slot_u, u, shared, a.T, 0, 1, a.S_g, a.S_u, nu)) return;
    const int n = U.n;
    const int rows = shared ? a.N_sh : a.N;
    const int r = blockIdx.x * GUX_ROWS + wave * 8 + rsub;
    if (blockIdx.x * GUX_ROWS >= rows) return;
    const size_t row_bytes = (size_t)NB * 144;
    const uint8_t * gbase = shared ? a.sh_gate : a.gate + (size_t)U.slot[0] * a.gate_slab;
    const uint8_t * ubase = shared ? a.sh_up : a.up + (size_t)U.slot[1] * a.up_slab;
    const int rc = min(r, rows - 1);
    // rows of up to 8 blocks are requested whole before the activations are
    // copied; longer rows (hidden sizes 3072 and 4096) in double-buffered
    // chunks of 4 blocks after it (q4k_dot8_chunked)
    constexpr int NBR = NB <= 8 ? NB : 1;
    XBlk G[NBR], W[NBR];
    if constexpr (NB <= 8) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            load_xblk(G[b], gbase + (size_t)rc * row_bytes + b * 144, m);
            load_xblk(W[b], ubase + (size_t)rc * row_bytes + b * 144, m);
        }
    }
    // the unit's tokens' activation blocks into LDS (uint4 copies)
    constexpr int Q4 = NB * XS / 4;
    for (int q = tid; q < n * Q4; q += 256) {
        const int i = q / Q4, o = q % Q4;
        int pi = U.pair[0];              // U.pair[i] by selects (a dynamic index would put U in scratch)
#pragma unroll
        for (int qq = 1; qq < MAXP; ++qq) if (i == qq) pi = U.pair[qq];
        const int t = shared ? pi : pi / a.k;
        reinterpret_cast<uint4 *>(s_x)[i * Q4 + o] = reinterpret_cast<const uint4 *>(a.xq_x + (size_t)t * NB * XS)[o];
    }
    __syncthreads();
    float g[MAXP], up[MAXP];
    if constexpr (NB <= 8) {
        q4k_dot8<NB, MAXP>(g, G, s_x, n, m);
        q4k_dot8<NB, MAXP>(up, W, s_x, n, m);
    } else {
        const uint8_t * const rw[2] = {gbase + (size_t)rc * row_bytes, ubase + (size_t)rc * row_bytes};
        float gu[2][MAXP];
        q4k_dot8_chunked<NB, 4, 2, MAXP>(gu, rw, s_x, n, m);
#pragma unroll
        for (int i = 0; i < MAXP; ++i) { g[i] = gu[0][i]; up[i] = gu[1][i]; }
    }
    if (m == 0 && r < rows) {
#pragma unroll
        for (int i = 0; i < MAXP; ++i)
            if (i < n) {
                const float v = (r < rows - (rows & 15)) ? v_silu(g[i]) * up[i] : g[i] / (1.0f + libm_expf(-g[i])) * up[i];
                if (shared) a.act_sh[(size_t)U.pair[i] * rows + r] = v;
                else a.act[(size_t)U.pair[i] * rows + r] = v;
            }
    }
}

// k_gateup_x for Q5_K gate/up pools: the same mapping and activations,
// rows through q5k_dot8.
template <int NB, int MAXP>
__global__ void __launch_bounds__(256) k_gateup_x5(GateUpArgs a) {
    __shared__ __align__(16) uint32_t s_x[MAXP * NB * XS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m = lane & 7, rsub = lane >> 3;
    const int u = blockIdx.y;
    const bool shared = u == a.unit_slots;
    UnitView<MAXP> U;
    int nu;
    if (!load_unit<MAXP>(U, a.units, a.n_units, a.uslot, a.slot_g, a.slot_u, u, shared, a.T, 0, 1, a.S_g, a.S_u, nu)) return;
    const int n = U.n;
    const int rows = shared ? a.N_sh : a.N;
    const int r = blockIdx.x * GUX_ROWS + wave * 8 + rsub;
    if (blockIdx.x * GUX_ROWS >= rows) return;
    const size_t row_bytes = (size_t)NB * 176;
    const uint8_t * gbase = shared ? a.sh_gate : a.gate + (size_t)U.slot[0] * a.gate_slab;
    const uint8_t * ubase = shared ? a.sh_up : a.up + (size_t)U.slot[1] * a.up_slab;
    const int rc = min(r, rows - 1);
    // the unit's tokens' activation blocks into LDS (uint4 copies)
    constexpr int Q4 = NB * XS / 4;
    for (int q = tid; q < n * Q4; q += 256) {
        const int i = q / Q4, o = q % Q4;
        int pi = U.pair[0];              // U.pair[i] by selects (a dynamic index would put U in scratch)
#pragma unroll
        for (int qq = 1; qq < MAXP; ++qq) if (i == qq) pi = U.pair[qq];
        const int t = shared ? pi : pi / a.k;
        reinterpret_cast<uint4 *>(s_x)[i * Q4 + o] = reinterpret_cast<const uint4 *>(a.xq_x + (size_t)t * NB * XS)[o];
    }
    __syncthreads();
    float g[MAXP], up[MAXP];
    q5k_dot8<NB, MAXP>(g, gbase + (size_t)rc * row_bytes, s_x, n, m);
    q5k_dot8<NB, MAXP>(up, ubase + (size_t)rc * row_bytes, s_x, n, m);
    if (m == 0 && r < rows) {
#pragma unroll
        for (int i = 0; i < MAXP; ++i)
            if (i < n) {
                const float v = (r < rows - (rows & 15)) ? v_silu(g[i]) * up[i] : g[i] / (1.0f + libm_expf(-g[i])) * up[i];
                if (shared) a.act_sh[(size_t)U.pair[i] * rows + r] = v;
                else a.act[(size_t)U.pair[i] * rows + r] = v;
            }
    }
}

// The Q8_0 form of k_gateup_x: ggml's Q8_0 dot order (q80_dot8), the unit's
// Q8_0 activations in LDS.
template <int NPAIR, int MAXP>
__global__ void __launch_bounds__(256) k_gateup_x80(GateUpArgs a) {
    constexpr int K = NPAIR * 64;
    __shared__ __align__(16) uint32_t s_q[MAXP * K / 4];
    __shared__ float s_d[MAXP * K / 32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m = lane & 7, rsub = lane >> 3;
    const int u = blockIdx.y;
    const bool shared = u == a.unit_slots;
    UnitView<MAXP> U;
    int nu;
    if (!load_unit<MAXP>(U, a.units, a.n_units, a.uslot, a.slot_g, a.slot_u, u, shared, a.T, 0, 1, a.S_g, a.S_u, nu)) return;
    const int n = U.n;
    const int rows = shared ? a.N_sh : a.N;
    const int r = blockIdx.x * GUX_ROWS + wave * 8 + rsub;
    if (blockIdx.x * GUX_ROWS >= rows) return;
    const size_t row_bytes = (size_t)NPAIR * 68;
    const uint8_t * gbase = shared ? a.sh_gate : a.gate + (size_t)U.slot[0] * a.gate_slab;
    const uint8_t * ubase = shared ? a.sh_up : a.up + (size_t)U.slot[1] * a.up_slab;
    const int rc = min(r, rows - 1);
    for (int q = tid; q < n * (K / 16); q += 256) {
        const int i = q / (K / 16), o = q % (K / 16);
        int pi = U.pair[0];              // U.pair[i] by selects (a dynamic index would put U in scratch)
#pragma unroll
        for (int qq = 1; qq < MAXP; ++qq) if (i == qq) pi = U.pair[qq];
        const int t = shared ? pi : pi / a.k;
        reinterpret_cast<uint4 *>(s_q)[i * (K / 16) + o] = reinterpret_cast<const uint4 *>(a.xq_qs + (size_t)t * K)[o];
        if (o < K / 32) s_d[i * (K / 32) + o] = a.xq_d[(size_t)t * (K / 32) + o];
    }
    __syncthreads();
    float g[MAXP], up[MAXP];
    q80_dot8<NPAIR, MAXP>(g, gbase + (size_t)rc * row_bytes, s_q, s_d, K / 4, K / 32, n, m);
    q80_dot8<NPAIR, MAXP>(up, ubase + (size_t)rc * row_bytes, s_q, s_d, K / 4, K / 32, n, m);
    if (m == 0 && r < rows) {
#pragma unroll
        for (int i = 0; i < MAXP; ++i)
            if (i < n) {
                const float v = (r < rows - (rows & 15)) ? v_silu(g[i]) * up[i] : g[i] / (1.0f + libm_expf(-g[i])) * up[i];
                if (shared) a.act_sh[(size_t)U.pair[i] * rows + r] = v;
                else a.act[(size_t)U.pair[i] * rows + r] = v;
            }
    }
}

// ---------------------------------------------------------------------
// down: ex[p][h] = down_e[h] . Q8_K(act[p]), then the combine of the row tile
// grid: (row tiles over H, unit slots [+1 shared]), block 256.  Each block
// first quantizes its unit's activation rows to Q8_K in LDS.  The last unit
// to finish a row tile combines it for every token:
//   out[t][h] = sum_j ex[t,j][h] * w[t][j] (+ shared) (+ resid)
//   T == 1: ggml_vec_dot_f32 with n = k (runtime.cpp:3815-3817): the whole
//           sum is the scalar tail, gcc-vectorized as unfused 16/8 groups,
//           then fused multiply-adds.
//   T  > 1: ggml_mul then the ggml_add chain (runtime.cpp:4544-4550).
// ---------------------------------------------------------------------
struct DownArgs {
    const uint8_t * down; size_t down_slab; const uint8_t * sh_down;
    const int32_t * slot_d;
    const int32_t * uslot;
    int S_d;                                                      // slots in the down pool
    const Unit * units; const int32_t * n_units; int unit_slots; int shared;
    const float * act; const float * act_sh;
    float * ex; float * ex_sh;
    int H, N, N_sh, k, T;
    int32_t * tile_counters;
    const float * w; const float * sh_gate; const float * resid; float * out;
};

constexpr int MAX_NDOWN = 2048;   // longest down-projection input held in LDS

QWM_DEV float combine_one(const DownArgs & a, int t, int h) {
    const int H = a.H, k = a.k;
    const float * wt = a.w + (size_t)t * k;
    const float * e = a.ex + (size_t)t * k * H + h;
    float s;
    if (a.T == 1) {
        s = 0.0f;
        int i = 0;
        for (; k - i >= 16; i += 16)
            for (int l = 0; l < 16; ++l) s = s + ld_agent(e + (size_t)(i + l) * H) * wt[i + l];
        if (k - i >= 8) {
            for (int l = 0; l < 8; ++l) s = s + ld_agent(e + (size_t)(i + l) * H) * wt[i + l];
            i += 8;
        }
        for (; i < k; ++i) s = __builtin_fmaf(ld_agent(e + (size_t)i * H), wt[i], s);
    } else {
        s = ld_agent(e) * wt[0];
        for (int j = 1; j < k; ++j) s = s + ld_agent(e + (size_t)j * H) * wt[j];
    }
    if (a.shared) {
        float v = ld_agent(a.ex_sh + (size_t)t * H + h);
        if (a.sh_gate) v = v * a.sh_gate[t];
        s = s + v;
    }
    if (a.resid) s = s + a.resid[(size_t)t * H + h];
    return s;
}

// Rows go 8 lanes each (q4k_dot8, NB = FFN width / 256 Q4_K blocks per
// row): a workgroup owns a tile of 32 rows, one wave step each.
template <int NB, int MAXP>
__global__ void __launch_bounds__(256) k_down_q4k(DownArgs a) {
    constexpr int RPS = 8;                   // rows per wave
    constexpr int TILE = 4 * RPS;
    constexpr size_t row_bytes = (size_t)NB * 144;
    __shared__ __align__(16) uint32_t s_x[MAXP * NB * XS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c8 = lane & 7, rsub = lane >> 3;
    const int u = blockIdx.y;
    const bool shared = u == a.unit_slots;
    UnitView<MAXP> U;
    int nu;
    if (!load_unit<MAXP>(U, a.units, a.n_units, a.uslot, a.slot_d, nullptr, u, shared, a.T, 2, 2, a.S_d, a.S_d, nu)) return;
    const int n = U.n;
    const uint8_t * base = shared ? a.sh_down : a.down + (size_t)U.slot[0] * a.down_slab;
    const int row0 = blockIdx.x * TILE;
    const int r = row0 + wave * RPS + rsub;
    // weight loads first: they do not depend on the activations
    XBlk W[NB];
    const uint8_t * rp = base + (size_t)min(r, a.H - 1) * row_bytes;
#pragma unroll
    for (int b = 0; b < NB; ++b) load_xblk(W[b], rp + b * 144, c8);
    // the unit's activation rows to Q8_K in the exact-dot layout (one 256-block per wave at a time)
    for (int jb = wave; jb < n * NB; jb += 4) {
        const int i = jb / NB, b = jb % NB;
        int pi = U.pair[0];              // U.pair[i] by selects (a dynamic index would put U in scratch)
#pragma unroll
        for (int q = 1; q < MAXP; ++q) if (i == q) pi = U.pair[q];
        const float * src = shared ? a.act_sh + (size_t)pi * (NB * QK_K) : a.act + (size_t)pi * (NB * QK_K);
        quantize_block_q8K_x(src + b * QK_K, s_x + (i * NB + b) * XS, lane);
    }
    __syncthreads();
    float acc[MAXP];
    q4k_dot8<NB, MAXP>(acc, W, s_x, n, c8);
#pragma unroll
    for (int i = 0; i < MAXP; ++i)
        if (i < n && c8 == 0 && r < a.H) {
            if (shared) st_agent(a.ex_sh + (size_t)U.pair[i] * a.H + r, acc[i]);
            else st_agent(a.ex + (size_t)U.pair[i] * a.H + r, acc[i]);
        }
    if (!last_workgroup(a.tile_counters + blockIdx.x, nu + a.shared)) return;
    for (int q = tid; q < a.T * TILE; q += 256) {
        const int t = q / TILE, h = row0 + q % TILE;
        if (h < a.H) a.out[(size_t)t * a.H + h] = combine_one(a, t, h);
    }
}

// k_down_q4k for Q6_K down pools (Q4_K_M model files store some layers'
// ffn_down_exps as Q6_K): the same tiles and combine, rows through q6k_dot8.
template <int NB, int MAXP>
__global__ void __launch_bounds__(256) k_down_q6k(DownArgs a) {
    constexpr int RPS = 8;                   // rows per wave
    constexpr int TILE = 4 * RPS;
    constexpr size_t row_bytes = (size_t)NB * 210;
    __shared__ __align__(16) uint32_t s_x[MAXP * NB * XS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c8 = lane & 7, rsub = lane >> 3;
    const int u = blockIdx.y;
    const bool shared = u == a.unit_slots;
    UnitView<MAXP> U;
    int nu;
    if (!load_unit<MAXP>(U, a.units, a.n_units, a.uslot, a.slot_d, nullptr, u, shared, a.T, 2, 2, a.S_d, a.S_d, nu)) return;
    const int n = U.n;
    const uint8_t * base = shared ? a.sh_down : a.down + (size_t)U.slot[0] * a.down_slab;
    const int row0 = blockIdx.x * TILE;
    const int r = row0 + wave * RPS + rsub;
    const uint8_t * rp = base + (size_t)min(r, a.H - 1) * row_bytes;
    // the unit's activation rows to Q8_K in the exact-dot layout (one 256-block per wave at a time)
    for (int jb = wave; jb < n * NB; jb += 4) {
        const int i = jb / NB, b = jb % NB;
        int pi = U.pair[0];              // U.pair[i] by selects (a dynamic index would put U in scratch)
#pragma unroll
        for (int q = 1; q < MAXP; ++q) if (i == q) pi = U.pair[q];
        const float * src = shared ? a.act_sh + (size_t)pi * (NB * QK_K) : a.act + (size_t)pi * (NB * QK_K);
        quantize_block_q8K_x(src + b * QK_K, s_x + (i * NB + b) * XS, lane);
    }
    __syncthreads();
    float acc[MAXP];
    q6k_dot8<NB, MAXP>(acc, rp, s_x, n, c8);
#pragma unroll
    for (int i = 0; i < MAXP; ++i)
        if (i < n && c8 == 0 && r < a.H) {
            if (shared) st_agent(a.ex_sh + (size_t)U.pair[i] * a.H + r, acc[i]);
            else st_agent(a.ex + (size_t)U.pair[i] * a.H + r, acc[i]);
        }
    if (!last_workgroup(a.tile_counters + blockIdx.x, nu + a.shared)) return;
    for (int q = tid; q < a.T * TILE; q += 256) {
        const int t = q / TILE, h = row0 + q % TILE;
        if (h < a.H) a.out[(size_t)t * a.H + h] = combine_one(a, t, h);
    }
}

// k_down_q4k for Q5_K down pools (Q5_K_S/M model files): rows through q5k_dot8.
template <int NB, int MAXP>
__global__ void __launch_bounds__(256) k_down_q5k(DownArgs a) {
    constexpr int RPS = 8;                   // rows per wave
    constexpr int TILE = 4 * RPS;
    constexpr size_t row_bytes = (size_t)NB * 176;
    __shared__ __align__(16) uint32_t s_x[MAXP * NB * XS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c8 = lane & 7, rsub = lane >> 3;
    const int u = blockIdx.y;
    const bool shared = u == a.unit_slots;
    UnitView<MAXP> U;
    int nu;
    if (!load_unit<MAXP>(U, a.units, a.n_units, a.uslot, a.slot_d, nullptr, u, shared, a.T, 2, 2, a.S_d, a.S_d, nu)) return;
    const int n = U.n;
    const uint8_t * base = shared ? a.sh_down : a.down + (size_t)U.slot[0] * a.down_slab;
    const int row0 = blockIdx.x * TILE;
    const int r = row0 + wave * RPS + rsub;
    const uint8_t * rp = base + (size_t)min(r, a.H - 1) * row_bytes;
    // the unit's activation rows to Q8_K in the exact-dot layout (one 256-block per wave at a time)
    for (int jb = wave; jb < n * NB; jb += 4) {
        const int i = jb / NB, b = jb % NB;
        int pi = U.pair[0];              // U.pair[i] by selects (a dynamic index would put U in scratch)
#pragma unroll
        for (int q = 1; q < MAXP; ++q) if (i == q) pi = U.pair[q];
        const float * src = shared ? a.act_sh + (size_t)pi * (NB * QK_K) : a.act + (size_t)pi * (NB * QK_K);
        quantize_block_q8K_x(src + b * QK_K, s_x + (i * NB + b) * XS, lane);
    }
    __syncthreads();
    float acc[MAXP];
    q5k_dot8<NB, MAXP>(acc, rp, s_x, n, c8);
#pragma unroll
    for (int i = 0; i < MAXP; ++i)
        if (i < n && c8 == 0 && r < a.H) {
            if (shared) st_agent(a.ex_sh + (size_t)U.pair[i] * a.H + r, acc[i]);
            else st_agent(a.ex + (size_t)U.pair[i] * a.H + r, acc[i]);
        }
    if (!last_workgroup(a.tile_counters + blockIdx.x, nu + a.shared)) return;
    for (int q = tid; q < a.T * TILE; q += 256) {
        const int t = q / TILE, h = row0 + q % TILE;
        if (h < a.H) a.out[(size_t)t * a.H + h] = combine_one(a, t, h);
    }
}

// The Q8_0 form of k_down_q4k: weight blocks of 32 (one per lane per step of
// the row), activations quantized to Q8_0 in LDS (ggml's x86 quantizer, the
// vec_dot_type of Q8_0).
template <int NB, int MAXP>
__global__ void __launch_bounds__(256) k_down_q80(DownArgs a) {
    constexpr int RPS = 8;                   // rows per wave
    constexpr int TILE = 4 * RPS;
    constexpr int K = NB * QK_K;             // FFN width
    constexpr size_t row_bytes = (size_t)(K / 32) * 34;
    __shared__ __align__(16) uint32_t s_q[MAXP * K / 4];
    __shared__ float s_d[MAXP * K / 32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c8 = lane & 7, rsub = lane >> 3;
    const int u = blockIdx.y;
    const bool shared = u == a.unit_slots;
    UnitView<MAXP> U;
    int nu;
    if (!load_unit<MAXP>(U, a.units, a.n_units, a.uslot, a.slot_d, nullptr, u, shared, a.T, 2, 2, a.S_d, a.S_d, nu)) return;
    const int n = U.n;
    const uint8_t * base = shared ? a.sh_down : a.down + (size_t)U.slot[0] * a.down_slab;
    const int row0 = blockIdx.x * TILE;
    const int r = row0 + wave * RPS + rsub;
    const uint8_t * rowp = base + (size_t)min(r, a.H - 1) * row_bytes;
    for (int jb = wave; jb < n * NB; jb += 4) {
        const int i = jb / NB, b = jb % NB;
        int pi = U.pair[0];              // U.pair[i] by selects (a dynamic index would put U in scratch)
#pragma unroll
        for (int q = 1; q < MAXP; ++q) if (i == q) pi = U.pair[q];
        const float * src = shared ? a.act_sh + (size_t)pi * K : a.act + (size_t)pi * K;
        quantize_q80_256(src + b * QK_K, reinterpret_cast<int8_t *>(s_q + i * (K / 4)) + b * QK_K,
                         s_d + i * (K / 32) + b * 8, lane);
    }
    __syncthreads();
    float acc[MAXP];
    q80_dot8<K / 64, MAXP>(acc, rowp, s_q, s_d, K / 4, K / 32, n, c8);
#pragma unroll
    for (int i = 0; i < MAXP; ++i)
        if (i < n && c8 == 0 && r < a.H) {
            if (shared) st_agent(a.ex_sh + (size_t)U.pair[i] * a.H + r, acc[i]);
            else st_agent(a.ex + (size_t)U.pair[i] * a.H + r, acc[i]);
        }
    if (!last_workgroup(a.tile_counters + blockIdx.x, nu + a.shared)) return;
    for (int q = tid; q < a.T * TILE; q += 256) {
        const int t = q / TILE, h = row0 + q % TILE;
        if (h < a.H) a.out[(size_t)t * a.H + h] = combine_one(a, t, h);
    }
}

// ======================================================================
// host launchers
// ======================================================================

bool moe_plan(const qwm_moe_layer * L, int64_t T, MoePlan & p, std::string & why) {
    p.H = L->router.ne[0];
    p.E = L->router.ne[1];
    p.k = L->n_expert_used;
    p.T = T;
    p.N = L->gate_pool.ne[1];
    p.shared = L->sh_gate.data != nullptr;
    p.shared_gate = L->sh_gate_inp.data != nullptr;
    p.N_sh = p.shared ? L->sh_gate.ne[1] : 0;
    if (T < 1 || T > MAX_T) { why = "T must be in [1, 8]"; return false; }
    if (p.k < 1 || p.k > MAX_K || p.k > p.E) { why = "n_expert_used out of range"; return false; }
    if (p.E < 1 || p.E > MAX_E) { why = "n_expert out of range"; return false; }
    if (!hidden_supported(p.H)) { why = "hidden size must be a multiple of 256 up to 2048, 3072 or 4096"; return false; }
    if (p.N % QK_K || p.N > MAX_NDOWN) { why = "expert FFN size must be a multiple of 256, <= 2048"; return false; }
    if (p.shared && p.N_sh != p.N) { why = "the shared expert's FFN width must equal the routed one"; return false; }
    const int64_t P = T * p.k;
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    p.counters = take(256);
    p.tile_counters = take(sizeof(int32_t) * MAX_TILES);
    p.logits = take(sizeof(float) * T * p.E);
    p.ids = take(sizeof(int32_t) * P);
    p.w = take(sizeof(float) * P);
    p.slots = take(sizeof(int32_t) * 3 * P);
    p.sh_gate = take(sizeof(float) * (T + 1));
    p.n_units = take(sizeof(int32_t));
    p.units = take(sizeof(Unit) * (P + 1));
    p.uslot = take(sizeof(int32_t) * 4 * (P + 1));
    p.xq_qs = take((size_t)T * p.H);
    p.xq_d = take(sizeof(float) * T * (p.H / QK_K));
    p.xq_bs = take(sizeof(int32_t) * T * (p.H / 16));
    p.xq_d0 = take(sizeof(float) * T * (p.H / 32));
    p.xq_x = take(sizeof(uint32_t) * T * (p.H / QK_K) * XS);
    p.act = take(sizeof(float) * P * p.N);
    p.act_sh = take(sizeof(float) * T * (p.N_sh ? p.N_sh : 1));
    p.ex = take(sizeof(float) * P * p.H);
    p.ex_sh = take(sizeof(float) * T * p.H);
    p.total = o;
    return true;
}

int launch_route(const RouteArgs & a, const MoePlan & p, uint8_t * ws, int32_t * ids_out, int64_t ids_ld,
                 float * w_out, int64_t w_ld, hipStream_t s) {
    RouteKArgs r;
    r.W = a.W; r.x = a.x; r.rm = a.rm; r.sgi = a.sh_gate_inp;
    r.E = (int)a.E; r.H = (int)a.H; r.T = (int)a.T; r.k = (int)a.k; r.norm = a.norm; r.scale = a.scale;
    r.sigm = a.sigm; r.bias = a.bias;
    r.n_row_wg = (int)a.E;
    r.logits = reinterpret_cast<float *>(ws + p.logits);
    float * sh = reinterpret_cast<float *>(ws + p.sh_gate);
    r.sh_logit = sh + p.T;
    r.ids_ws = reinterpret_cast<int32_t *>(ws + p.ids);
    r.w_ws = reinterpret_cast<float *>(ws + p.w);
    r.ids_out = ids_out; r.ids_ld = ids_ld; r.w_out = w_out; r.w_ld = w_ld;
    r.res_bits = a.res_bits; r.res_flag = a.res_flag;
    r.sh_gate = a.sh_gate_inp ? sh : nullptr;
    r.xq_qs = reinterpret_cast<int8_t *>(ws + p.xq_qs);
    r.xq_d = reinterpret_cast<float *>(ws + p.xq_d);
    r.xq_bs = reinterpret_cast<int32_t *>(ws + p.xq_bs);
    r.q80 = a.wtype == T_Q8_0;
    r.xq_d0 = reinterpret_cast<float *>(ws + p.xq_d0);
    r.xq_x = reinterpret_cast<uint32_t *>(ws + p.xq_x);
    r.units = reinterpret_cast<Unit *>(ws + p.units);
    r.n_units = reinterpret_cast<int32_t *>(ws + p.n_units);
    r.counter = reinterpret_cast<int32_t *>(ws + p.counters);
    r.shared = p.shared ? 1 : 0;
    r.slot_tables = a.slot_tables; r.table_stride = a.table_stride; r.layer = a.layer;
    r.slots_ws = reinterpret_cast<int32_t *>(ws + p.slots);
    r.uslot = reinterpret_cast<int32_t *>(ws + p.uslot);
    const int quant_wgs = (int)((a.T * (a.H / QK_K) + 3) / 4);
    const int grid = std::max((int)a.E + (a.sh_gate_inp ? 1 : 0), quant_wgs);
    const dim3 gd((unsigned)grid);
    if (a.E <= 128) QWM_TIMED("route", s, k_route<2><<<gd, dim3(256), 0, s>>>(r));
    else if (a.E <= 512) QWM_TIMED("route", s, k_route<8><<<gd, dim3(256), 0, s>>>(r));
    else QWM_TIMED("route", s, k_route<MAX_E / 64><<<gd, dim3(256), 0, s>>>(r));
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

template <int NB>
static void launch_gateup_x_nb(const GateUpArgs & g, int maxp, dim3 grid, hipStream_t s) {
    switch (maxp) {
        case 1: k_gateup_x<NB, 1><<<grid, 256, 0, s>>>(g); break;
        case 2: k_gateup_x<NB, 2><<<grid, 256, 0, s>>>(g); break;
        case 4: k_gateup_x<NB, 4><<<grid, 256, 0, s>>>(g); break;
        default: k_gateup_x<NB, 8><<<grid, 256, 0, s>>>(g); break;
    }
}
static bool launch_gateup_x(const GateUpArgs & g, int nb, int maxp, dim3 grid, hipStream_t s) {
    switch (nb) {
        case 1: launch_gateup_x_nb<1>(g, maxp, grid, s); return true;
        case 2: launch_gateup_x_nb<2>(g, maxp, grid, s); return true;
        case 3: launch_gateup_x_nb<3>(g, maxp, grid, s); return true;
        case 4: launch_gateup_x_nb<4>(g, maxp, grid, s); return true;
        case 5: launch_gateup_x_nb<5>(g, maxp, grid, s); return true;
        case 6: launch_gateup_x_nb<6>(g, maxp, grid, s); return true;
        case 7: launch_gateup_x_nb<7>(g, maxp, grid, s); return true;
        case 8: launch_gateup_x_nb<8>(g, maxp, grid, s); return true;
        case 12: launch_gateup_x_nb<12>(g, maxp, grid, s); return true;
        case 16: launch_gateup_x_nb<16>(g, maxp, grid, s); return true;
        default: return false;
    }
}
template <int NB>
static void launch_gateup_x5_nb(const GateUpArgs & g, int maxp, dim3 grid, hipStream_t s) {
    switch (maxp) {
        case 1: k_gateup_x5<NB, 1><<<grid, 256, 0, s>>>(g); break;
        case 2: k_gateup_x5<NB, 2><<<grid, 256, 0, s>>>(g); break;
        case 4: k_gateup_x5<NB, 4><<<grid, 256, 0, s>>>(g); break;
        default: k_gateup_x5<NB, 8><<<grid, 256, 0, s>>>(g); break;
    }
}
static bool launch_gateup_x5(const GateUpArgs & g, int nb, int maxp, dim3 grid, hipStream_t s) {
    switch (nb) {
        case 1: launch_gateup_x5_nb<1>(g, maxp, grid, s); return true;
        case 2: launch_gateup_x5_nb<2>(g, maxp, grid, s); return true;
        case 3: launch_gateup_x5_nb<3>(g, maxp, grid, s); return true;
        case 4: launch_gateup_x5_nb<4>(g, maxp, grid, s); return true;
        case 5: launch_gateup_x5_nb<5>(g, maxp, grid, s); return true;
        case 6: launch_gateup_x5_nb<6>(g, maxp, grid, s); return true;
        case 7: launch_gateup_x5_nb<7>(g, maxp, grid, s); return true;
        case 8: launch_gateup_x5_nb<8>(g, maxp, grid, s); return true;
        case 12: launch_gateup_x5_nb<12>(g, maxp, grid, s); return true;
        case 16: launch_gateup_x5_nb<16>(g, maxp, grid, s); return true;
        default: return false;
    }
}
template <int NPAIR>
static void launch_gateup_x80_np(const GateUpArgs & g, int maxp, dim3 grid, hipStream_t s) {
    switch (maxp) {
        case 1: k_gateup_x80<NPAIR, 1><<<grid, 256, 0, s>>>(g); break;
        case 2: k_gateup_x80<NPAIR, 2><<<grid, 256, 0, s>>>(g); break;
        case 4: k_gateup_x80<NPAIR, 4><<<grid, 256, 0, s>>>(g); break;
        default: k_gateup_x80<NPAIR, 8><<<grid, 256, 0, s>>>(g); break;
    }
}
static bool launch_gateup_x80(const GateUpArgs & g, int npair, int maxp, dim3 grid, hipStream_t s) {
    switch (npair) {
        case 4: launch_gateup_x80_np<4>(g, maxp, grid, s); return true;
        case 8: launch_gateup_x80_np<8>(g, maxp, grid, s); return true;
        case 12: launch_gateup_x80_np<12>(g, maxp, grid, s); return true;
        case 16: launch_gateup_x80_np<16>(g, maxp, grid, s); return true;
        case 20: launch_gateup_x80_np<20>(g, maxp, grid, s); return true;
        case 24: launch_gateup_x80_np<24>(g, maxp, grid, s); return true;
        case 28: launch_gateup_x80_np<28>(g, maxp, grid, s); return true;
        case 32: launch_gateup_x80_np<32>(g, maxp, grid, s); return true;
        case 48: launch_gateup_x80_np<48>(g, maxp, grid, s); return true;
        case 64: launch_gateup_x80_np<64>(g, maxp, grid, s); return true;
        default: return false;
    }
}
template <int NB>
static void launch_down_nb(const DownArgs & d, bool q80, int32_t dtype, int maxp, dim3 grid, hipStream_t s) {
    if (dtype == T_Q5_K) {
        switch (maxp) {
            case 1: k_down_q5k<NB, 1><<<grid, 256, 0, s>>>(d); break;
            case 2: k_down_q5k<NB, 2><<<grid, 256, 0, s>>>(d); break;
            case 4: k_down_q5k<NB, 4><<<grid, 256, 0, s>>>(d); break;
            default: k_down_q5k<NB, 8><<<grid, 256, 0, s>>>(d); break;
        }
        return;
    }
    if (dtype == T_Q6_K) {
        switch (maxp) {
            case 1: k_down_q6k<NB, 1><<<grid, 256, 0, s>>>(d); break;
            case 2: k_down_q6k<NB, 2><<<grid, 256, 0, s>>>(d); break;
            case 4: k_down_q6k<NB, 4><<<grid, 256, 0, s>>>(d); break;
            default: k_down_q6k<NB, 8><<<grid, 256, 0, s>>>(d); break;
        }
        return;
    }
    if (q80) {
        switch (maxp) {
            case 1: k_down_q80<NB, 1><<<grid, 256, 0, s>>>(d); break;
            case 2: k_down_q80<NB, 2><<<grid, 256, 0, s>>>(d); break;
            case 4: k_down_q80<NB, 4><<<grid, 256, 0, s>>>(d); break;
            default: k_down_q80<NB, 8><<<grid, 256, 0, s>>>(d); break;
        }
        return;
    }
    switch (maxp) {
        case 1: k_down_q4k<NB, 1><<<grid, 256, 0, s>>>(d); break;
        case 2: k_down_q4k<NB, 2><<<grid, 256, 0, s>>>(d); break;
        case 4: k_down_q4k<NB, 4><<<grid, 256, 0, s>>>(d); break;
        default: k_down_q4k<NB, 8><<<grid, 256, 0, s>>>(d); break;
    }
}

static int pow2_maxp(int64_t T) { return T <= 1 ? 1 : T <= 2 ? 2 : T <= 4 ? 4 : 8; }

int launch_experts(const ExpertArgs & a, const MoePlan & p, uint8_t * ws, hipStream_t s) {
    if (a.wtype != T_Q4_K && a.wtype != T_Q8_0 && a.wtype != T_Q5_K)
        return fail(QWM_ERR_UNSUPPORTED, "expert gate/up pools must be Q4_K, Q5_K or Q8_0");
    const bool q80 = a.wtype == T_Q8_0;
    if (a.down_type != a.wtype && !(a.down_type == T_Q6_K && (a.wtype == T_Q4_K || a.wtype == T_Q5_K)))
        return fail(QWM_ERR_UNSUPPORTED, "down pools: the gate/up type, or Q6_K beside Q4_K / Q5_K");
    const int maxp = pow2_maxp(p.T);
    const int P = (int)(p.T * p.k);
    const int unit_slots = P;
    const int grid_y = unit_slots + (p.shared ? 1 : 0);
    Unit * units = reinterpret_cast<Unit *>(ws + p.units);
    const int32_t * n_units = reinterpret_cast<const int32_t *>(ws + p.n_units);

    GateUpArgs g;
    g.gate = a.gate; g.up = a.up; g.gate_slab = a.gate_slab; g.up_slab = a.up_slab;
    g.sh_gate = a.sh_gate; g.sh_up = a.sh_up;
    g.slot_g = a.slot_g; g.slot_u = a.slot_u; g.uslot = a.uslot;
    g.S_g = a.n_slots_g; g.S_u = a.n_slots_u;
    g.units = units; g.n_units = n_units; g.unit_slots = unit_slots;
    g.xq_qs = reinterpret_cast<const int8_t *>(ws + p.xq_qs);
    g.xq_d = reinterpret_cast<const float *>(ws + (q80 ? p.xq_d0 : p.xq_d));
    g.xq_bs = reinterpret_cast<const int32_t *>(ws + p.xq_bs);
    g.xq_x = reinterpret_cast<const uint32_t *>(ws + p.xq_x);
    g.act = reinterpret_cast<float *>(ws + p.act);
    g.act_sh = reinterpret_cast<float *>(ws + p.act_sh);
    g.H = (int)p.H; g.N = (int)p.N; g.N_sh = (int)p.N_sh; g.k = (int)p.k; g.T = (int)p.T;
    const int rows_g = (int)std::max(p.N, p.N_sh);
    prof_begin("gate_up", s);
    const dim3 grid_x((rows_g + GUX_ROWS - 1) / GUX_ROWS, grid_y);
    if (q80 ? !launch_gateup_x80(g, (int)(p.H / 64), maxp, grid_x, s)
            : a.wtype == T_Q5_K ? !launch_gateup_x5(g, (int)(p.H / QK_K), maxp, grid_x, s)
                                : !launch_gateup_x(g, (int)(p.H / QK_K), maxp, grid_x, s))
        return fail(QWM_ERR_UNSUPPORTED, "hidden size not instantiated for the exact gate/up");
    prof_end("gate_up", s);

    DownArgs d;
    d.down = a.down; d.down_slab = a.down_slab; d.sh_down = a.sh_down;
    d.slot_d = a.slot_d; d.uslot = a.uslot; d.S_d = a.n_slots_d;
    d.units = units; d.n_units = n_units; d.unit_slots = unit_slots;
    d.act = g.act; d.act_sh = g.act_sh;
    d.ex = reinterpret_cast<float *>(ws + p.ex);
    d.ex_sh = reinterpret_cast<float *>(ws + p.ex_sh);
    d.H = (int)p.H; d.N = (int)p.N; d.N_sh = (int)p.N_sh; d.k = (int)p.k; d.T = (int)p.T;
    d.shared = p.shared ? 1 : 0;
    d.tile_counters = reinterpret_cast<int32_t *>(ws + p.tile_counters);
    d.w = reinterpret_cast<const float *>(a.weights);
    d.sh_gate = p.shared_gate ? reinterpret_cast<const float *>(ws + p.sh_gate) : nullptr;
    d.resid = a.resid; d.out = a.out;
    const int nb_d = (int)(p.N / QK_K);           // moe_plan: 1..8, shared width equal
    const int tile_d = 32;                        // k_down_q4k: 4 waves x 8 rows
    dim3 grid_d(((int)p.H + tile_d - 1) / tile_d, grid_y);
    if (grid_d.x > (unsigned)MAX_TILES) return fail(QWM_ERR_UNSUPPORTED, "hidden size needs too many down tiles");
    prof_begin("down", s);
    switch (nb_d) {
        case 1: launch_down_nb<1>(d, q80, a.down_type, maxp, grid_d, s); break;
        case 2: launch_down_nb<2>(d, q80, a.down_type, maxp, grid_d, s); break;
        case 3: launch_down_nb<3>(d, q80, a.down_type, maxp, grid_d, s); break;
        case 4: launch_down_nb<4>(d, q80, a.down_type, maxp, grid_d, s); break;
        case 5: launch_down_nb<5>(d, q80, a.down_type, maxp, grid_d, s); break;
        case 6: launch_down_nb<6>(d, q80, a.down_type, maxp, grid_d, s); break;
        case 7: launch_down_nb<7>(d, q80, a.down_type, maxp, grid_d, s); break;
        default: launch_down_nb<8>(d, q80, a.down_type, maxp, grid_d, s); break;
    }
    prof_end("down", s);

    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

// ======================================================================
// generic GGML_OP_MUL_MAT_ID (Q4_K): prep quantizes b and builds units
// ======================================================================
struct MmidPrep {
    const float * b; size_t b_nb1, b_nb2;   // bytes
    const int32_t * ids; size_t ids_nb1;    // bytes
    int K, ne11, T, n_ids, n_as, cap;       // cap: pairs per unit
    int q80;                                // Q8_0 weights: b as Q8_0 (d per 32) instead of Q8_K
    int8_t * qs; float * d; int32_t * bs;   // [T*ne11] rows of Q8_0 (Q8_0 weights)
    uint32_t * xq;                          // [T*ne11][K/256][XS] rows of Q8_K, exact-dot layout (Q4_K weights)
    Unit * units; int32_t * n_units; int32_t * ids_ws; int32_t * err;
};

// Blocks quantize b's columns; block 0's first wave then groups the (t, e)
// pairs by expert in pair order, at most `cap` pairs per unit.
__global__ void __launch_bounds__(256) k_mmid_prep(MmidPrep a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rows = a.T * a.ne11, nb = a.K / QK_K;
    for (int jb = blockIdx.x * 4 + wave; jb < rows * nb; jb += gridDim.x * 4) {
        const int row = jb / nb, b = jb % nb;
        const int t = row / a.ne11, i = row % a.ne11;
        const float * src = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(a.b) + t * a.b_nb2 + i * a.b_nb1);
        if (a.q80)
            quantize_q80_256(src + b * QK_K, a.qs + (size_t)row * a.K + b * QK_K, a.d + (size_t)row * (a.K / 32) + b * 8, lane);
        else
            quantize_block_q8K_x(src + b * QK_K, a.xq + (size_t)(row * nb + b) * XS, lane);
    }
    if (blockIdx.x != 0 || wave != 0) return;
    const int P = a.T * a.n_ids;
    __shared__ int32_t eid[MAX_PAIRS], rank[MAX_PAIRS], uidx[MAX_PAIRS];
    int bad = 0;
    for (int p = lane; p < P; p += 64) {
        const int t = p / a.n_ids, e = p % a.n_ids;
        int v = *reinterpret_cast<const int32_t *>(reinterpret_cast<const uint8_t *>(a.ids) + t * a.ids_nb1 + e * 4);
        if (v < 0 || v >= a.n_as) { bad = 1; v = 0; }
        eid[p] = v;
        a.ids_ws[p] = v;
    }
    if (__any(bad) && lane == 0) *a.err = 1;
    __syncthreads();
    for (int p = lane; p < P; p += 64) {
        int r = 0;
        for (int q = 0; q < p; ++q) r += eid[q] == eid[p];
        rank[p] = r;
    }
    __syncthreads();
    int base = 0;
    for (int c = 0; c < P; c += 64) {
        const int p = c + lane;
        const bool isf = p < P && rank[p] % a.cap == 0;
        const unsigned long long bal = __ballot(isf);
        if (isf) uidx[p] = base + __popcll(bal & ((1ull << lane) - 1ull));
        base += __popcll(bal);
    }
    __syncthreads();
    for (int p = lane; p < P; p += 64) {
        const int r0 = rank[p] - rank[p] % a.cap;   // rank of the unit's first pair
        int f = p;
        for (int q = 0; q <= p; ++q)
            if (eid[q] == eid[p] && rank[q] == r0) { f = q; break; }
        int total = 0;
        for (int q = 0; q < P; ++q) total += eid[q] == eid[p];
        Unit & u = a.units[uidx[f]];
        u.pair[rank[p] - r0] = p;
        if (p == f) { u.expert = eid[p]; u.n = min(a.cap, total - r0); }
    }
    if (lane == 0) *a.n_units = base;
}

struct MmidGemv {
    const uint8_t * as; size_t slab; size_t row_bytes;
    const Unit * units; const int32_t * n_units;
    const int8_t * qs; const float * d; const int32_t * bs;
    const uint32_t * xq;
    int K, N, ne11, n_ids;
    float * dst; size_t dst_nb1, dst_nb2;
};

// Q4_K MUL_MAT_ID columns in ggml-CPU's exact float order (qwm_exact.h): a
// workgroup owns 32 rows (4 waves x 8 rows, 8 lanes per row) of one unit;
// the unit's Q8_K columns are copied into LDS first.
template <int NB, int MAXP>
__global__ void __launch_bounds__(256) k_mmid_x(MmidGemv a) {
    __shared__ __align__(16) uint32_t s_x[MAXP * NB * XS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m = lane & 7, rsub = lane >> 3;
    const int u = blockIdx.y;
    const int nu = *a.n_units;
    const Unit U = a.units[u];
    if (u >= nu) return;
    const int n = U.n;
    const uint8_t * base = a.as + (size_t)U.expert * a.slab;
    const int r = blockIdx.x * 32 + wave * 8 + rsub;
    const int rc = min(r, a.N - 1);
    // rows of up to 8 blocks requested whole before the column copy, longer
    // rows in double-buffered chunks of 8 (or 6) blocks after it
    constexpr int NBR = NB <= 8 ? NB : 1;
    XBlk W[NBR];
    if constexpr (NB <= 8) {
#pragma unroll
        for (int b = 0; b < NB; ++b) load_xblk(W[b], base + (size_t)rc * a.row_bytes + b * 144, m);
    }
    constexpr int Q4 = NB * XS / 4;
    for (int q = tid; q < n * Q4; q += 256) {
        const int i = q / Q4, o = q % Q4;
        int p = U.pair[0];
#pragma unroll
        for (int qq = 1; qq < MAXP; ++qq) if (i == qq) p = U.pair[qq];
        const int row = (p / a.n_ids) * a.ne11 + (p % a.n_ids) % a.ne11;
        reinterpret_cast<uint4 *>(s_x)[q] = reinterpret_cast<const uint4 *>(a.xq + (size_t)row * NB * XS)[o];
    }
    __syncthreads();
    float acc[MAXP];
    if constexpr (NB <= 8) {
        q4k_dot8<NB, MAXP>(acc, W, s_x, n, m);
    } else {
        const uint8_t * const rw[1] = {base + (size_t)rc * a.row_bytes};
        float o1[1][MAXP];
        q4k_dot8_chunked<NB, (NB % 8 == 0 ? 8 : 6), 1, MAXP>(o1, rw, s_x, n, m);
#pragma unroll
        for (int i = 0; i < MAXP; ++i) acc[i] = o1[0][i];
    }
    if (m == 0 && r < a.N) {
#pragma unroll
        for (int i = 0; i < MAXP; ++i)
            if (i < n) {
                const int p = U.pair[i];
                float * o = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(a.dst) + (p / a.n_ids) * a.dst_nb2 +
                                                      (p % a.n_ids) * a.dst_nb1);
                o[r] = acc[i];
            }
    }
}

// k_mmid_x for Q6_K weights: the same columns in LDS, rows through q6k_dot8.
template <int NB, int MAXP>
__global__ void __launch_bounds__(256) k_mmid_x6(MmidGemv a) {
    __shared__ __align__(16) uint32_t s_x[MAXP * NB * XS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m = lane & 7, rsub = lane >> 3;
    const int u = blockIdx.y;
    const int nu = *a.n_units;
    const Unit U = a.units[u];
    if (u >= nu) return;
    const int n = U.n;
    const uint8_t * base = a.as + (size_t)U.expert * a.slab;
    const int r = blockIdx.x * 32 + wave * 8 + rsub;
    const int rc = min(r, a.N - 1);
    constexpr int Q4 = NB * XS / 4;
    for (int q = tid; q < n * Q4; q += 256) {
        const int i = q / Q4, o = q % Q4;
        int p = U.pair[0];
#pragma unroll
        for (int qq = 1; qq < MAXP; ++qq) if (i == qq) p = U.pair[qq];
        const int row = (p / a.n_ids) * a.ne11 + (p % a.n_ids) % a.ne11;
        reinterpret_cast<uint4 *>(s_x)[q] = reinterpret_cast<const uint4 *>(a.xq + (size_t)row * NB * XS)[o];
    }
    __syncthreads();
    float acc[MAXP];
    q6k_dot8<NB, MAXP>(acc, base + (size_t)rc * a.row_bytes, s_x, n, m);
    if (m == 0 && r < a.N) {
#pragma unroll
        for (int i = 0; i < MAXP; ++i)
            if (i < n) {
                const int p = U.pair[i];
                float * o = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(a.dst) + (p / a.n_ids) * a.dst_nb2 +
                                                      (p % a.n_ids) * a.dst_nb1);
                o[r] = acc[i];
            }
    }
}

// k_mmid_x for Q5_K weights: rows through q5k_dot8.
template <int NB, int MAXP>
__global__ void __launch_bounds__(256) k_mmid_x5(MmidGemv a) {
    __shared__ __align__(16) uint32_t s_x[MAXP * NB * XS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m = lane & 7, rsub = lane >> 3;
    const int u = blockIdx.y;
    const int nu = *a.n_units;
    const Unit U = a.units[u];
    if (u >= nu) return;
    const int n = U.n;
    const uint8_t * base = a.as + (size_t)U.expert * a.slab;
    const int r = blockIdx.x * 32 + wave * 8 + rsub;
    const int rc = min(r, a.N - 1);
    constexpr int Q4 = NB * XS / 4;
    for (int q = tid; q < n * Q4; q += 256) {
        const int i = q / Q4, o = q % Q4;
        int p = U.pair[0];
#pragma unroll
        for (int qq = 1; qq < MAXP; ++qq) if (i == qq) p = U.pair[qq];
        const int row = (p / a.n_ids) * a.ne11 + (p % a.n_ids) % a.ne11;
        reinterpret_cast<uint4 *>(s_x)[q] = reinterpret_cast<const uint4 *>(a.xq + (size_t)row * NB * XS)[o];
    }
    __syncthreads();
    float acc[MAXP];
    q5k_dot8<NB, MAXP>(acc, base + (size_t)rc * a.row_bytes, s_x, n, m);
    if (m == 0 && r < a.N) {
#pragma unroll
        for (int i = 0; i < MAXP; ++i)
            if (i < n) {
                const int p = U.pair[i];
                float * o = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(a.dst) + (p / a.n_ids) * a.dst_nb2 +
                                                      (p % a.n_ids) * a.dst_nb1);
                o[r] = acc[i];
            }
    }
}

// The Q8_0 form of k_mmid_x: ggml's Q8_0 dot order, the unit's Q8_0 columns in LDS.
template <int NPAIR, int MAXP>
__global__ void __launch_bounds__(256) k_mmid_x80(MmidGemv a) {
    constexpr int K = NPAIR * 64;
    __shared__ __align__(16) uint32_t s_q[MAXP * K / 4];
    __shared__ float s_d[MAXP * K / 32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m = lane & 7, rsub = lane >> 3;
    const int u = blockIdx.y;
    const int nu = *a.n_units;
    const Unit U = a.units[u];
    if (u >= nu) return;
    const int n = U.n;
    const uint8_t * base = a.as + (size_t)U.expert * a.slab;
    const int r = blockIdx.x * 32 + wave * 8 + rsub;
    const int rc = min(r, a.N - 1);
    for (int q = tid; q < n * (K / 16); q += 256) {
        const int i = q / (K / 16), o = q % (K / 16);
        int p = U.pair[0];
#pragma unroll
        for (int qq = 1; qq < MAXP; ++qq) if (i == qq) p = U.pair[qq];
        const int row = (p / a.n_ids) * a.ne11 + (p % a.n_ids) % a.ne11;
        reinterpret_cast<uint4 *>(s_q)[i * (K / 16) + o] = reinterpret_cast<const uint4 *>(a.qs + (size_t)row * K)[o];
        if (o < K / 32) s_d[i * (K / 32) + o] = a.d[(size_t)row * (K / 32) + o];
    }
    __syncthreads();
    float acc[MAXP];
    q80_dot8<NPAIR, MAXP>(acc, base + (size_t)rc * a.row_bytes, s_q, s_d, K / 4, K / 32, n, m);
    if (m == 0 && r < a.N) {
#pragma unroll
        for (int i = 0; i < MAXP; ++i)
            if (i < n) {
                const int p = U.pair[i];
                float * o = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(a.dst) + (p / a.n_ids) * a.dst_nb2 +
                                                      (p % a.n_ids) * a.dst_nb1);
                o[r] = acc[i];
            }
    }
}

size_t mmid_workspace(int64_t K, int64_t T, int64_t ne11, int64_t n_ids) {
    const int64_t rows = T * ne11;
    size_t o = 0;
    auto take = [&](size_t bytes) { o = align_up(o + bytes, 256); };
    take((size_t)rows * K);                       // qs
    take(sizeof(float) * rows * (K / 32));        // d (Q8_K: K / 256 used)
    take(sizeof(int32_t) * rows * (K / 16));      // bsums
    take(sizeof(Unit) * T * n_ids);               // units
    take(sizeof(int32_t) * 4);                    // n_units, err
    take(sizeof(int32_t) * T * n_ids);            // ids copy
    take(sizeof(uint32_t) * rows * (K / QK_K) * XS);   // Q8_K columns, exact-dot layout
    return o;
}

int launch_mmid(const MmidArgs & a, uint8_t * ws, hipStream_t s) {
    if (a.wtype != T_Q4_K && a.wtype != T_Q8_0 && a.wtype != T_Q6_K && a.wtype != T_Q5_K)
        return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: weights must be Q4_K, Q5_K, Q6_K or Q8_0");
    const bool q80 = a.wtype == T_Q8_0;
    const int64_t rows = a.T * a.ne11;
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    const size_t o_qs = take((size_t)rows * a.K), o_d = take(sizeof(float) * rows * (a.K / 32)),
                 o_bs = take(sizeof(int32_t) * rows * (a.K / 16)), o_u = take(sizeof(Unit) * a.T * a.n_ids),
                 o_n = take(sizeof(int32_t) * 4), o_ids = take(sizeof(int32_t) * a.T * a.n_ids),
                 o_x = take(sizeof(uint32_t) * rows * (a.K / QK_K) * XS);
    MmidPrep pr;
    pr.b = a.b; pr.b_nb1 = a.b_nb1; pr.b_nb2 = a.b_nb2; pr.ids = a.ids; pr.ids_nb1 = a.ids_nb1;
    const int maxp = pow2_maxp(a.T);
    pr.K = (int)a.K; pr.ne11 = (int)a.ne11; pr.T = (int)a.T; pr.n_ids = (int)a.n_ids; pr.n_as = (int)a.n_as;
    pr.cap = maxp;
    pr.q80 = q80 ? 1 : 0;
    pr.qs = reinterpret_cast<int8_t *>(ws + o_qs); pr.d = reinterpret_cast<float *>(ws + o_d);
    pr.bs = reinterpret_cast<int32_t *>(ws + o_bs); pr.units = reinterpret_cast<Unit *>(ws + o_u);
    pr.n_units = reinterpret_cast<int32_t *>(ws + o_n); pr.err = pr.n_units + 1;
    pr.ids_ws = reinterpret_cast<int32_t *>(ws + o_ids);
    pr.xq = reinterpret_cast<uint32_t *>(ws + o_x);
    const int nblk = (int)(rows * (a.K / QK_K));
    QWM_TIMED("mul_mat_id_prep", s, k_mmid_prep<<<dim3((unsigned)std::max(1, std::min(256, (nblk + 3) / 4))), 256, 0, s>>>(pr));
    MmidGemv g;
    g.as = a.as; g.slab = a.slab;
    g.row_bytes = q80 ? (size_t)(a.K / 32) * 34
                      : (size_t)(a.K / QK_K) * (a.wtype == T_Q6_K ? 210 : a.wtype == T_Q5_K ? 176 : 144);
    g.units = pr.units; g.n_units = pr.n_units; g.qs = pr.qs; g.d = pr.d; g.bs = pr.bs; g.xq = pr.xq;
    g.K = (int)a.K; g.N = (int)a.N; g.ne11 = (int)a.ne11; g.n_ids = (int)a.n_ids;
    g.dst = a.dst; g.dst_nb1 = a.dst_nb1; g.dst_nb2 = a.dst_nb2;
    if (!hidden_supported(a.K)) return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: K must be 256 .. 2048, 3072 or 4096");
    if (!q80) {
        const dim3 gx((unsigned)((a.N + 31) / 32), (unsigned)(a.T * a.n_ids));
#define QWM_MMIDX(NB_)                                                              \
        case NB_:                                                                   \
            if (a.wtype == T_Q6_K)                                                  \
                switch (maxp) {                                                     \
                    case 1: k_mmid_x6<NB_, 1><<<gx, 256, 0, s>>>(g); break;         \
                    case 2: k_mmid_x6<NB_, 2><<<gx, 256, 0, s>>>(g); break;         \
                    case 4: k_mmid_x6<NB_, 4><<<gx, 256, 0, s>>>(g); break;         \
                    default: k_mmid_x6<NB_, 8><<<gx, 256, 0, s>>>(g); break;        \
                }                                                                   \
            else if (a.wtype == T_Q5_K)                                             \
                switch (maxp) {                                                     \
                    case 1: k_mmid_x5<NB_, 1><<<gx, 256, 0, s>>>(g); break;         \
                    case 2: k_mmid_x5<NB_, 2><<<gx, 256, 0, s>>>(g); break;         \
                    case 4: k_mmid_x5<NB_, 4><<<gx, 256, 0, s>>>(g); break;         \
                    default: k_mmid_x5<NB_, 8><<<gx, 256, 0, s>>>(g); break;        \
                }                                                                   \
            else                                                                    \
                switch (maxp) {                                                     \
                    case 1: k_mmid_x<NB_, 1><<<gx, 256, 0, s>>>(g); break;          \
                    case 2: k_mmid_x<NB_, 2><<<gx, 256, 0, s>>>(g); break;          \
                    case 4: k_mmid_x<NB_, 4><<<gx, 256, 0, s>>>(g); break;          \
                    default: k_mmid_x<NB_, 8><<<gx, 256, 0, s>>>(g); break;         \
                }                                                                   \
            break;
        prof_begin("mul_mat_id", s);
        switch (a.K / QK_K) {
            QWM_MMIDX(1) QWM_MMIDX(2) QWM_MMIDX(3) QWM_MMIDX(4)
            QWM_MMIDX(5) QWM_MMIDX(6) QWM_MMIDX(7) QWM_MMIDX(8) QWM_MMIDX(12) QWM_MMIDX(16)
            default: return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: K must be 256 .. 2048, 3072 or 4096");
        }
        prof_end("mul_mat_id", s);
#undef QWM_MMIDX
        QWM_HIP_CHECK(hipGetLastError());
        return QWM_OK;
    }
    const dim3 gx((unsigned)((a.N + 31) / 32), (unsigned)(a.T * a.n_ids));
#define QWM_MMIDX80(NP_)                                                            \
    case NP_:                                                                       \
        switch (maxp) {                                                             \
            case 1: k_mmid_x80<NP_, 1><<<gx, 256, 0, s>>>(g); break;                \
            case 2: k_mmid_x80<NP_, 2><<<gx, 256, 0, s>>>(g); break;                \
            case 4: k_mmid_x80<NP_, 4><<<gx, 256, 0, s>>>(g); break;                \
            default: k_mmid_x80<NP_, 8><<<gx, 256, 0, s>>>(g); break;               \
        }                                                                           \
        break;
    prof_begin("mul_mat_id", s);
    switch (a.K / 64) {                       // pairs of Q8_0 blocks per row
        QWM_MMIDX80(4) QWM_MMIDX80(8) QWM_MMIDX80(12) QWM_MMIDX80(16)
        QWM_MMIDX80(20) QWM_MMIDX80(24) QWM_MMIDX80(28) QWM_MMIDX80(32) QWM_MMIDX80(48) QWM_MMIDX80(64)
        default: return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: K must be 256 .. 2048, 3072 or 4096");
    }
    prof_end("mul_mat_id", s);
#undef QWM_MMIDX80
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

__global__ void k_fill_zero(uint32_t * p, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

int launch_fill_zero(void * p, size_t bytes, hipStream_t s) {
    if (bytes % 4) return fail(QWM_ERR_ARG, "workspace size must be a multiple of 4");
    const size_t n = bytes / 4;
    if (n == 0) return QWM_OK;
    const unsigned blocks = (unsigned)std::min<size_t>(1024, (n + 255) / 256);
    k_fill_zero<<<blocks, 256, 0, s>>>(reinterpret_cast<uint32_t *>(p), n);
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

}  // namespace qwm
