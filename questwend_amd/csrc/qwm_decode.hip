// qwm_decode.hip -- the decode loop over stacked MoE layers (x = x + MoE_l(x),
// the per-layer segment B of decode_cached with every expert resident,
// core/runtime.cpp:5064-5888, MoE blocks only) as one persistent launch per
// group of up to DEC_LAYERS layers, on the fused step's phases
// (qwm_step_kernel.h): per layer
//
//   P0  router rows: their workgroups request the layer's router row first
//       and then wait until every down tile of the previous layer is
//       combined (its output is this layer's x)                 -> count
//   P1  every workgroup selects (softmax or sigmoid, top-k, weights, union,
//       slots) in wave 0 while waves 1..3 quantize x to Q8_K in its LDS
//   P2  gate/up + SwiGLU items                                    -> per unit
//   P3  down items; the last unit of a row tile combines it into the next
//       layer's x (+ the residual)                                -> tiles
//
// with no launch boundary between layers: a workgroup goes on to the next
// layer as soon as its own items are done, and only the router rows wait
// for the whole previous layer.  Every layer of a launch has its own logits,
// x, expert outputs, router count and unit counts in the workspace, so a workgroup that is behind (one with no items in a layer)
// never finds a buffer that a later layer already rewrote; the SwiGLU
// activations, shared by the layers, are read with agent-scope loads, and
// each layer's down items finish before the next layer's gate/up can start.
// The caller's x is read by the launch's first layer and written by its last
// (in place when the launch holds one layer: each combine thread reads its
// residual element before it writes it, and every other read of x precedes
// the router count).  The last workgroup to finish re-arms the counters.
#include <cstring>

#include "qwm_step_kernel.h"

namespace qwm {

constexpr int DEC_LAYERS = 16;              // layers per launch (their descriptors travel as kernel arguments)
constexpr int DEC_UNIT_LINES = MAX_PAIRS + 1;

struct DecodeLayer {
    const float * W_r; const float * sgi; const float * bias;
    const uint8_t * gate; const uint8_t * up; const uint8_t * down;
    const uint8_t * sh_gate; const uint8_t * sh_up; const uint8_t * sh_down;
    uint32_t gu_slab, down_slab;
    int32_t n_slots[3];
    int32_t norm, sigm, d6;
    float scale;
};

struct DecodeArgs {
    StepArgs base[1];                   // shapes, the shared buffers, slot tables, counters, spin bound
    DecodeLayer L[DEC_LAYERS];
    int n_layers, first;                // global index of the launch's first layer
    float * x;                          // the caller's x [T][H]
    float * lg; uint32_t lg_stride;     // per layer: logits [E + 1][32]
    float * xs; uint32_t x_stride;      // x of the launch's layers 1.. (layer j reads xs + (j - 1) * x_stride)
    float * ex; uint32_t ex_stride;     // per layer: expert outputs [T * k][H]
    float * ex_sh; uint32_t exs_stride; // per layer: shared expert outputs [T][H]
    int32_t * rows_done;                // per layer: one 32-word line
    int32_t * gu_done;                  // per layer: DEC_UNIT_LINES lines of 32 words
    int32_t * done;                     // launch completion ticket
    int32_t * ids_all;                  // [layer][T][k] by global layer, or null
    const uint32_t * res_bits; int32_t res_words; int32_t * res_flag;
};
static_assert(sizeof(DecodeArgs) <= 3072, "the decode launch's arguments stay well inside the kernarg segment");

// P0 of layer j (one token): the router rows (ggml_vec_dot_f32's AVX-512
// order, as step_router), after the previous layer's tiles are all
// combined; the row's weights are requested before that wait.  The count's
// parts are the router workgroups (dec_p0_parts).  The Q8_K of x is not part
// of P0: every workgroup quantizes x into its own LDS during the selection.
QWM_DEV int dec_p0_parts(const StepArgs & a, int G) {
    const int rows = a.E + (a.sgi ? 1 : 0);
    return rows < G ? rows : G;
}
QWM_DEV void dec_router(const StepArgs & a, int g, int G, int32_t tiles_before) {
    constexpr int NT = 1;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E;
    const int rows = E + (a.sgi ? 1 : 0);
    if (g >= rows) return;                        // uniform per workgroup
    float wv[SH / 64];
    {
        const float * w = g == E ? a.sgi : a.W_r + (size_t)g * SH;
#pragma unroll
        for (int s = 0; s < SH / 64; ++s) wv[s] = w[64 * s + lane];
    }
    if (tiles_before > 0) wait_count(a.tiles_done, tiles_before, a.err, a.spin);
    for (int e = g; e < rows; e += G) {
        if (e != g) {
            const float * w = e == E ? a.sgi : a.W_r + (size_t)e * SH;
#pragma unroll
            for (int s = 0; s < SH / 64; ++s) wv[s] = w[64 * s + lane];
        }
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
            if (lane == 0) st_agent(a.lg + (size_t)e * 32 + t, acc);
        }
    }
    signal_count(a.rows_done);
}

template <int NT, int NB_D>
__global__ void __launch_bounds__(256, 2) k_decode(DecodeArgs d) {
    static_assert(NT == 1, "dec_router computes one token");
    constexpr int MAXP = NT <= 1 ? 1 : NT <= 2 ? 2 : NT <= 4 ? 4 : 8;
    constexpr size_t down_bytes = (size_t)MAXP * (NB_D * XS * 4 + DN_TR * 4);
    constexpr size_t smem_bytes = cmax(STEP_SELECT_LDS, down_bytes);
    constexpr int ntiles = SH / DN_TR;
    __shared__ __align__(16) uint8_t smem[smem_bytes];
    __shared__ __align__(16) uint32_t s_xq[NT * SNB * XS];
    __shared__ StepShared S;
    const int g = blockIdx.x, G = gridDim.x;
    for (int j = 0; j < d.n_layers; ++j) {
        // the arguments shared by the layers are read through an index the
        // compiler cannot see is 0, so their loads stay inside the layer's
        // iteration instead of living (in registers) across the whole loop
        int z;
        asm volatile("s_mov_b32 %0, 0" : "=s"(z));
        const DecodeLayer & Lj = d.L[j];
        StepArgs a = d.base[z];
        a.W_r = Lj.W_r; a.sgi = Lj.sgi; a.bias = Lj.bias;
        a.norm = Lj.norm; a.sigm = Lj.sigm; a.scale = Lj.scale;
        a.gate = Lj.gate; a.up = Lj.up; a.down = Lj.down;
        a.gate_slab = a.up_slab = Lj.gu_slab; a.down_slab = Lj.down_slab;
        a.n_slots[0] = Lj.n_slots[0]; a.n_slots[1] = Lj.n_slots[1]; a.n_slots[2] = Lj.n_slots[2];
        a.sh_gate = Lj.sh_gate; a.sh_up = Lj.sh_up; a.sh_down = Lj.sh_down;
        a.d6 = Lj.d6;
        a.layer = d.first + j;
        a.x = j == 0 ? d.x : d.xs + (size_t)(j - 1) * d.x_stride;
        a.resid = a.x;
        a.out = j == d.n_layers - 1 ? d.x : d.xs + (size_t)j * d.x_stride;
        a.lg = d.lg + (size_t)j * d.lg_stride;
        a.xq_x = nullptr;                 // x is quantized into LDS
        a.ex = d.ex + (size_t)j * d.ex_stride;
        a.ex_sh = d.ex_sh + (size_t)j * d.exs_stride;
        a.rows_done = d.rows_done + 32 * j;
        a.gu_done = d.gu_done + (size_t)32 * DEC_UNIT_LINES * j;
        a.ids_out = d.ids_all ? d.ids_all + (size_t)(d.first + j) * NT * a.k : nullptr;
        a.ids_ld = a.k;
        a.w_out = nullptr;

        // the layer's slot tables, requested first (as k_step)
        constexpr int SLQ = 3 * STEP_MAX_E / 256;
        int32_t sl[SLQ];
#pragma unroll
        for (int q = 0; q < SLQ; ++q) {
            const int idx = threadIdx.x + 256 * q;
            sl[q] = idx < 3 * a.E ? a.slot_tables[(size_t)(idx / a.E) * a.table_stride + (size_t)a.layer * a.E + idx % a.E] : 0;
        }
        dec_router(a, g, G, ntiles * j);
#pragma unroll
        for (int q = 0; q < SLQ; ++q) S.slot_of[threadIdx.x + 256 * q] = sl[q];
        wait_count(a.rows_done, dec_p0_parts(a, G), a.err, a.spin);
        // the router count implies the previous layer's tiles (this x) are
        // all in: waves 1..3 quantize x to Q8_K into LDS while wave 0 selects
        if (threadIdx.x >= 64)
            for (int b = (int)(threadIdx.x >> 6) - 1; b < SNB; b += 3)
                quantize_block_q8K_x(a.x + (size_t)b * QK_K, s_xq + b * XS, threadIdx.x & 63);
        if (a.E <= 128) step_select<NT, 2>(a, g, S, smem);
        else step_select<NT, STEP_MAX_E / 64>(a, g, S, smem);
        // the optimistic path's residency check (runtime.cpp:6155-6166)
        if (g == 0 && d.res_bits && (int)threadIdx.x < NT * a.k) {
            const uint32_t * bits = d.res_bits + (size_t)(d.first + j) * d.res_words;
            const int e = S.ids[threadIdx.x];
            if (!((bits[e >> 5] >> (e & 31)) & 1u)) __hip_atomic_fetch_or(d.res_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        step_gateup<MAXP>(a, g, G, S, s_xq);
        step_down<NT, NB_D, MAXP>(a, g, G, S, smem);
        __syncthreads();
    }
    if (last_workgroup(d.done, G)) {
        // every workgroup has passed all its waits: re-arm the counters and
        // the tile tickets (see k_step: after a wait gave up, workgroups may
        // disagree on a layer's unit count)
        for (int q = threadIdx.x; q < d.n_layers * DEC_UNIT_LINES; q += 256) st_agent(d.gu_done + 32 * q, 0);
        if (threadIdx.x < ntiles) st_agent(d.base[0].tile_counters + threadIdx.x, 0);
        for (int q = threadIdx.x; q < d.n_layers; q += 256) st_agent(d.rows_done + 32 * q, 0);
        if (threadIdx.x == 0) st_agent(d.base[0].tiles_done, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0 && ld_agent(d.base[0].err)) {
            if (d.res_flag) __hip_atomic_fetch_or(d.res_flag, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            st_agent(d.base[0].err, 0);
        }
    }
}

// ======================================================================
// host side
// ======================================================================

template <int NT, int NB_D>
static int decode_grid() {
    static int grid = 0;
    if (!grid) {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return -1;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(k_decode<NT, NB_D>), 256, 0) != hipSuccess)
            return -1;
        grid = std::min(std::min(per_cu, 2) * cus, MAX_STEP_WG);
    }
    return grid;
}

bool decode_plan(const qwm_moe_layer * layers, int32_t n_layers, int64_t T, DecodePlan & p, std::string & why) {
    if (T != 1) { why = "the persistent decode runs one token"; return false; }
    if (!moe_plan(&layers[0], T, p.moe, why)) return false;
    const MoePlan & m = p.moe;
    if (m.H != SH) { why = "the persistent decode is built for hidden size 2048"; return false; }
    if (m.N != 512 && m.N != 768 && m.N != 1024 && m.N != 2048) { why = "FFN width not instantiated"; return false; }
    if (m.shared && m.N_sh != m.N) { why = "the shared expert's FFN width differs from the routed one"; return false; }
    if (m.E > STEP_MAX_E) { why = "more than 512 experts"; return false; }
    for (int32_t l = 0; l < n_layers; ++l) {
        const qwm_moe_layer & L = layers[l];
        if (L.gate_pool.type != T_Q4_K || (L.down_pool.type != T_Q4_K && L.down_pool.type != T_Q6_K)) {
            why = "the persistent decode needs Q4_K gate/up pools and Q4_K or Q6_K down pools";
            return false;
        }
        if (L.gate_pool.nb[2] > UINT32_MAX || L.down_pool.nb[2] > UINT32_MAX) { why = "slab too large"; return false; }
    }
    const int nl = std::min<int32_t>(n_layers, DEC_LAYERS);
    const size_t E1 = (size_t)m.E + 1;
    size_t o = align_up(m.total, 256);
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    p.lg_stride = (uint32_t)(align_up(sizeof(float) * 32 * E1, 256) / 4);
    p.x_stride = (uint32_t)(align_up(sizeof(float) * T * SH, 256) / 4);
    p.ex_stride = (uint32_t)(align_up(sizeof(float) * T * m.k * SH, 256) / 4);
    p.exs_stride = (uint32_t)(align_up(sizeof(float) * T * SH, 256) / 4);
    p.lg = take(4 * (size_t)p.lg_stride * nl);
    p.xs = take(4 * (size_t)p.x_stride * nl);
    p.ex = take(4 * (size_t)p.ex_stride * nl);
    p.ex_sh = take(4 * (size_t)p.exs_stride * nl);
    p.rows_done = take(128 * (size_t)nl);
    p.gu_done = take(128 * (size_t)DEC_UNIT_LINES * nl);
    p.tiles_done = take(128);
    p.err = take(128);
    p.done = take(128);
    p.total = o;
    return true;
}

int launch_decode(const DecodeCall & c, const DecodePlan & p, uint8_t * ws, hipStream_t s) {
    const MoePlan & m = p.moe;
    const int nb_d = (int)(m.N / QK_K);
    int G = 0;
    switch (nb_d) {
        case 2: G = decode_grid<1, 2>(); break;
        case 3: G = decode_grid<1, 3>(); break;
        case 4: G = decode_grid<1, 4>(); break;
        default: G = decode_grid<1, 8>(); break;
    }
    if (G <= 0) return fail(QWM_ERR_HIP, "persistent decode: occupancy query failed");
    if (G < m.T * m.k + (m.shared ? 1 : 0)) return fail(QWM_ERR_UNSUPPORTED, "persistent decode: grid smaller than the units");
    DecodeArgs d;
    std::memset(&d, 0, sizeof d);
    StepArgs & a = d.base[0];
    a.x = nullptr; a.rm = nullptr;
    a.E = (int)m.E; a.k = (int)m.k;
    a.N = (int)m.N; a.N_sh = (int)m.N_sh; a.shared = m.shared ? 1 : 0;
    a.slot_tables = c.slot_tables; a.table_stride = c.table_stride;
    a.act = reinterpret_cast<float *>(ws + m.act); a.act_sh = reinterpret_cast<float *>(ws + m.act_sh);
    a.tile_counters = reinterpret_cast<int32_t *>(ws + m.tile_counters);
    a.err = reinterpret_cast<int32_t *>(ws + p.err);
    a.tiles_done = reinterpret_cast<int32_t *>(ws + p.tiles_done);
    a.spin = spin_limit();
    d.lg = reinterpret_cast<float *>(ws + p.lg); d.lg_stride = p.lg_stride;
    d.xs = reinterpret_cast<float *>(ws + p.xs); d.x_stride = p.x_stride;
    d.ex = reinterpret_cast<float *>(ws + p.ex); d.ex_stride = p.ex_stride;
    d.ex_sh = reinterpret_cast<float *>(ws + p.ex_sh); d.exs_stride = p.exs_stride;
    d.rows_done = reinterpret_cast<int32_t *>(ws + p.rows_done);
    d.gu_done = reinterpret_cast<int32_t *>(ws + p.gu_done);
    d.done = reinterpret_cast<int32_t *>(ws + p.done);
    d.x = c.x;
    d.ids_all = c.ids_all;
    d.res_bits = c.res_bits; d.res_words = (int32_t)((m.E + 31) / 32); d.res_flag = c.res_flag;
    for (int32_t first = 0; first < c.n_layers; first += DEC_LAYERS) {
        d.first = first;
        d.n_layers = std::min<int32_t>(DEC_LAYERS, c.n_layers - first);
        for (int j = 0; j < d.n_layers; ++j) {
            const qwm_moe_layer & L = c.layers[first + j];
            DecodeLayer & D = d.L[j];
            D.W_r = (const float *)L.router.data;
            D.sgi = (m.shared && L.sh_gate_inp.data) ? (const float *)L.sh_gate_inp.data : nullptr;
            D.bias = L.exp_probs_b.data ? (const float *)L.exp_probs_b.data : nullptr;
            D.gate = (const uint8_t *)L.gate_pool.data; D.up = (const uint8_t *)L.up_pool.data;
            D.down = (const uint8_t *)L.down_pool.data;
            D.sh_gate = (const uint8_t *)L.sh_gate.data; D.sh_up = (const uint8_t *)L.sh_up.data;
            D.sh_down = (const uint8_t *)L.sh_down.data;
            D.gu_slab = (uint32_t)L.gate_pool.nb[2]; D.down_slab = (uint32_t)L.down_pool.nb[2];
            D.n_slots[0] = (int32_t)L.gate_pool.ne[2]; D.n_slots[1] = (int32_t)L.up_pool.ne[2];
            D.n_slots[2] = (int32_t)L.down_pool.ne[2];
            D.norm = L.norm_weights; D.sigm = L.gating_func == 2 ? 1 : 0; D.scale = L.weights_scale;
            D.d6 = L.down_pool.type == T_Q6_K ? 1 : 0;
        }
        prof_begin("decode", s);
        switch (nb_d) {
            case 2: k_decode<1, 2><<<dim3((unsigned)G), dim3(256), 0, s>>>(d); break;
            case 3: k_decode<1, 3><<<dim3((unsigned)G), dim3(256), 0, s>>>(d); break;
            case 4: k_decode<1, 4><<<dim3((unsigned)G), dim3(256), 0, s>>>(d); break;
            default: k_decode<1, 8><<<dim3((unsigned)G), dim3(256), 0, s>>>(d); break;
        }
        prof_end("decode", s);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return failf(QWM_ERR_HIP, "persistent decode launch: %s", hipGetErrorString(e));
    }
    return QWM_OK;
}

}  // namespace qwm
