// qwm_step.hip -- the whole MTP verify step in one persistent launch: the MoE
// block (router, selection, gate/up + SwiGLU, down + combine + residual) and
// the verify head (rms_norm, Q8_0 lm_head GEMV + argmax, greedy accept).
//
// The per-op kernels (qwm_moe.hip, qwm_verify.hip) spend most of a verify step
// in latency: kernel boundaries, single-shot waves that occupy the GPU in
// rounds, and the serial selection tail of one workgroup.  Here a grid of
// exactly the co-resident workgroups (sized by the occupancy query) walks the
// phases:
//
//   P0  router rows (CPU summation order) and Q8_K of x, counted per
//       workgroup                                                -> count
//   P1  every workgroup repeats the selection for all tokens from the logits
//       (softmax, top-k, weights, expert union, slots) in registers and LDS:
//       no hand-off and no serial tail
//   P2  gate/up GEMVs over the expert union in ggml-CPU's exact float order
//       (qwm_exact.h), fused SwiGLU; each finished item counts for its unit
//   P3  down GEMVs: an item requests its weight rows, then waits for its
//       unit's gate/up items only; the last unit to finish a row tile
//       combines it (CPU order, + shared expert, + residual) and counts it
//   P4  the verify head of qwm_vhead.h on the block's output: the first
//       lm_head tiles are requested, then the workgroup waits for every
//       combined tile
//
// Data that crosses workgroups inside the launch is written with agent-scope
// stores (write-through, coherent across the XCDs' L2s) into buffers that no
// workgroup reads before the counter or ticket that publishes them.  Every
// 128-byte line of such a buffer has a single writing workgroup (the router
// logits and the combine tiles are padded or aligned for that), so a
// consumer's ordinary L2-cached load can only find that writer's fresh line
// or none; the one multi-writer buffer (SwiGLU activations) is read with
// agent-scope loads.  Every hand-off is a completion counter: P0 -> P1 counts
// the workgroups holding router rows or x blocks (the others do not take
// part, so a workgroup that starts late delays nobody), P2 -> P3 counts per unit and
// P3 -> P4 the combined tiles, so no workgroup waits for work it does not
// read.  Every wait is bounded (a timeout sets an error word and the result
// reports a = -1 instead of hanging); the last workgroup of the launch
// re-arms the counters.
#include "qwm_step_kernel.h"

// ======================================================================
// host side
// ======================================================================
namespace qwm {


bool step_plan(const qwm_moe_layer * L, const qwm_tensor * lm_head, int64_t T, StepPlan & p, std::string & why) {
    if (!moe_plan(L, T, p.moe, why)) return false;
    if (p.moe.H != SH) { why = "the fused step is built for hidden size 2048"; return false; }
    if (L->gate_pool.type != T_Q4_K || (L->down_pool.type != T_Q4_K && L->down_pool.type != T_Q6_K)) {
        why = "the fused step needs Q4_K gate/up pools and Q4_K or Q6_K down pools";
        return false;
    }
    if (p.moe.N != 512 && p.moe.N != 768 && p.moe.N != 1024 && p.moe.N != 2048) {
        why = "the fused step is built for FFN widths 512, 768, 1024 and 2048";
        return false;
    }
    if (p.moe.shared && p.moe.N_sh != p.moe.N) { why = "the fused step needs the shared expert's FFN width = the routed one"; return false; }
    if (p.moe.E > STEP_MAX_E) { why = "the fused step handles up to 512 experts"; return false; }
    if (lm_head->type != T_Q8_0 || lm_head->ne[0] != SH) { why = "lm_head must be Q8_0 [2048, V]"; return false; }
    p.V = lm_head->ne[1];
    if (p.V < 8LL * MAX_STEP_WG || p.V > (1LL << 30)) { why = "the fused step needs 8192 <= V <= 2^30"; return false; }
    size_t o = align_up(p.moe.total, 256);
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    p.v_counter = take(256);
    p.v_pv = take(sizeof(float) * MAX_STEP_WG * T);
    p.v_pi = take(sizeof(int32_t) * MAX_STEP_WG * T);
    p.lg = take(sizeof(float) * 32 * (p.moe.E + 1));
    p.xq_x = take(sizeof(uint32_t) * XSP * T * SNB);
    p.bar = take(512);                        // P0 workgroup count at 0, error word at 256
    p.gu_done = take(128 * (MAX_PAIRS + 1));
    p.tiles_done = take(128);
    p.total = o;
    return true;
}

static uint32_t g_spin_limit = SPIN_LIMIT;
uint32_t spin_limit() { return __atomic_load_n(&g_spin_limit, __ATOMIC_RELAXED); }
void set_spin_limit(uint32_t n) { __atomic_store_n(&g_spin_limit, n, __ATOMIC_RELAXED); }

int launch_step(const StepCall & c, const StepPlan & p, uint8_t * ws, hipStream_t s) {
    const qwm_moe_layer * L = c.L;
    const MoePlan & m = p.moe;
    StepArgs a;
    a.W_r = (const float *)L->router.data; a.x = c.x; a.rm = c.rm;
    a.sgi = (L->sh_gate.data && L->sh_gate_inp.data) ? (const float *)L->sh_gate_inp.data : nullptr;
    a.E = (int)m.E; a.k = (int)m.k; a.norm = L->norm_weights; a.scale = L->weights_scale;
    a.sigm = L->gating_func == 2 ? 1 : 0;
    a.bias = L->exp_probs_b.data ? (const float *)L->exp_probs_b.data : nullptr;
    a.N = (int)m.N; a.N_sh = (int)m.N_sh; a.shared = m.shared ? 1 : 0;
    a.gate = (const uint8_t *)L->gate_pool.data; a.up = (const uint8_t *)L->up_pool.data;
    a.down = (const uint8_t *)L->down_pool.data;
    a.gate_slab = L->gate_pool.nb[2]; a.up_slab = L->up_pool.nb[2]; a.down_slab = L->down_pool.nb[2];
    a.n_slots[0] = (int)L->gate_pool.ne[2]; a.n_slots[1] = (int)L->up_pool.ne[2];
    a.n_slots[2] = (int)L->down_pool.ne[2];
    a.sh_gate = (const uint8_t *)L->sh_gate.data; a.sh_up = (const uint8_t *)L->sh_up.data;
    a.sh_down = (const uint8_t *)L->sh_down.data;
    a.slot_tables = c.slot_tables; a.table_stride = c.table_stride; a.layer = c.layer;
    a.resid = c.resid; a.out = c.out;
    a.ids_out = c.ids_out; a.ids_ld = c.ids_ld; a.w_out = c.w_out; a.w_ld = c.w_ld;
    a.lg = reinterpret_cast<float *>(ws + p.lg);
    a.act = reinterpret_cast<float *>(ws + m.act); a.act_sh = reinterpret_cast<float *>(ws + m.act_sh);
    a.ex = reinterpret_cast<float *>(ws + m.ex); a.ex_sh = reinterpret_cast<float *>(ws + m.ex_sh);
    a.xq_x = reinterpret_cast<uint32_t *>(ws + p.xq_x);
    a.rows_done = reinterpret_cast<int32_t *>(ws + p.bar);
    a.err = reinterpret_cast<int32_t *>(ws + p.bar + 256);
    a.tile_counters = reinterpret_cast<int32_t *>(ws + m.tile_counters);
    a.gu_done = reinterpret_cast<int32_t *>(ws + p.gu_done);
    a.tiles_done = reinterpret_cast<int32_t *>(ws + p.tiles_done);
    a.spin = spin_limit();
    VerifyArgs & v = a.v;
    v.W = c.lm_head; v.H = SH; v.V = (int)p.V;
    v.x = c.out; v.norm_w = c.norm_w; v.eps = c.eps;
    v.drafts = c.drafts; v.result = c.result;
    v.pv = reinterpret_cast<float *>(ws + p.v_pv);
    v.pi = reinterpret_cast<int32_t *>(ws + p.v_pi);
    v.counter = reinterpret_cast<int32_t *>(ws + p.v_counter);
    const int nb_d = (int)(m.N / QK_K);          // step_plan: 2, 3, 4 or 8
    a.d6 = L->down_pool.type == T_Q6_K ? 1 : 0;   // step_plan: Q4_K, or Q6_K down
    switch (m.T) {
        case 1: return launch_step_nt<1>(a, nb_d, s);
        case 2: return launch_step_nt<2>(a, nb_d, s);
        case 3: return launch_step_nt<3>(a, nb_d, s);
        case 4: return launch_step_nt<4>(a, nb_d, s);
        case 5: return launch_step_nt<5>(a, nb_d, s);
        case 8: return launch_step_t8(a, nb_d, s);
        default: return launch_step_hi(a, (int)m.T, nb_d, s);
    }
}

}  // namespace qwm
