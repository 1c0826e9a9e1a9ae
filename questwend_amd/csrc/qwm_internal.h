// qwm_internal.h -- host-side declarations shared by the libqwmoe sources:
// workspace plans and the kernel launchers each .hip file provides.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>
#include <string>

#include "../../include/qwmoe.h"

namespace qwm {

// ggml_type values (ggml.h:390-420)
enum : int32_t { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_Q8_K = 15, T_I32 = 26 };

// The calling thread's last error lives in a fixed buffer: recording one
// never allocates, so an error path (out of memory included) cannot throw.
void set_error(const char * msg) noexcept;
const char * last_error() noexcept;
int fail(int code, const char * msg) noexcept;
int fail(int code, const std::string & msg) noexcept;
int failf(int code, const char * fmt, ...) noexcept __attribute__((format(printf, 2, 3)));
void set_spin_limit(uint32_t n);   // qwm_step.hip
#define QWM_HIP_CHECK(expr)                                                          \
    do {                                                                             \
        hipError_t e_ = (expr);                                                      \
        if (e_ != hipSuccess)                                                        \
            return ::qwm::failf(QWM_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

// The exception barrier of the C ABI: every extern "C" entry point runs its
// body through guard(), which turns std::bad_alloc into QWM_ERR_NOMEM and any
// other exception into QWM_ERR_INTERNAL, so nothing unwinds into C callers.
int fail_exception(const char * who) noexcept;   // call only inside a catch block
template <class F>
inline int guard(const char * who, F && f) noexcept {
    try {
        return f();
    } catch (...) {
        return fail_exception(who);
    }
}
template <class F>
inline size_t guard_size(const char * who, F && f) noexcept {   // 0 on an exception
    try {
        return f();
    } catch (...) {
        fail_exception(who);
        return 0;
    }
}
template <class F>
inline void guard_void(const char * who, F && f) noexcept {
    try {
        f();
    } catch (...) {
        fail_exception(who);
    }
}

constexpr int MAX_T = 8;        // tokens per GEMV batch (decode / verify)
constexpr int MAX_TILES = 512;  // row tiles of the down projection (combine tickets)
constexpr int MAX_K = 16;       // experts per token
constexpr int MAX_E = 2048;     // experts per layer
constexpr int MAX_PAIRS = MAX_T * MAX_K;

// Row lengths the expert GEMVs are built for (the hidden size as their K):
// 256 .. 2048 in steps of 256, then 3072 and 4096.
inline bool hidden_supported(int64_t K) {
    return K > 0 && K % 256 == 0 && (K <= 2048 || K == 3072 || K == 4096);
}

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// One expert of the layer's batch union and the (token, slot) pairs that
// routed to it, in token-major order (pair = t * k + j).
struct Unit {
    int32_t expert;     // expert id; -1 for the shared expert
    int32_t n;          // number of pairs
    int32_t pair[MAX_T];
};

// Byte offsets into the caller's workspace for one MoE layer call.
struct MoePlan {
    int64_t H, N, N_sh, E, k, T;
    bool shared, shared_gate;
    size_t counters, tile_counters, logits, ids, w, slots, sh_gate, units, uslot, n_units;
    size_t xq_qs, xq_d, xq_bs, xq_d0, xq_x, act, act_sh, ex, ex_sh;
    size_t total;
};
bool moe_plan(const qwm_moe_layer * L, int64_t T, MoePlan & p, std::string & why);

struct VerifyPlan {
    int64_t H, V, T;
    int n_wg;
    size_t counters, hq, partial_v, partial_i;
    size_t total;
};
bool verify_plan(const qwm_tensor * lm_head, int64_t T, VerifyPlan & p, std::string & why);

// ---- launchers (qwm_moe.hip) ----
struct RouteArgs {
    const float * W; const float * x; const float * rm;   // router [E][H], x [T][H], rm [T][E] or null
    const float * sh_gate_inp;                           // [H] or null
    int64_t E, H, T, k; int norm, sigm; float scale;
    const float * bias;                                  // exp_probs_b [E] or null
    const int32_t * slot_tables; int64_t table_stride; int32_t layer;  // resident remap or null
    int32_t wtype;                                       // pool type: the activation format of x
    const uint32_t * res_bits = nullptr;                 // residency bits of the layer's experts, or null
    int32_t * res_flag = nullptr;                        // set to 1 when a selected expert's bit is clear
};
int launch_route(const RouteArgs & a, const MoePlan & p, uint8_t * ws, int32_t * ids_out, int64_t ids_ld,
                 float * w_out, int64_t w_ld, hipStream_t s);

struct ExpertArgs {
    int32_t wtype;          // gate and up pools (and the shared expert's)
    int32_t down_type;      // down pools: wtype, or Q6_K beside Q4_K / Q5_K gate/up
    const uint8_t * gate; const uint8_t * up; const uint8_t * down;   // pool bases
    size_t gate_slab, up_slab, down_slab;                             // bytes per slot
    int32_t n_slots_g, n_slots_u, n_slots_d;                          // slots per pool: ids are clamped into them
    const uint8_t * sh_gate; const uint8_t * sh_up; const uint8_t * sh_down;
    const int32_t * slot_g; const int32_t * slot_u; const int32_t * slot_d;  // [T][k]
    const int32_t * uslot;  // [unit][4] from the route's resident remap, or null
    const float * weights;  // [T][k]
    const float * resid;    // [T][H] or null
    float * out;            // [T][H]
};
int launch_experts(const ExpertArgs & a, const MoePlan & p, uint8_t * ws, hipStream_t s);

// the persistent decode loop (qwm_decode.hip): layers of one launch keep
// their own logits, Q8_K of x, x, expert outputs and counters
struct DecodePlan {
    MoePlan moe;                                              // act, act_sh, tile tickets
    uint32_t lg_stride, xq_stride, x_stride, ex_stride, exs_stride;   // dwords per layer
    size_t lg, xq, xs, ex, ex_sh, rows_done, gu_done, tiles_done, err, done;
    size_t total;
};
struct DecodeCall {
    const qwm_moe_layer * layers; int32_t n_layers;
    const int32_t * slot_tables; int64_t table_stride;
    float * x;                                                // [T][H], in and out
    int32_t * ids_all;                                        // [layer][T][k] or null
    const uint32_t * res_bits; int32_t * res_flag;            // or null
};
bool decode_plan(const qwm_moe_layer * layers, int32_t n_layers, int64_t T, DecodePlan & p, std::string & why);
int launch_decode(const DecodeCall & c, const DecodePlan & p, uint8_t * ws, hipStream_t s);

// generic GGML_OP_MUL_MAT_ID (qwm_moe.hip)
struct MmidArgs {
    int32_t wtype; const uint8_t * as; size_t slab; int64_t K, N, n_as;
    const float * b; int64_t ne11, T; const int32_t * ids; int64_t n_ids;
    size_t b_nb1, b_nb2, ids_nb1, dst_nb1, dst_nb2;
    float * dst;
};
size_t mmid_workspace(int64_t K, int64_t T, int64_t ne11, int64_t n_ids);
int launch_mmid(const MmidArgs & a, uint8_t * ws, hipStream_t s);
// prefill-sized batches (T > MAX_T), qwm_prefill.hip
size_t prefill_workspace(int64_t K, int64_t N, int64_t n_as, int64_t T, int64_t ne11, int64_t n_ids);
// the grouped GEMM's reach: Q4_K or Q8_0 weights, K % 256 == 0 and <= 2048, N % 64 == 0,
// at most 4096 experts, slabs below 2 GiB, `as` 16-byte aligned (nullptr: not checked)
bool prefill_supported(int32_t wtype, int64_t K, int64_t N, int64_t n_as, const void * as, std::string & why);
// up != nullptr: the gate/up/SwiGLU pass (a.as = gate, dst = act)
int launch_prefill(const MmidArgs & a, uint8_t * ws, hipStream_t s, const uint8_t * up = nullptr);

// ---- the fused verify step (qwm_step.hip) ----
struct StepPlan {
    MoePlan moe;
    int64_t V;
    size_t v_counter, v_pv, v_pi, lg, xq_x, bar, gu_done, tiles_done, total;
};
bool step_plan(const qwm_moe_layer * L, const qwm_tensor * lm_head, int64_t T, StepPlan & p, std::string & why);
struct StepCall {
    const qwm_moe_layer * L; int32_t layer; const int32_t * slot_tables; int64_t table_stride;
    const float * x; const float * rm; const float * resid; float * out;
    int32_t * ids_out; int64_t ids_ld; float * w_out; int64_t w_ld;
    const uint8_t * lm_head; const float * norm_w; float eps; const int32_t * drafts; int32_t * result;
};
int launch_step(const StepCall & c, const StepPlan & p, uint8_t * ws, hipStream_t s);

// ---- launchers (qwm_verify.hip) ----
int launch_verify(const uint8_t * lm_head, const float * x, const float * norm_w, float eps,
                  const int32_t * drafts, int32_t * result, const VerifyPlan & p, uint8_t * ws, hipStream_t s);

int launch_fill_zero(void * p, size_t bytes, hipStream_t s);

// ---- batched MoE layer tail (qwm_batch.hip) ----
int launch_swiglu_rows(const float * g, const float * u, float * act, int n, int64_t rows, hipStream_t s);
int launch_combine_batch(const float * ex, const float * w, const float * sh, const float * shg, const float * resid,
                         float * out, int H, int k, int64_t T, hipStream_t s);
int launch_sh_gate(const float * gw, const float * x, float * shg, int H, int T, hipStream_t s);

// ---- slab gather (qwm_fetch.hip) ----
constexpr int GATHER_MAX = 224;   // misses per launch (kernel arguments stay under 2 KiB)
struct GatherItem {
    int32_t expert;   // slab index in the role's host tensor of the layer
    int16_t slot;     // pool slot
    int16_t role;     // 0 gate, 1 up, 2 down
};
struct GatherArgs {
    const uint8_t * src[3];   // device-visible address of the layer's pinned host slabs, per role
    uint8_t * dst[3];         // pool base, per role
    uint64_t slab[3];         // bytes per slab (multiples of 16)
    uint64_t src_stride[3];   // bytes between source slabs (0: slab)
    int32_t n, wg_per_item;
    GatherItem item[GATHER_MAX];
};
int launch_slab_gather(const GatherArgs & a, hipStream_t s);

// ---- qwm_pool.cpp: what qwm_gguf.cpp needs of a pool ----
int32_t pool_n_layer(const qwm_pool * p);
int32_t pool_n_expert(const qwm_pool * p);
size_t pool_slab_bytes(const qwm_pool * p, int role, int32_t layer);
int pool_check_layer(const qwm_pool * p, int32_t layer, const qwm_tensor * const t[3], const char * who);

// ---- qwm_quant.hip ----
int launch_quantize(int32_t type, const float * src, void * dst, int64_t n, hipStream_t s);

// ---- per-kernel event timing (qwm_capi.cpp) ----
void prof_begin(const char * kernel, hipStream_t s);
void prof_end(const char * kernel, hipStream_t s);
#define QWM_TIMED(NAME, STREAM, ...)       \
    do {                                   \
        ::qwm::prof_begin(NAME, STREAM);   \
        __VA_ARGS__;                       \
        ::qwm::prof_end(NAME, STREAM);     \
    } while (0)

}  // namespace qwm
