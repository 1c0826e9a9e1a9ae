// qwm_capi.cpp -- the extern "C" entry points of libqwmoe (include/qwmoe.h):
// argument validation against ggml's op contracts, workspace planning, and
// dispatch to the gfx950 kernels.  No C++ exception crosses the ABI.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "qwm_internal.h"

namespace qwm {


static size_t type_size(int32_t type) {
    switch (type) {
        case T_F32: return 4;
        case T_I32: return 4;
        case T_Q8_0: return 34;
        case T_Q4_K: return 144;
        case T_Q6_K: return 210;
        case T_Q5_K: return 176;
    }
    return 0;
}
static int64_t block_len(int32_t type) {
    switch (type) {
        case T_Q8_0: return 32;
        case T_Q4_K: return 256;
        case T_Q6_K: return 256;
        case T_Q5_K: return 256;
    }
    return 1;
}

// rows contiguous and densely packed in the first two dimensions
static bool contiguous_rows(const qwm_tensor * t) {
    const size_t ts = type_size(t->type);
    if (!ts || t->ne[0] % block_len(t->type)) return false;
    if (t->nb[0] != ts) return false;
    return t->nb[1] == ts * (size_t)(t->ne[0] / block_len(t->type));
}
static bool fully_contiguous(const qwm_tensor * t) {
    if (!contiguous_rows(t)) return false;
    return t->nb[2] == t->nb[1] * (size_t)t->ne[1] && t->nb[3] == t->nb[2] * (size_t)t->ne[2];
}

// ---- per-kernel event timing ----
struct Profile {
    std::string kernel;
    std::vector<hipEvent_t> ev;    // start/stop pairs
    int used = 0;
    bool open = false;
};
static Profile g_prof;

// the profiled name, or with a trailing '*' every name it prefixes
static bool prof_match(const char * kernel) {
    const std::string & k = g_prof.kernel;
    if (!k.empty() && k.back() == '*') return std::strncmp(kernel, k.data(), k.size() - 1) == 0;
    return k == kernel;
}

void prof_begin(const char * kernel, hipStream_t s) {
    if (!g_prof.open || !prof_match(kernel) || 2 * g_prof.used + 1 >= (int)g_prof.ev.size()) return;
    (void)hipEventRecord(g_prof.ev[2 * g_prof.used], s);
}
void prof_end(const char * kernel, hipStream_t s) {
    if (!g_prof.open || !prof_match(kernel) || 2 * g_prof.used + 1 >= (int)g_prof.ev.size()) return;
    (void)hipEventRecord(g_prof.ev[2 * g_prof.used + 1], s);
    g_prof.used++;
}

}  // namespace qwm

using namespace qwm;

extern "C" {

void qwm_tensor_init(qwm_tensor * t, int32_t type, int64_t ne0, int64_t ne1, int64_t ne2, void * data) {
    guard_void("qwm_tensor_init", [&]() {
        std::memset(t, 0, sizeof(*t));
        t->type = type;
        t->ne[0] = ne0; t->ne[1] = ne1; t->ne[2] = ne2; t->ne[3] = 1;
        t->nb[0] = type_size(type);
        t->nb[1] = t->nb[0] * (size_t)(ne0 / block_len(type));
        t->nb[2] = t->nb[1] * (size_t)ne1;
        t->nb[3] = t->nb[2] * (size_t)ne2;
        t->data = data;
    });
}

const char * qwm_version(void) { return "qwmoe 0.1 gfx950"; }
const char * qwm_last_error(void) { return last_error(); }

int qwm_workspace_init(void * workspace, size_t bytes, void * stream) {
    return guard("qwm_workspace_init", [&]() -> int {
        if (!workspace && bytes) return fail(QWM_ERR_ARG, "workspace is NULL");
        return launch_fill_zero(workspace, bytes & ~(size_t)3, (hipStream_t)stream);
    });
}

int qwm_quantize(int32_t type, const float * src, void * dst, int64_t n, void * stream) {
    return guard("qwm_quantize", [&]() -> int {
        if (type != T_Q4_K && type != T_Q8_0) return fail(QWM_ERR_UNSUPPORTED, "quantize: only Q4_K and Q8_0");
        if (!src || !dst || n < 0 || n % block_len(type)) return fail(QWM_ERR_ARG, "quantize: bad arguments");
        return launch_quantize(type, src, dst, n, (hipStream_t)stream);
    });
}

int qwm_profile_start(const char * kernel, int32_t max_launches) {
    return guard("qwm_profile_start", [&]() -> int {
        if (!kernel || max_launches < 1) return fail(QWM_ERR_ARG, "profile_start: bad arguments");
        for (hipEvent_t e : g_prof.ev) (void)hipEventDestroy(e);
        g_prof.ev.assign(2 * (size_t)max_launches, nullptr);
        for (auto & e : g_prof.ev) QWM_HIP_CHECK(hipEventCreate(&e));
        g_prof.kernel = kernel;
        g_prof.used = 0;
        g_prof.open = true;
        return QWM_OK;
    });
}

int qwm_set_spin_limit(uint32_t polls) {
    set_spin_limit(polls);
    return QWM_OK;
}

int qwm_profile_stop(float * durations_ms, int32_t capacity) {
    return guard("qwm_profile_stop", [&]() -> int {
        if (!g_prof.open) return fail(QWM_ERR_STATE, "profile_stop: profiling was not started");
        g_prof.open = false;
        const int n = std::min(g_prof.used, capacity);
        int rc = QWM_OK;
        for (int i = 0; i < n && rc == QWM_OK; ++i) {
            float ms = 0.f;
            hipError_t e = hipEventSynchronize(g_prof.ev[2 * i + 1]);
            if (e == hipSuccess) e = hipEventElapsedTime(&ms, g_prof.ev[2 * i], g_prof.ev[2 * i + 1]);
            if (e != hipSuccess) rc = fail(QWM_ERR_HIP, std::string("profile_stop: ") + hipGetErrorString(e));
            else if (durations_ms) durations_ms[i] = ms;
        }
        // the events are released here, not left for process exit (where the HIP
        // runtime and a profiler may already be tearing down)
        for (hipEvent_t e : g_prof.ev) (void)hipEventDestroy(e);
        g_prof.ev.clear();
        g_prof.used = 0;
        return rc == QWM_OK ? n : rc;
    });
}

// ------------------------------------------------------------ mul_mat_id --

// The grouped GEMM takes more than MAX_T columns of Q4_K or Q8_0 weights in the
// shapes it supports (N % 64, K up to 2048, 3072 or 4096, 16-byte aligned
// data); `data` false
// leaves the alignment out (a size query before the weights are placed).
static bool prefill_shape(const qwm_tensor * as, const qwm_tensor * b, bool data = true) {
    std::string why;
    return b->ne[2] > MAX_T && prefill_supported(as->type, as->ne[0], as->ne[1], as->ne[2], data ? as->data : nullptr, why);
}
static bool prefill_path(const qwm_tensor * as, const qwm_tensor * b) { return prefill_shape(as, b, true); }

static int check_mmid(const qwm_tensor * as, const qwm_tensor * b, const qwm_tensor * ids, const qwm_tensor * dst) {
    if (!as || !b || !ids) return fail(QWM_ERR_ARG, "mul_mat_id: NULL tensor");
    if (as->type != T_Q4_K && as->type != T_Q8_0 && as->type != T_Q6_K && as->type != T_Q5_K)
        return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: weights must be Q4_K, Q5_K, Q6_K or Q8_0");
    if (as->type == T_Q5_K && ((uintptr_t)as->data % 16))
        return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: Q5_K weights need 16-byte aligned data");
    if (as->type == T_Q6_K && ((uintptr_t)as->data % 4))   // rows and slabs may start 2 bytes off: handled
        return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: Q6_K weights need 4-byte aligned data");
    if (as->type == T_Q8_0 && ((uintptr_t)as->data % 4))   // the row dots read dwords from the row start
        return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: Q8_0 weights need 4-byte aligned data");
    if (b->type != T_F32 || ids->type != T_I32) return fail(QWM_ERR_ARG, "mul_mat_id: b must be f32 and ids i32");
    // ggml.c:3418-3428
    if (as->ne[3] != 1 || b->ne[3] != 1 || ids->ne[2] != 1 || ids->ne[3] != 1)
        return fail(QWM_ERR_ARG, "mul_mat_id: as/b must be 3-d and ids 2-d");
    if (ids->ne[1] != b->ne[2]) return fail(QWM_ERR_ARG, "mul_mat_id: ids->ne[1] != b->ne[2]");
    if (as->ne[0] != b->ne[0]) return fail(QWM_ERR_ARG, "mul_mat_id: as->ne[0] != b->ne[0]");
    if (b->ne[1] < 1 || ids->ne[0] % b->ne[1]) return fail(QWM_ERR_ARG, "mul_mat_id: ids->ne[0] % b->ne[1] != 0");
    if (!fully_contiguous(as)) return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: as must be contiguous");
    if (b->nb[0] != 4 || ids->nb[0] != 4) return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: b/ids must have unit element stride");
    if ((b->nb[1] | b->nb[2]) % 16) return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: b rows must be 16-byte aligned");
    if (prefill_path(as, b)) {                  // prefill: the grouped GEMM (qwm_prefill.hip)
        if (ids->ne[0] * ids->ne[1] > (1 << 22)) return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: too many (expert, column) pairs");
    } else if (b->ne[2] > MAX_T) {              // other types and shapes: the GEMV path over column chunks
        if (ids->ne[0] > MAX_PAIRS) return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: too many ids per column");
    } else if (ids->ne[0] * ids->ne[1] > MAX_PAIRS) {
        return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: too many (expert, column) pairs");
    }
    if (!hidden_supported(as->ne[0])) return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: K must be 256 .. 2048, 3072 or 4096");
    if (as->type == T_Q8_0 && as->ne[0] % 256) return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id: Q8_0 needs K a multiple of 256");
    if (dst) {
        if (dst->type != T_F32 || dst->ne[0] != as->ne[1] || dst->ne[1] != ids->ne[0] || dst->ne[2] != b->ne[2])
            return fail(QWM_ERR_ARG, "mul_mat_id: dst must be f32 [N, n_ids, T]");
        if (dst->nb[0] != 4) return fail(QWM_ERR_ARG, "mul_mat_id: dst must not be transposed");
    }
    return QWM_OK;
}

// Columns per GEMV launch when a batch of more than MAX_T columns of a type
// without the prefill GEMM is split (the pair table holds MAX_PAIRS pairs).
static int64_t mmid_chunk(int64_t n_ids) { return std::max<int64_t>(1, std::min<int64_t>(MAX_T, MAX_PAIRS / n_ids)); }

size_t qwm_mul_mat_id_workspace_size(const qwm_tensor * as, const qwm_tensor * b, const qwm_tensor * ids) {
    return guard_size("qwm_mul_mat_id_workspace_size", [&]() -> size_t {
        if (check_mmid(as, b, ids, nullptr) != QWM_OK) return 0;
        // either path's need: the grouped GEMM, or the GEMV chunks it falls back to for unaligned weights
        size_t need = 0;
        if (ids->ne[0] <= MAX_PAIRS)
            need = mmid_workspace(as->ne[0], std::min<int64_t>(b->ne[2], mmid_chunk(ids->ne[0])), b->ne[1], ids->ne[0]);
        if (prefill_shape(as, b, false))
            need = std::max(need, prefill_workspace(as->ne[0], as->ne[1], as->ne[2], b->ne[2], b->ne[1], ids->ne[0]));
        return need;
    });
}

int qwm_mul_mat_id(const qwm_tensor * as, const qwm_tensor * b, const qwm_tensor * ids, qwm_tensor * dst,
                   void * workspace, size_t ws_bytes, void * stream) {
    return guard("qwm_mul_mat_id", [&]() -> int {
        int rc = check_mmid(as, b, ids, dst);
        if (rc != QWM_OK) return rc;
        if (!dst) return fail(QWM_ERR_ARG, "mul_mat_id: dst is NULL");
        const bool prefill = prefill_path(as, b);
        const int64_t chunk = std::min<int64_t>(b->ne[2], mmid_chunk(ids->ne[0]));
        const size_t need = prefill ? prefill_workspace(as->ne[0], as->ne[1], as->ne[2], b->ne[2], b->ne[1], ids->ne[0])
                                    : mmid_workspace(as->ne[0], chunk, b->ne[1], ids->ne[0]);
        if (!workspace || ws_bytes < need) return fail(QWM_ERR_WORKSPACE, "mul_mat_id: workspace too small");
        MmidArgs a;
        a.wtype = as->type; a.as = (const uint8_t *)as->data; a.slab = as->nb[2];
        a.K = as->ne[0]; a.N = as->ne[1]; a.n_as = as->ne[2];
        a.b = (const float *)b->data; a.ne11 = b->ne[1]; a.T = b->ne[2];
        a.ids = (const int32_t *)ids->data; a.n_ids = ids->ne[0];
        a.b_nb1 = b->nb[1]; a.b_nb2 = b->nb[2]; a.ids_nb1 = ids->nb[1];
        a.dst_nb1 = dst->nb[1]; a.dst_nb2 = dst->nb[2];
        a.dst = (float *)dst->data;
        if (prefill) return launch_prefill(a, (uint8_t *)workspace, (hipStream_t)stream);
        // column chunks in order on one stream (each launch rewrites the workspace after the previous one)
        const int64_t T = b->ne[2];
        for (int64_t t0 = 0; t0 < T; t0 += chunk) {
            MmidArgs c = a;
            c.T = std::min(chunk, T - t0);
            c.b = (const float *)((const uint8_t *)b->data + t0 * b->nb[2]);
            c.ids = (const int32_t *)((const uint8_t *)ids->data + t0 * ids->nb[1]);
            c.dst = (float *)((uint8_t *)dst->data + t0 * dst->nb[2]);
            if ((rc = launch_mmid(c, (uint8_t *)workspace, (hipStream_t)stream)) != QWM_OK) return rc;
        }
        return QWM_OK;
    });
}

int qwm_swiglu(const qwm_tensor * gate, const qwm_tensor * up, qwm_tensor * act, void * stream) {
    return guard("qwm_swiglu", [&]() -> int {
        if (!gate || !up || !act) return fail(QWM_ERR_ARG, "swiglu: NULL tensor");
        const qwm_tensor * t3[3] = {gate, up, act};
        for (const qwm_tensor * t : t3) {
            if (t->type != T_F32) return fail(QWM_ERR_ARG, "swiglu: tensors must be f32");
            if (!fully_contiguous(t)) return fail(QWM_ERR_UNSUPPORTED, "swiglu: tensors must be contiguous");
            for (int i = 0; i < 4; ++i)
                if (t->ne[i] != gate->ne[i]) return fail(QWM_ERR_ARG, "swiglu: gate, up and act differ in shape");
        }
        const int64_t n = gate->ne[0], rows = gate->ne[1] * gate->ne[2] * gate->ne[3];
        if (n < 1 || n > INT32_MAX) return fail(QWM_ERR_UNSUPPORTED, "swiglu: row length out of range");
        return launch_swiglu_rows((const float *)gate->data, (const float *)up->data, (float *)act->data, (int)n, rows,
                                  (hipStream_t)stream);
    });
}

// gate and up of one expert FFN: both the same quantized [K, N, n_as] layout
// (the same slab stride too), act a contiguous f32 [N, n_ids, T].
static int check_swiglu(const qwm_tensor * gate, const qwm_tensor * up, const qwm_tensor * b, const qwm_tensor * ids,
                        const qwm_tensor * act) {
    int rc = check_mmid(gate, b, ids, act);
    if (rc != QWM_OK) return rc;
    if ((rc = check_mmid(up, b, ids, nullptr)) != QWM_OK) return rc;
    if (up->type != gate->type) return fail(QWM_ERR_ARG, "mul_mat_id_swiglu: gate and up differ in type");
    for (int i = 0; i < 4; ++i)
        if (up->ne[i] != gate->ne[i] || up->nb[i] != gate->nb[i])
            return fail(QWM_ERR_ARG, "mul_mat_id_swiglu: gate and up differ in shape or strides");
    if (act && !fully_contiguous(act)) return fail(QWM_ERR_UNSUPPORTED, "mul_mat_id_swiglu: act must be contiguous");
    return QWM_OK;
}

static bool swiglu_fused(const qwm_tensor * gate, const qwm_tensor * up, const qwm_tensor * b) {
    return prefill_path(gate, b) && prefill_path(up, b);
}

// the separate path's layout: g and u [N, n_ids, T] f32, then the MUL_MAT_ID workspace
static size_t swiglu_split_bytes(const qwm_tensor * gate, const qwm_tensor * b, const qwm_tensor * ids) {
    return align_up(sizeof(float) * (size_t)gate->ne[1] * ids->ne[0] * b->ne[2], 256);
}

// workspace of one path: the grouped pass (fused) or the two calls and SwiGLU
static size_t swiglu_need(const qwm_tensor * gate, const qwm_tensor * b, const qwm_tensor * ids, bool fused) {
    if (fused) return prefill_workspace(gate->ne[0], gate->ne[1], gate->ne[2], b->ne[2], b->ne[1], ids->ne[0]);
    return 2 * swiglu_split_bytes(gate, b, ids) + qwm_mul_mat_id_workspace_size(gate, b, ids);
}

size_t qwm_mul_mat_id_swiglu_workspace_size(const qwm_tensor * gate, const qwm_tensor * up, const qwm_tensor * b,
                                            const qwm_tensor * ids) {
    return guard_size("qwm_mul_mat_id_swiglu_workspace_size", [&]() -> size_t {
        if (check_swiglu(gate, up, b, ids, nullptr) != QWM_OK) return 0;
        // either path's need (the split path serves weights the grouped pass cannot take)
        return std::max(swiglu_need(gate, b, ids, prefill_shape(gate, b, false)), swiglu_need(gate, b, ids, false));
    });
}

int qwm_mul_mat_id_swiglu(const qwm_tensor * gate, const qwm_tensor * up, const qwm_tensor * b, const qwm_tensor * ids,
                          qwm_tensor * act, void * workspace, size_t ws_bytes, void * stream) {
    return guard("qwm_mul_mat_id_swiglu", [&]() -> int {
        int rc = check_swiglu(gate, up, b, ids, act);
        if (rc != QWM_OK) return rc;
        if (!act) return fail(QWM_ERR_ARG, "mul_mat_id_swiglu: act is NULL");
        const bool fused = swiglu_fused(gate, up, b);
        const size_t need = swiglu_need(gate, b, ids, fused);
        if (!workspace || ws_bytes < need) return fail(QWM_ERR_WORKSPACE, "mul_mat_id_swiglu: workspace too small");
        hipStream_t s = (hipStream_t)stream;
        if (fused) {
            MmidArgs a;
            a.wtype = gate->type; a.as = (const uint8_t *)gate->data; a.slab = gate->nb[2];
            a.K = gate->ne[0]; a.N = gate->ne[1]; a.n_as = gate->ne[2];
            a.b = (const float *)b->data; a.ne11 = b->ne[1]; a.T = b->ne[2];
            a.ids = (const int32_t *)ids->data; a.n_ids = ids->ne[0];
            a.b_nb1 = b->nb[1]; a.b_nb2 = b->nb[2]; a.ids_nb1 = ids->nb[1];
            a.dst_nb1 = act->nb[1]; a.dst_nb2 = act->nb[2];
            a.dst = (float *)act->data;
            return launch_prefill(a, (uint8_t *)workspace, s, (const uint8_t *)up->data);
        }
        // two MUL_MAT_ID calls into the workspace, then the element-wise SwiGLU
        const size_t gb = swiglu_split_bytes(gate, b, ids);
        uint8_t * w = (uint8_t *)workspace;
        qwm_tensor g = *act, u = *act;
        g.data = w; u.data = w + gb;
        if ((rc = qwm_mul_mat_id(gate, b, ids, &g, w + 2 * gb, ws_bytes - 2 * gb, stream)) != QWM_OK) return rc;
        if ((rc = qwm_mul_mat_id(up, b, ids, &u, w + 2 * gb, ws_bytes - 2 * gb, stream)) != QWM_OK) return rc;
        return launch_swiglu_rows((const float *)g.data, (const float *)u.data, (float *)act->data, (int)gate->ne[1],
                                  ids->ne[0] * b->ne[2], s);
    });
}

// ------------------------------------------------------------- MoE block --

static int check_layer(const qwm_moe_layer * L, int64_t T, MoePlan & p) {
    if (!L) return fail(QWM_ERR_ARG, "moe: layer is NULL");
    std::string why;
    if (L->router.type != T_F32 || !contiguous_rows(&L->router)) return fail(QWM_ERR_UNSUPPORTED, "moe: router must be contiguous f32 [H, E]");
    const qwm_tensor * pools[3] = {&L->gate_pool, &L->up_pool, &L->down_pool};
    for (const qwm_tensor * t : pools) {
        if (t->type != T_Q4_K && t->type != T_Q8_0 && t->type != T_Q5_K && t->type != T_Q6_K)
            return fail(QWM_ERR_UNSUPPORTED, "moe: pools must be Q4_K, Q5_K, Q8_0 or (down only) Q6_K");
        if (!fully_contiguous(t)) return fail(QWM_ERR_UNSUPPORTED, "moe: pools must be contiguous");
    }
    // gate and up of one type; down the same, or Q6_K beside Q4_K / Q5_K (K-quant "_M" files)
    const int32_t gt = L->gate_pool.type;
    if (L->up_pool.type != gt || gt == T_Q6_K ||
        (L->down_pool.type != gt && !(L->down_pool.type == T_Q6_K && (gt == T_Q4_K || gt == T_Q5_K))))
        return fail(QWM_ERR_UNSUPPORTED, "moe: mixed pool types (only a Q6_K down pool beside Q4_K or Q5_K gate/up is handled)");
    for (const qwm_tensor * t : pools)
        if (t->type == T_Q5_K && ((uintptr_t)t->data % 16)) return fail(QWM_ERR_UNSUPPORTED, "moe: Q5_K pools need 16-byte aligned data");
    if (L->down_pool.type == T_Q6_K && ((uintptr_t)L->down_pool.data % 4))
        return fail(QWM_ERR_UNSUPPORTED, "moe: Q6_K pools need 4-byte aligned data");
    if (L->gate_pool.ne[0] != L->router.ne[0] || L->up_pool.ne[0] != L->router.ne[0] ||
        L->up_pool.ne[1] != L->gate_pool.ne[1] || L->down_pool.ne[0] != L->gate_pool.ne[1] ||
        L->down_pool.ne[1] != L->router.ne[0])
        return fail(QWM_ERR_ARG, "moe: pool shapes disagree (gate/up [H, N, S], down [N, H, S])");
    for (const qwm_tensor * t : pools)   // the kernels clamp slot ids into [0, S)
        if (t->ne[2] < 1 || t->ne[2] > INT32_MAX || t->ne[3] != 1)
            return fail(QWM_ERR_ARG, "moe: a pool needs 1..2^31-1 slots (ne[2]) and ne[3] == 1");
    if (L->sh_gate.data) {
        if (!L->sh_up.data || !L->sh_down.data) return fail(QWM_ERR_ARG, "moe: shared expert needs gate, up and down");
        if (L->sh_gate.type != L->gate_pool.type || L->sh_up.type != L->gate_pool.type || L->sh_down.type != L->down_pool.type)
            return fail(QWM_ERR_UNSUPPORTED, "moe: shared expert types must match the pools'");
        if (L->sh_down.type == T_Q6_K && ((uintptr_t)L->sh_down.data % 4))
            return fail(QWM_ERR_UNSUPPORTED, "moe: Q6_K shared down must be 4-byte aligned");
        if (L->sh_gate.ne[0] != L->router.ne[0] || L->sh_up.ne[1] != L->sh_gate.ne[1] || L->sh_down.ne[0] != L->sh_gate.ne[1] ||
            L->sh_down.ne[1] != L->router.ne[0])
            return fail(QWM_ERR_ARG, "moe: shared expert shapes disagree");
        if (L->sh_gate_inp.data && (L->sh_gate_inp.type != T_F32 || L->sh_gate_inp.ne[0] != L->router.ne[0]))
            return fail(QWM_ERR_ARG, "moe: shared gate row must be f32 [H]");
    }
    // core/model.cpp:751-756: expert_gating_func is 1 (soft_max) or 2 (sigmoid); 0 is taken as the default
    if (L->gating_func != 0 && L->gating_func != 1 && L->gating_func != 2)
        return fail(QWM_ERR_UNSUPPORTED, "moe: gating_func must be 1 (soft_max) or 2 (sigmoid)");
    if (!moe_plan(L, T, p, why)) return fail(QWM_ERR_UNSUPPORTED, "moe: " + why);
    if (L->exp_probs_b.data && (L->exp_probs_b.type != T_F32 || L->exp_probs_b.ne[0] != p.E ||
                                L->exp_probs_b.ne[1] != 1 || L->exp_probs_b.nb[0] != 4))
        return fail(QWM_ERR_ARG, "moe: exp_probs_b must be f32 [E]");
    return QWM_OK;
}

static int check_act(const qwm_tensor * x, int64_t H, const char * what) {
    if (!x || !x->data) return fail(QWM_ERR_ARG, std::string("moe: ") + what + " is NULL");
    if (x->type != T_F32 || x->ne[0] != H || !fully_contiguous(x)) return fail(QWM_ERR_ARG, std::string("moe: ") + what + " must be contiguous f32 [H, T]");
    if ((uintptr_t)x->data % 16) return fail(QWM_ERR_ARG, std::string("moe: ") + what + " must be 16-byte aligned");
    return QWM_OK;
}

size_t qwm_moe_workspace_size(const qwm_moe_layer * layer, int64_t T) {
    return guard_size("qwm_moe_workspace_size", [&]() -> size_t {
        MoePlan p;
        if (check_layer(layer, T, p) != QWM_OK) return 0;
        return p.total;
    });
}

static int do_route(const qwm_moe_layer * L, const MoePlan & p, const qwm_tensor * x, const qwm_tensor * rm,
                    const int32_t * tables, int64_t stride, int32_t layer_index, int32_t * ids_out, int64_t ids_ld,
                    float * w_out, int64_t w_ld, uint8_t * ws, hipStream_t s, const uint32_t * res_bits = nullptr,
                    int32_t * res_flag = nullptr) {
    RouteArgs a;
    a.res_bits = res_bits; a.res_flag = res_flag;
    a.W = (const float *)L->router.data; a.x = (const float *)x->data;
    a.rm = rm ? (const float *)rm->data : nullptr;
    a.sh_gate_inp = (L->sh_gate.data && L->sh_gate_inp.data) ? (const float *)L->sh_gate_inp.data : nullptr;
    a.E = p.E; a.H = p.H; a.T = p.T; a.k = p.k; a.norm = L->norm_weights; a.scale = L->weights_scale;
    a.sigm = L->gating_func == 2 ? 1 : 0;
    a.bias = L->exp_probs_b.data ? (const float *)L->exp_probs_b.data : nullptr;
    a.slot_tables = tables; a.table_stride = stride; a.layer = layer_index;
    a.wtype = L->gate_pool.type;
    return launch_route(a, p, ws, ids_out, ids_ld, w_out, w_ld, s);
}

int qwm_moe_route(const qwm_moe_layer * layer, const qwm_tensor * x, const qwm_tensor * rm,
                  qwm_tensor * ids_out, qwm_tensor * w_out, void * workspace, size_t ws_bytes, void * stream) {
    return guard("qwm_moe_route", [&]() -> int {
        if (!x) return fail(QWM_ERR_ARG, "moe_route: x is NULL");
        MoePlan p;
        int rc = check_layer(layer, x->ne[1], p);
        if (rc != QWM_OK) return rc;
        if ((rc = check_act(x, p.H, "x")) != QWM_OK) return rc;
        if (rm && (rm->type != T_F32 || rm->ne[0] != p.E || rm->ne[1] != p.T || !fully_contiguous(rm)))
            return fail(QWM_ERR_ARG, "moe_route: rm must be contiguous f32 [E, T]");
        if (ids_out && (ids_out->type != T_I32 || ids_out->ne[0] != p.k || ids_out->ne[1] != p.T || ids_out->nb[0] != 4))
            return fail(QWM_ERR_ARG, "moe_route: ids_out must be i32 [k, T]");
        if (w_out && (w_out->type != T_F32 || w_out->ne[0] != p.k || w_out->ne[1] != p.T || w_out->nb[0] != 4))
            return fail(QWM_ERR_ARG, "moe_route: w_out must be f32 [k, T]");
        if (!workspace || ws_bytes < p.total) return fail(QWM_ERR_WORKSPACE, "moe_route: workspace too small");
        return do_route(layer, p, x, rm, nullptr, 0, 0, ids_out ? (int32_t *)ids_out->data : nullptr,
                        ids_out ? (int64_t)(ids_out->nb[1] / 4) : 0, w_out ? (float *)w_out->data : nullptr,
                        w_out ? (int64_t)(w_out->nb[1] / 4) : 0, (uint8_t *)workspace, (hipStream_t)stream);
    });
}

static int do_experts(const qwm_moe_layer * L, const MoePlan & p, const int32_t * sg, const int32_t * su,
                      const int32_t * sd, const float * w, const float * resid, float * out, uint8_t * ws, hipStream_t s,
                      const int32_t * uslot = nullptr) {
    ExpertArgs a;
    a.wtype = L->gate_pool.type;
    a.down_type = L->down_pool.type;
    a.gate = (const uint8_t *)L->gate_pool.data; a.up = (const uint8_t *)L->up_pool.data;
    a.down = (const uint8_t *)L->down_pool.data;
    a.gate_slab = L->gate_pool.nb[2]; a.up_slab = L->up_pool.nb[2]; a.down_slab = L->down_pool.nb[2];
    a.n_slots_g = (int32_t)L->gate_pool.ne[2]; a.n_slots_u = (int32_t)L->up_pool.ne[2];
    a.n_slots_d = (int32_t)L->down_pool.ne[2];
    a.sh_gate = (const uint8_t *)L->sh_gate.data; a.sh_up = (const uint8_t *)L->sh_up.data;
    a.sh_down = (const uint8_t *)L->sh_down.data;
    a.slot_g = sg; a.slot_u = su; a.slot_d = sd; a.uslot = uslot;
    a.weights = w; a.resid = resid; a.out = out;
    return launch_experts(a, p, ws, s);
}

int qwm_moe_experts(const qwm_moe_layer * layer, const qwm_tensor * x, const qwm_tensor * slot_g,
                    const qwm_tensor * slot_u, const qwm_tensor * slot_d, const qwm_tensor * weights,
                    const qwm_tensor * resid, qwm_tensor * out, void * workspace, size_t ws_bytes, void * stream) {
    return guard("qwm_moe_experts", [&]() -> int {
        if (!x) return fail(QWM_ERR_ARG, "moe_experts: x is NULL");
        MoePlan p;
        int rc = check_layer(layer, x->ne[1], p);
        if (rc != QWM_OK) return rc;
        if ((rc = check_act(x, p.H, "x")) != QWM_OK) return rc;
        if ((rc = check_act(out, p.H, "out")) != QWM_OK) return rc;
        if (out->ne[1] != p.T) return fail(QWM_ERR_ARG, "moe_experts: out must be [H, T]");
        if (resid && ((rc = check_act(resid, p.H, "resid")) != QWM_OK || resid->ne[1] != p.T))
            return rc != QWM_OK ? rc : fail(QWM_ERR_ARG, "moe_experts: resid must be [H, T]");
        const qwm_tensor * slots[3] = {slot_g, slot_u, slot_d};
        for (const qwm_tensor * sl : slots)
            if (!sl || sl->type != T_I32 || sl->ne[0] != p.k || sl->ne[1] != p.T || !fully_contiguous(sl))
                return fail(QWM_ERR_ARG, "moe_experts: slot ids must be contiguous i32 [k, T]");
        if (!weights || weights->type != T_F32 || weights->ne[0] != p.k || weights->ne[1] != p.T || !fully_contiguous(weights))
            return fail(QWM_ERR_ARG, "moe_experts: weights must be contiguous f32 [k, T]");
        if (!workspace || ws_bytes < p.total) return fail(QWM_ERR_WORKSPACE, "moe_experts: workspace too small");
        return do_experts(layer, p, (const int32_t *)slot_g->data, (const int32_t *)slot_u->data,
                          (const int32_t *)slot_d->data, (const float *)weights->data,
                          resid ? (const float *)resid->data : nullptr, (float *)out->data, (uint8_t *)workspace,
                          (hipStream_t)stream);
    });
}

static int block_resident(const qwm_moe_layer * layer, int32_t layer_index, const int32_t * slot_tables,
                          int64_t table_stride, const qwm_tensor * x, const qwm_tensor * rm, const qwm_tensor * resid,
                          qwm_tensor * out, qwm_tensor * ids_out, qwm_tensor * w_out, void * workspace,
                          size_t ws_bytes, void * stream, const uint32_t * res_bits, int32_t * res_flag) {
    if (!x) return fail(QWM_ERR_ARG, "moe_block: x is NULL");
    if (!slot_tables) return fail(QWM_ERR_ARG, "moe_block: slot tables are NULL");
    MoePlan p;
    int rc = check_layer(layer, x->ne[1], p);
    if (rc != QWM_OK) return rc;
    if ((rc = check_act(x, p.H, "x")) != QWM_OK) return rc;
    if ((rc = check_act(out, p.H, "out")) != QWM_OK) return rc;
    if (out->ne[1] != p.T) return fail(QWM_ERR_ARG, "moe_block: out must be [H, T]");
    if (resid && ((rc = check_act(resid, p.H, "resid")) != QWM_OK || resid->ne[1] != p.T))
        return rc != QWM_OK ? rc : fail(QWM_ERR_ARG, "moe_block: resid must be [H, T]");
    if (rm && (rm->type != T_F32 || rm->ne[0] != p.E || rm->ne[1] != p.T || !fully_contiguous(rm)))
        return fail(QWM_ERR_ARG, "moe_block: rm must be contiguous f32 [E, T]");
    if (ids_out && (ids_out->type != T_I32 || ids_out->ne[0] != p.k || ids_out->ne[1] != p.T || ids_out->nb[0] != 4))
        return fail(QWM_ERR_ARG, "moe_block: ids_out must be i32 [k, T]");
    if (w_out && (w_out->type != T_F32 || w_out->ne[0] != p.k || w_out->ne[1] != p.T || w_out->nb[0] != 4))
        return fail(QWM_ERR_ARG, "moe_block: w_out must be f32 [k, T]");
    if (table_stride < (int64_t)(layer_index + 1) * p.E) return fail(QWM_ERR_ARG, "moe_block: slot table stride too small");
    if (!workspace || ws_bytes < p.total) return fail(QWM_ERR_WORKSPACE, "moe_block: workspace too small");
    uint8_t * ws = (uint8_t *)workspace;
    hipStream_t s = (hipStream_t)stream;
    rc = do_route(layer, p, x, rm, slot_tables, table_stride, layer_index,
                  ids_out ? (int32_t *)ids_out->data : nullptr, ids_out ? (int64_t)(ids_out->nb[1] / 4) : 0,
                  w_out ? (float *)w_out->data : nullptr, w_out ? (int64_t)(w_out->nb[1] / 4) : 0, ws, s,
                  res_bits, res_flag);
    if (rc != QWM_OK) return rc;
    const int64_t P = p.T * p.k;
    const int32_t * slots = (const int32_t *)(ws + p.slots);
    return do_experts(layer, p, slots, slots + P, slots + 2 * P, (const float *)(ws + p.w),
                      resid ? (const float *)resid->data : nullptr, (float *)out->data, ws, s,
                      (const int32_t *)(ws + p.uslot));
}

int qwm_moe_block_resident(const qwm_moe_layer * layer, int32_t layer_index, const int32_t * slot_tables,
                           int64_t table_stride, const qwm_tensor * x, const qwm_tensor * rm,
                           const qwm_tensor * resid, qwm_tensor * out, qwm_tensor * ids_out, qwm_tensor * w_out,
                           void * workspace, size_t ws_bytes, void * stream) {
    return guard("qwm_moe_block_resident", [&]() -> int {
        return block_resident(layer, layer_index, slot_tables, table_stride, x, rm, resid, out, ids_out, w_out, workspace,
                              ws_bytes, stream, nullptr, nullptr);
    });
}

// ------------------------------------------------------------ layer loop --

// The decode loop over stacked MoE blocks (decode_cached's per-layer segment B,
// runtime.cpp:5064-5888, in the resident form of 2759-2787 / 5792-5841): each
// layer's block reads the previous layer's output as input and residual.  The
// workspace holds one MoE workspace, reused by every layer in stream order,
// and a ping-pong activation buffer.
static int check_layers(const qwm_moe_layer * layers, int32_t n_layers, int64_t T, MoePlan & p) {
    if (!layers || n_layers < 1) return fail(QWM_ERR_ARG, "moe_decode: no layers");
    int rc = check_layer(&layers[0], T, p);
    if (rc != QWM_OK) return rc;
    for (int32_t l = 1; l < n_layers; ++l) {
        MoePlan q;
        if ((rc = check_layer(&layers[l], T, q)) != QWM_OK) return rc;
        if (q.H != p.H || q.N != p.N || q.E != p.E || q.k != p.k || q.shared != p.shared || q.N_sh != p.N_sh)
            return fail(QWM_ERR_ARG, "moe_decode: layers must share one shape");
    }
    return QWM_OK;
}

// ---------------------------------------------------- cached layer step --
// decode_cached's per-layer expert path (runtime.cpp:5292-5341): route on the
// device, the ids read back (synchronous), the pool's decisions and copies,
// the slot ids uploaded, the compute stream waiting for the copies, the
// experts on the slot ids.  Workspace: the MoE workspace, then ids [T k] i32,
// weights [T k] f32 and slots [3][T k] i32.
static size_t cached_extra(const MoePlan & p) {
    const size_t n = (size_t)(p.T * p.k);
    return align_up(4 * n, 256) * 2 + align_up(12 * n, 256);
}

size_t qwm_moe_cached_workspace_size(const qwm_moe_layer * layer, int64_t T) {
    return guard_size("qwm_moe_cached_workspace_size", [&]() -> size_t {
        MoePlan p;
        if (check_layer(layer, T, p) != QWM_OK) return 0;
        return align_up(p.total, 256) + cached_extra(p);
    });
}

int qwm_moe_cached_step(const qwm_moe_layer * layer, qwm_pool * pool, int32_t layer_index, const qwm_tensor * x,
                        const qwm_tensor * rm, const qwm_tensor * resid, qwm_tensor * out, int32_t * ids_host,
                        void * workspace, size_t ws_bytes, void * stream) {
    return guard("qwm_moe_cached_step", [&]() -> int {
        if (!pool || !x || !out) return fail(QWM_ERR_ARG, "moe_cached_step: NULL argument");
        MoePlan p;
        int rc = check_layer(layer, x->ne[1], p);
        if (rc != QWM_OK) return rc;
        if (layer_index < 0 || layer_index >= pool_n_layer(pool) || pool_n_expert(pool) != p.E)
            return fail(QWM_ERR_ARG, "moe_cached_step: layer index or expert count disagrees with the pool");
        const qwm_tensor * const lt[3] = {&layer->gate_pool, &layer->up_pool, &layer->down_pool};
        if ((rc = pool_check_layer(pool, layer_index, lt, "moe_cached_step")) != QWM_OK) return rc;
        const size_t base = align_up(p.total, 256);
        if (!workspace || ws_bytes < base + cached_extra(p)) return fail(QWM_ERR_WORKSPACE, "moe_cached_step: workspace too small");
        const int64_t n = p.T * p.k;
        uint8_t * ws = (uint8_t *)workspace;
        int32_t * d_ids = (int32_t *)(ws + base);
        float * d_w = (float *)(ws + base + align_up(4 * (size_t)n, 256));
        int32_t * d_sl = (int32_t *)(ws + base + 2 * align_up(4 * (size_t)n, 256));
        hipStream_t s = (hipStream_t)stream;
        qwm_tensor t_ids, t_w, t_sl[3];
        qwm_tensor_init(&t_ids, QWM_TYPE_I32, p.k, p.T, 1, d_ids);
        qwm_tensor_init(&t_w, QWM_TYPE_F32, p.k, p.T, 1, d_w);
        for (int r = 0; r < 3; ++r) qwm_tensor_init(&t_sl[r], QWM_TYPE_I32, p.k, p.T, 1, d_sl + r * n);
        if ((rc = qwm_moe_route(layer, x, rm, &t_ids, &t_w, ws, p.total, stream)) != QWM_OK) return rc;
        std::vector<int32_t> ids((size_t)n), sl((size_t)(3 * n));
        QWM_HIP_CHECK(hipMemcpyAsync(ids.data(), d_ids, 4 * (size_t)n, hipMemcpyDeviceToHost, s));
        QWM_HIP_CHECK(hipStreamSynchronize(s));
        if (ids_host) std::copy(ids.begin(), ids.end(), ids_host);
        if ((rc = qwm_pool_ensure(pool, layer_index, ids.data(), (int32_t)n, sl.data(), sl.data() + n, sl.data() + 2 * n)) != QWM_OK)
            return rc;
        QWM_HIP_CHECK(hipMemcpyAsync(d_sl, sl.data(), 12 * (size_t)n, hipMemcpyHostToDevice, s));
        if ((rc = qwm_pool_wait(pool, stream)) != QWM_OK) return rc;
        return qwm_moe_experts(layer, x, &t_sl[0], &t_sl[1], &t_sl[2], &t_w, resid, out, ws, p.total, stream);
    });
}

// ------------------------------------------------------ batched layer --
// decode_cached_batch's per-layer path for a batch of tokens (runtime.cpp:
// 4509-4572 with plan_slices / ensure_slice, 4639-4698): the router over the
// batch in groups of MAX_T tokens, the ids read back, the slices planned on
// the pool, then per slice ensure + slot upload + the expert MUL_MAT_IDs,
// SwiGLU, the k-ordered weighted sum, the shared expert and the residual.
static bool overlaps(const qwm_tensor * a, const qwm_tensor * b);

struct BatchPlan {
    MoePlan route;                   // one router group (<= MAX_T tokens)
    int64_t T = 0, S = 0;            // batch length, longest slice
    size_t route_ws = 0, ids = 0, w = 0, slots = 0, zeros = 0, shg = 0;
    size_t gate = 0, up = 0, act = 0, ex = 0, sh_g = 0, sh_u = 0, sh_act = 0, sh_out = 0, mmid = 0, mmid_bytes = 0;
    size_t total = 0;
};

static size_t mmid_need(const qwm_tensor & as, int64_t K, int64_t ne11, int64_t n_ids, int64_t T) {
    qwm_tensor b, ids;
    qwm_tensor_init(&b, QWM_TYPE_F32, K, ne11, T, (void *)64);
    qwm_tensor_init(&ids, QWM_TYPE_I32, n_ids, T, 1, (void *)64);
    return qwm_mul_mat_id_workspace_size(&as, &b, &ids);
}

static int batch_plan(const qwm_moe_layer * L, int64_t T, int32_t max_slice, BatchPlan & b) {
    if (T < 1 || T > QWM_BATCH_MAX_T) return fail(QWM_ERR_UNSUPPORTED, "moe_batch: 1 <= T <= 4096");
    if (max_slice < 0) return fail(QWM_ERR_ARG, "moe_batch: max_slice must be >= 0");
    int rc = check_layer(L, std::min<int64_t>(T, MAX_T), b.route);
    if (rc != QWM_OK) return rc;
    const MoePlan & p = b.route;
    b.T = T;
    b.S = std::min<int64_t>(T, max_slice ? max_slice : 1024);
    const int64_t S = b.S, k = p.k, H = p.H, N = p.N, Nsh = p.N_sh;
    // the MUL_MAT_ID workspaces at the longest slice and at the GEMV width
    size_t mm = 0;
    for (int64_t t : {S, std::min<int64_t>(S, MAX_T)}) {
        const size_t need[3] = {mmid_need(L->gate_pool, H, 1, k, t), mmid_need(L->up_pool, H, 1, k, t),
                                mmid_need(L->down_pool, N, k, k, t)};
        for (size_t v : need) {
            if (!v) return fail(QWM_ERR_UNSUPPORTED, std::string("moe_batch: expert MUL_MAT_ID: ") + qwm_last_error());
            mm = std::max(mm, v);
        }
        if (p.shared) {
            qwm_tensor g = L->sh_gate, u = L->sh_up, d = L->sh_down;
            g.ne[2] = u.ne[2] = d.ne[2] = 1;
            const size_t sh[3] = {mmid_need(g, H, 1, 1, t), mmid_need(u, H, 1, 1, t), mmid_need(d, Nsh, 1, 1, t)};
            for (size_t v : sh) {
                if (!v) return fail(QWM_ERR_UNSUPPORTED, std::string("moe_batch: shared expert: ") + qwm_last_error());
                mm = std::max(mm, v);
            }
        }
    }
    size_t o = 0;
    auto take = [&](size_t bytes) { size_t at = o; o = align_up(o + bytes, 256); return at; };
    b.route_ws = take(p.total);
    b.ids = take(4 * (size_t)(k * T));
    b.w = take(4 * (size_t)(k * T));
    b.slots = take(12 * (size_t)(k * T));
    b.zeros = take(4 * (size_t)S);
    b.shg = take(4 * (size_t)T);
    b.gate = take(4 * (size_t)(N * k * S));
    b.up = take(4 * (size_t)(N * k * S));
    b.act = take(4 * (size_t)(N * k * S));
    b.ex = take(4 * (size_t)(H * k * S));
    if (p.shared) {
        b.sh_g = take(4 * (size_t)(Nsh * S));
        b.sh_u = take(4 * (size_t)(Nsh * S));
        b.sh_act = take(4 * (size_t)(Nsh * S));
        b.sh_out = take(4 * (size_t)(H * S));
    }
    b.mmid = take(mm);
    b.mmid_bytes = mm;
    b.total = o;
    return QWM_OK;
}

size_t qwm_moe_cached_batch_workspace_size(const qwm_moe_layer * layer, int64_t T, int32_t max_slice) {
    return guard_size("qwm_moe_cached_batch_workspace_size", [&]() -> size_t {
        BatchPlan b;
        return batch_plan(layer, T, max_slice, b) == QWM_OK ? b.total : 0;
    });
}

int qwm_moe_cached_batch(const qwm_moe_layer * layer, qwm_pool * pool, int32_t layer_index, const qwm_tensor * x,
                         const qwm_tensor * rm, const qwm_tensor * resid, qwm_tensor * out, int32_t max_slice,
                         int32_t * ids_host, int32_t * slices_host, int32_t * n_slices, void * workspace,
                         size_t ws_bytes, void * stream) {
    return guard("qwm_moe_cached_batch", [&]() -> int {
        if (!pool || !x || !out) return fail(QWM_ERR_ARG, "moe_batch: NULL argument");
        BatchPlan b;
        int rc = batch_plan(layer, x->ne[1], max_slice, b);
        if (rc != QWM_OK) return rc;
        const MoePlan & p = b.route;
        const int64_t T = b.T, k = p.k, H = p.H, N = p.N, E = p.E;
        if ((rc = check_act(x, H, "x")) != QWM_OK) return rc;
        if ((rc = check_act(out, H, "out")) != QWM_OK) return rc;
        if (out->ne[1] != T) return fail(QWM_ERR_ARG, "moe_batch: out must be [H, T]");
        if (resid && ((rc = check_act(resid, H, "resid")) != QWM_OK || resid->ne[1] != T))
            return rc != QWM_OK ? rc : fail(QWM_ERR_ARG, "moe_batch: resid must be [H, T]");
        if (overlaps(out, x)) return fail(QWM_ERR_ARG, "moe_batch: out must not overlap x");
        if (rm && (rm->type != T_F32 || rm->ne[0] != E || rm->ne[1] != T || !fully_contiguous(rm)))
            return fail(QWM_ERR_ARG, "moe_batch: rm must be contiguous f32 [E, T]");
        if (layer_index < 0 || layer_index >= pool_n_layer(pool) || pool_n_expert(pool) != E)
            return fail(QWM_ERR_ARG, "moe_batch: layer index or expert count disagrees with the pool");
        const qwm_tensor * const lt[3] = {&layer->gate_pool, &layer->up_pool, &layer->down_pool};
        if ((rc = pool_check_layer(pool, layer_index, lt, "moe_batch")) != QWM_OK) return rc;
        if (!workspace || ws_bytes < b.total) return fail(QWM_ERR_WORKSPACE, "moe_batch: workspace too small");
        uint8_t * ws = (uint8_t *)workspace;
        hipStream_t s = (hipStream_t)stream;
        int32_t * d_ids = (int32_t *)(ws + b.ids);
        float * d_w = (float *)(ws + b.w);
        int32_t * d_sl = (int32_t *)(ws + b.slots);
        float * d_shg = (float *)(ws + b.shg);
        const float * xd = (const float *)x->data;

        // the router, MAX_T tokens at a time (the route workspace is cleared
        // whenever the group's shape changes: its counters sit at shape-dependent
        // places)
        int64_t prev_n = -1;
        for (int64_t t0 = 0; t0 < T; t0 += MAX_T) {
            const int64_t n = std::min<int64_t>(MAX_T, T - t0);
            MoePlan pg;
            if ((rc = check_layer(layer, n, pg)) != QWM_OK) return rc;
            if (n != prev_n && (rc = launch_fill_zero(ws + b.route_ws, pg.total & ~(size_t)3, s)) != QWM_OK) return rc;
            prev_n = n;
            qwm_tensor xg, rg;
            qwm_tensor_init(&xg, QWM_TYPE_F32, H, n, 1, (void *)(xd + t0 * H));
            if (rm) qwm_tensor_init(&rg, QWM_TYPE_F32, E, n, 1, (float *)rm->data + t0 * E);
            if ((rc = do_route(layer, pg, &xg, rm ? &rg : nullptr, nullptr, 0, 0, d_ids + t0 * k, k, d_w + t0 * k, k,
                               ws + b.route_ws, s)) != QWM_OK)
                return rc;
        }
        const bool sh_gate = p.shared && layer->sh_gate_inp.data;
        if (sh_gate && (rc = launch_sh_gate((const float *)layer->sh_gate_inp.data, xd, d_shg, (int)H, (int)T, s)) != QWM_OK)
            return rc;
        if (p.shared && (rc = launch_fill_zero(ws + b.zeros, 4 * (size_t)b.S, s)) != QWM_OK) return rc;

        // the routed ids on the host (synchronizes the stream, as the
        // reference's read of `selected` does)
        std::vector<int32_t> ids((size_t)(k * T)), sl((size_t)(3 * k * T)), slices((size_t)(2 * T));
        QWM_HIP_CHECK(hipMemcpyAsync(ids.data(), d_ids, 4 * ids.size(), hipMemcpyDeviceToHost, s));
        QWM_HIP_CHECK(hipStreamSynchronize(s));
        if (ids_host) std::copy(ids.begin(), ids.end(), ids_host);
        int32_t ns = 0;
        if ((rc = qwm_pool_plan_slices(pool, layer_index, ids.data(), (int32_t)T, (int32_t)k, max_slice, slices.data(), &ns,
                                       nullptr)) != QWM_OK)
            return rc;
        if (slices_host) std::copy(slices.begin(), slices.begin() + 2 * ns, slices_host);
        if (n_slices) *n_slices = ns;

        auto mmid = [&](const qwm_tensor & as, const float * bdata, int64_t K, int64_t ne11, const int32_t * idd,
                        int64_t n_ids, int64_t len, float * dst, int64_t Nout) {
            qwm_tensor bt, it, dt;
            qwm_tensor_init(&bt, QWM_TYPE_F32, K, ne11, len, (void *)bdata);
            qwm_tensor_init(&it, QWM_TYPE_I32, n_ids, len, 1, (void *)idd);
            qwm_tensor_init(&dt, QWM_TYPE_F32, Nout, n_ids, len, dst);
            return qwm_mul_mat_id(&as, &bt, &it, &dt, ws + b.mmid, b.mmid_bytes, s);
        };
        // the fused gate/up pass: both pools in one layout that the grouped GEMM takes
        bool fuse_gate_up = layer->gate_pool.type == layer->up_pool.type;
        for (int i = 0; i < 4 && fuse_gate_up; ++i)
            fuse_gate_up = layer->gate_pool.ne[i] == layer->up_pool.ne[i] && layer->gate_pool.nb[i] == layer->up_pool.nb[i];
        float * gbuf = (float *)(ws + b.gate);
        float * ubuf = (float *)(ws + b.up);
        float * abuf = (float *)(ws + b.act);
        float * ebuf = (float *)(ws + b.ex);
        for (int32_t si = 0; si < ns; ++si) {
            const int64_t t0 = slices[2 * si], len = slices[2 * si + 1];
            // ensure_slice (runtime.cpp:4690-4698); before it, the previous
            // slice's kernels must be done with the slots ensure may recycle
            if (si > 0) QWM_HIP_CHECK(hipStreamSynchronize(s));
            const size_t off = (size_t)(t0 * k), cnt = (size_t)(len * k);
            int32_t * sg = sl.data() + off, * su = sl.data() + k * T + off, * sd = sl.data() + 2 * k * T + off;
            if ((rc = qwm_pool_ensure(pool, layer_index, ids.data() + off, (int32_t)cnt, sg, su, sd)) != QWM_OK) return rc;
            int32_t * dsg = d_sl + off, * dsu = d_sl + k * T + off, * dsd = d_sl + 2 * k * T + off;
            QWM_HIP_CHECK(hipMemcpyAsync(dsg, sg, 4 * cnt, hipMemcpyHostToDevice, s));
            QWM_HIP_CHECK(hipMemcpyAsync(dsu, su, 4 * cnt, hipMemcpyHostToDevice, s));
            QWM_HIP_CHECK(hipMemcpyAsync(dsd, sd, 4 * cnt, hipMemcpyHostToDevice, s));
            if ((rc = qwm_pool_wait(pool, stream)) != QWM_OK) return rc;
            const float * xs = xd + t0 * H;
            qwm_tensor xb;
            qwm_tensor_init(&xb, QWM_TYPE_F32, H, 1, len, (void *)xs);
            if (fuse_gate_up && swiglu_fused(&layer->gate_pool, &layer->up_pool, &xb) &&
                std::memcmp(sg, su, 4 * cnt) == 0) {
                // gate and up rows under the same slots: one grouped pass writes act (equal, bit
                // for bit, to the two calls and SwiGLU below; same workspace as one prefill call)
                qwm_tensor bt, it, at;
                qwm_tensor_init(&bt, QWM_TYPE_F32, H, 1, len, (void *)xs);
                qwm_tensor_init(&it, QWM_TYPE_I32, k, len, 1, (void *)dsg);
                qwm_tensor_init(&at, QWM_TYPE_F32, N, k, len, abuf);
                if ((rc = qwm_mul_mat_id_swiglu(&layer->gate_pool, &layer->up_pool, &bt, &it, &at, ws + b.mmid,
                                                b.mmid_bytes, s)) != QWM_OK)
                    return rc;
            } else {
                if ((rc = mmid(layer->up_pool, xs, H, 1, dsu, k, len, ubuf, N)) != QWM_OK) return rc;
                if ((rc = mmid(layer->gate_pool, xs, H, 1, dsg, k, len, gbuf, N)) != QWM_OK) return rc;
                if ((rc = launch_swiglu_rows(gbuf, ubuf, abuf, (int)N, k * len, s)) != QWM_OK) return rc;
            }
            if ((rc = mmid(layer->down_pool, abuf, N, k, dsd, k, len, ebuf, H)) != QWM_OK) return rc;
            const float * shout = nullptr;
            if (p.shared) {
                qwm_tensor g = layer->sh_gate, u = layer->sh_up, d = layer->sh_down;
                g.ne[2] = u.ne[2] = d.ne[2] = 1;
                const int32_t * z = (const int32_t *)(ws + b.zeros);
                float * shg_b = (float *)(ws + b.sh_g), * shu_b = (float *)(ws + b.sh_u);
                float * sha_b = (float *)(ws + b.sh_act), * sho_b = (float *)(ws + b.sh_out);
                if ((rc = mmid(g, xs, H, 1, z, 1, len, shg_b, p.N_sh)) != QWM_OK) return rc;
                if ((rc = mmid(u, xs, H, 1, z, 1, len, shu_b, p.N_sh)) != QWM_OK) return rc;
                if ((rc = launch_swiglu_rows(shg_b, shu_b, sha_b, (int)p.N_sh, len, s)) != QWM_OK) return rc;
                if ((rc = mmid(d, sha_b, p.N_sh, 1, z, 1, len, sho_b, H)) != QWM_OK) return rc;
                shout = sho_b;
            }
            if ((rc = launch_combine_batch(ebuf, d_w + t0 * k, shout, sh_gate ? d_shg + t0 : nullptr,
                                           resid ? (const float *)resid->data + t0 * H : nullptr,
                                           (float *)out->data + t0 * H, (int)H, (int)k, len, s)) != QWM_OK)
                return rc;
        }
        return QWM_OK;
    });
}

size_t qwm_moe_decode_workspace_size(const qwm_moe_layer * layers, int32_t n_layers, int64_t T) {
    return guard_size("qwm_moe_decode_workspace_size", [&]() -> size_t {
        MoePlan p;
        if (check_layers(layers, n_layers, T, p) != QWM_OK) return 0;
        const size_t loop = align_up(p.total, 256) + align_up(sizeof(float) * (size_t)(T * p.H), 256);
        DecodePlan dp;
        std::string why;
        return decode_plan(layers, n_layers, T, dp, why) ? std::max(loop, dp.total) : loop;
    });
}

int qwm_moe_decode(const qwm_moe_layer * layers, int32_t n_layers, const int32_t * slot_tables, int64_t table_stride,
                   qwm_tensor * x, void * workspace, size_t ws_bytes, void * stream) {
    return guard("qwm_moe_decode", [&]() -> int {
        return qwm_moe_decode_sel(layers, n_layers, slot_tables, table_stride, x, nullptr, nullptr, nullptr, workspace,
                                  ws_bytes, stream);
    });
}

int qwm_moe_decode_sel(const qwm_moe_layer * layers, int32_t n_layers, const int32_t * slot_tables,
                       int64_t table_stride, qwm_tensor * x, int32_t * ids_all, const uint32_t * resident_bits,
                       int32_t * miss_flag, void * workspace, size_t ws_bytes, void * stream) {
    return guard("qwm_moe_decode_sel", [&]() -> int {
        if (!x) return fail(QWM_ERR_ARG, "moe_decode: x is NULL");
        if (resident_bits && !miss_flag) return fail(QWM_ERR_ARG, "moe_decode: resident_bits needs miss_flag");
        if (!slot_tables) return fail(QWM_ERR_ARG, "moe_decode: slot tables are NULL");
        MoePlan p;
        int rc = check_layers(layers, n_layers, x->ne[1], p);
        if (rc != QWM_OK) return rc;
        if ((rc = check_act(x, p.H, "x")) != QWM_OK) return rc;
        if (table_stride < (int64_t)n_layers * p.E) return fail(QWM_ERR_ARG, "moe_decode: slot table stride too small");
        DecodePlan dp;
        std::string why;
        const bool persistent = decode_plan(layers, n_layers, p.T, dp, why);
        const size_t loop = align_up(p.total, 256) + align_up(sizeof(float) * (size_t)(p.T * p.H), 256);
        const size_t need = persistent ? std::max(loop, dp.total) : loop;
        if (!workspace || ws_bytes < need) return fail(QWM_ERR_WORKSPACE, "moe_decode: workspace too small");
        uint8_t * ws = (uint8_t *)workspace;
        if (persistent) {   // one launch per group of layers (qwm_decode.hip)
            if (miss_flag && (rc = launch_fill_zero(miss_flag, 4, (hipStream_t)stream)) != QWM_OK) return rc;
            DecodeCall c{layers, n_layers, slot_tables, table_stride, (float *)x->data, ids_all, resident_bits,
                         miss_flag};
            return launch_decode(c, dp, ws, (hipStream_t)stream);
        }
        qwm_tensor buf = *x;
        buf.data = ws + align_up(p.total, 256);
        hipStream_t s = (hipStream_t)stream;
        if (miss_flag && (rc = launch_fill_zero(miss_flag, 4, s)) != QWM_OK) return rc;
        const int64_t words = (p.E + 31) / 32;
        for (int32_t l = 0; l < n_layers; ++l) {
            qwm_tensor * src = (l & 1) ? &buf : x;
            qwm_tensor * dst = (l & 1) ? x : &buf;
            qwm_tensor ids_l;
            if (ids_all) qwm_tensor_init(&ids_l, QWM_TYPE_I32, p.k, p.T, 1, ids_all + (size_t)l * p.k * p.T);
            rc = block_resident(&layers[l], l, slot_tables, table_stride, src, nullptr, src, dst, ids_all ? &ids_l : nullptr,
                                nullptr, ws, p.total, s, resident_bits ? resident_bits + (size_t)l * words : nullptr,
                                miss_flag);
            if (rc != QWM_OK) return rc;
        }
        if (n_layers & 1)
            QWM_HIP_CHECK(hipMemcpyAsync(x->data, buf.data, sizeof(float) * (size_t)(p.T * p.H), hipMemcpyDeviceToDevice, s));
        return QWM_OK;
    });
}

// -------------------------------------------------------------- fused step --

size_t qwm_verify_step_workspace_size(const qwm_moe_layer * layer, const qwm_tensor * lm_head, int64_t T) {
    return guard_size("qwm_verify_step_workspace_size", [&]() -> size_t {
        MoePlan m;
        StepPlan p;
        std::string why;
        if (!lm_head || check_layer(layer, T, m) != QWM_OK || !step_plan(layer, lm_head, T, p, why)) return 0;
        return p.total;
    });
}

static bool overlaps(const qwm_tensor * a, const qwm_tensor * b) {
    const uintptr_t a0 = (uintptr_t)a->data, a1 = a0 + a->nb[3] * (size_t)a->ne[3];
    const uintptr_t b0 = (uintptr_t)b->data, b1 = b0 + b->nb[3] * (size_t)b->ne[3];
    return a0 < b1 && b0 < a1;
}

int qwm_verify_step(const qwm_moe_layer * layer, int32_t layer_index, const int32_t * slot_tables,
                    int64_t table_stride, const qwm_tensor * x, const qwm_tensor * rm, const qwm_tensor * resid,
                    qwm_tensor * out, qwm_tensor * ids_out, qwm_tensor * w_out, const qwm_tensor * lm_head,
                    const float * norm_w, float eps, const int32_t * drafts, int32_t * result,
                    void * workspace, size_t ws_bytes, void * stream) {
    return guard("qwm_verify_step", [&]() -> int {
        if (!x || !lm_head || !result) return fail(QWM_ERR_ARG, "verify_step: NULL argument");
        if (!slot_tables) return fail(QWM_ERR_ARG, "verify_step: slot tables are NULL");
        MoePlan m;
        int rc = check_layer(layer, x->ne[1], m);
        if (rc != QWM_OK) return rc;
        StepPlan p;
        std::string why;
        if (!step_plan(layer, lm_head, x->ne[1], p, why)) return fail(QWM_ERR_UNSUPPORTED, "verify_step: " + why);
        if ((rc = check_act(x, p.moe.H, "x")) != QWM_OK) return rc;
        if ((rc = check_act(out, p.moe.H, "out")) != QWM_OK) return rc;
        if (out->ne[1] != p.moe.T) return fail(QWM_ERR_ARG, "verify_step: out must be [H, T]");
        if (resid && ((rc = check_act(resid, p.moe.H, "resid")) != QWM_OK || resid->ne[1] != p.moe.T))
            return rc != QWM_OK ? rc : fail(QWM_ERR_ARG, "verify_step: resid must be [H, T]");
        if (overlaps(out, x) || (resid && overlaps(out, resid)))
            return fail(QWM_ERR_ARG, "verify_step: out must not overlap x or resid");
        if (rm && (rm->type != T_F32 || rm->ne[0] != p.moe.E || rm->ne[1] != p.moe.T || !fully_contiguous(rm)))
            return fail(QWM_ERR_ARG, "verify_step: rm must be contiguous f32 [E, T]");
        if (ids_out && (ids_out->type != T_I32 || ids_out->ne[0] != p.moe.k || ids_out->ne[1] != p.moe.T || ids_out->nb[0] != 4))
            return fail(QWM_ERR_ARG, "verify_step: ids_out must be i32 [k, T]");
        if (w_out && (w_out->type != T_F32 || w_out->ne[0] != p.moe.k || w_out->ne[1] != p.moe.T || w_out->nb[0] != 4))
            return fail(QWM_ERR_ARG, "verify_step: w_out must be f32 [k, T]");
        if (table_stride < (int64_t)(layer_index + 1) * p.moe.E) return fail(QWM_ERR_ARG, "verify_step: slot table stride too small");
        if (!contiguous_rows(lm_head)) return fail(QWM_ERR_UNSUPPORTED, "verify_step: lm_head rows must be contiguous");
        if ((uintptr_t)lm_head->data % 4 || (uintptr_t)norm_w % 16) return fail(QWM_ERR_ARG, "verify_step: misaligned lm_head or norm_w");
        if (p.moe.T > 1 && !drafts) return fail(QWM_ERR_ARG, "verify_step: drafts are NULL");
        if (!workspace || ws_bytes < p.total) return fail(QWM_ERR_WORKSPACE, "verify_step: workspace too small");
        StepCall c;
        c.L = layer; c.layer = layer_index; c.slot_tables = slot_tables; c.table_stride = table_stride;
        c.x = (const float *)x->data; c.rm = rm ? (const float *)rm->data : nullptr;
        c.resid = resid ? (const float *)resid->data : nullptr; c.out = (float *)out->data;
        c.ids_out = ids_out ? (int32_t *)ids_out->data : nullptr; c.ids_ld = ids_out ? (int64_t)(ids_out->nb[1] / 4) : 0;
        c.w_out = w_out ? (float *)w_out->data : nullptr; c.w_ld = w_out ? (int64_t)(w_out->nb[1] / 4) : 0;
        c.lm_head = (const uint8_t *)lm_head->data; c.norm_w = norm_w; c.eps = eps; c.drafts = drafts; c.result = result;
        return launch_step(c, p, (uint8_t *)workspace, (hipStream_t)stream);
    });
}

// ------------------------------------------------------------------ verify --

size_t qwm_verify_workspace_size(const qwm_tensor * lm_head, int64_t T) {
    return guard_size("qwm_verify_workspace_size", [&]() -> size_t {
        VerifyPlan p;
        std::string why;
        if (!lm_head || !verify_plan(lm_head, T, p, why)) return 0;
        return p.total;
    });
}

int qwm_verify_accept(const qwm_tensor * lm_head, const qwm_tensor * x, const float * norm_w, float eps,
                      const int32_t * drafts, int32_t * result, void * workspace, size_t ws_bytes, void * stream) {
    return guard("qwm_verify_accept", [&]() -> int {
        if (!lm_head || !x || !result) return fail(QWM_ERR_ARG, "verify: NULL argument");
        VerifyPlan p;
        std::string why;
        if (!verify_plan(lm_head, x->ne[1], p, why)) return fail(QWM_ERR_UNSUPPORTED, "verify: " + why);
        if (!contiguous_rows(lm_head)) return fail(QWM_ERR_UNSUPPORTED, "verify: lm_head rows must be contiguous");
        if (x->type != T_F32 || x->ne[0] != p.H || !fully_contiguous(x)) return fail(QWM_ERR_ARG, "verify: x must be contiguous f32 [H, T]");
        if (p.T > 1 && !drafts) return fail(QWM_ERR_ARG, "verify: drafts are NULL");
        if ((uintptr_t)x->data % 16 || (uintptr_t)norm_w % 16) return fail(QWM_ERR_ARG, "verify: x and norm_w must be 16-byte aligned");
        if ((uintptr_t)lm_head->data % 4) return fail(QWM_ERR_ARG, "verify: lm_head data must be 4-byte aligned");
        if (!workspace || ws_bytes < p.total) return fail(QWM_ERR_WORKSPACE, "verify: workspace too small");
        return launch_verify((const uint8_t *)lm_head->data, (const float *)x->data, norm_w, eps, drafts, result, p,
                             (uint8_t *)workspace, (hipStream_t)stream);
    });
}

}  // extern "C"
