// ggml-qwmoe.cpp -- a ggml backend (backend API v3) whose device runs the MoE
// expert ops on libqwmoe: GGML_OP_MUL_MAT_ID, GGML_OP_GLU (SWIGLU, split form),
// the up / gate / SWIGLU node run of build_segB fused into one
// qwm_mul_mat_id_swiglu call, and the view ops (no work).
//
// The interfaces are those of ggml-backend-impl.h:17-287: a buffer type over
// device memory (hipMalloc), a GPU device (supports_op, supports_buft, events),
// a backend per stream (graph_compute, async tensor copies, events), and a reg
// that a process finds through ggml_backend_load (the exported
// ggml_backend_init, ggml-backend-impl.h:251-287) or ggml_backend_qwmoe_reg().
// Ops outside that set are reported unsupported, so a ggml_backend_sched over
// this device and another places them there.
//
// The backend owns one workspace per stream for the ops that need one, grown
// (synchronously) when a graph needs more; libqwmoe itself allocates nothing.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-qwmoe.h"
#include "qwmoe.h"

namespace {

constexpr size_t QWM_ALIGN = 256;

bool hip_ok(hipError_t e, const char * what) {
    if (e == hipSuccess) return true;
    std::fprintf(stderr, "ggml-qwmoe: %s: %s\n", what, hipGetErrorString(e));
    return false;
}

qwm_tensor to_qwm(const ggml_tensor * t) {
    qwm_tensor q;
    q.type = (int32_t)t->type;                         // the ggml_type values (ggml.h)
    for (int i = 0; i < 4; ++i) { q.ne[i] = t->ne[i]; q.nb[i] = t->nb[i]; }
    q.data = t->data;
    return q;
}

bool is_view_op(const ggml_tensor * t) {
    return t->op == GGML_OP_NONE || t->op == GGML_OP_RESHAPE || t->op == GGML_OP_VIEW || t->op == GGML_OP_PERMUTE ||
           t->op == GGML_OP_TRANSPOSE;
}

// ggml_swiglu_split: GGML_OP_GLU with op_params {GGML_GLU_OP_SWIGLU, swapped = 0} and src[1] set (ggml.c:3082)
bool is_swiglu_split(const ggml_tensor * t) {
    return t->op == GGML_OP_GLU && ggml_get_glu_op(t) == GGML_GLU_OP_SWIGLU && t->src[1] != nullptr &&
           t->op_params[1] == 0;
}

// ------------------------------------------------------------------ buffer --

struct Buffer {
    int device;
    void * dev;
};

void buf_free(ggml_backend_buffer_t b) {
    Buffer * c = (Buffer *)b->context;
    (void)hipSetDevice(c->device);
    (void)hip_ok(hipFree(c->dev), "hipFree");
    delete c;
}

void * buf_base(ggml_backend_buffer_t b) { return ((Buffer *)b->context)->dev; }

void buf_memset(ggml_backend_buffer_t b, ggml_tensor * t, uint8_t v, size_t off, size_t n) {
    (void)hipSetDevice(((Buffer *)b->context)->device);
    if (hip_ok(hipMemset((uint8_t *)t->data + off, v, n), "hipMemset")) (void)hip_ok(hipDeviceSynchronize(), "sync");
}

void buf_set(ggml_backend_buffer_t b, ggml_tensor * t, const void * src, size_t off, size_t n) {
    (void)hipSetDevice(((Buffer *)b->context)->device);
    (void)hip_ok(hipMemcpy((uint8_t *)t->data + off, src, n, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

void buf_get(ggml_backend_buffer_t b, const ggml_tensor * t, void * dst, size_t off, size_t n) {
    (void)hipSetDevice(((Buffer *)b->context)->device);
    (void)hip_ok(hipMemcpy(dst, (const uint8_t *)t->data + off, n, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

bool buf_is_ours(ggml_backend_buffer_t b);

bool buf_cpy(ggml_backend_buffer_t b, const ggml_tensor * src, ggml_tensor * dst) {
    if (!src->buffer || !buf_is_ours(src->buffer)) return false;     // only device-to-device here
    (void)hipSetDevice(((Buffer *)b->context)->device);
    return hip_ok(hipMemcpy(dst->data, src->data, ggml_nbytes(src), hipMemcpyDeviceToDevice), "hipMemcpy D2D");
}

void buf_clear(ggml_backend_buffer_t b, uint8_t v) {
    Buffer * c = (Buffer *)b->context;
    (void)hipSetDevice(c->device);
    if (hip_ok(hipMemset(c->dev, v, b->size), "hipMemset")) (void)hip_ok(hipDeviceSynchronize(), "sync");
}

const ggml_backend_buffer_i buffer_iface = {
    /* .free_buffer   = */ buf_free,
    /* .get_base      = */ buf_base,
    /* .init_tensor   = */ nullptr,
    /* .memset_tensor = */ buf_memset,
    /* .set_tensor    = */ buf_set,
    /* .get_tensor    = */ buf_get,
    /* .set_tensor_2d = */ nullptr,
    /* .get_tensor_2d = */ nullptr,
    /* .cpy_tensor    = */ buf_cpy,
    /* .clear         = */ buf_clear,
    /* .reset         = */ nullptr,
};

bool buf_is_ours(ggml_backend_buffer_t b) { return b->iface.get_base == buffer_iface.get_base; }

// ------------------------------------------------------------- buffer type --

struct Device;

struct BufferType {
    int device;
    std::string name;
};

const char * buft_name(ggml_backend_buffer_type_t t) { return ((BufferType *)t->context)->name.c_str(); }

ggml_backend_buffer_t buft_alloc(ggml_backend_buffer_type_t t, size_t size) {
    const int dev = ((BufferType *)t->context)->device;
    if (!hip_ok(hipSetDevice(dev), "hipSetDevice")) return nullptr;
    void * p = nullptr;
    if (!hip_ok(hipMalloc(&p, size ? size : QWM_ALIGN), "hipMalloc")) return nullptr;
    return ggml_backend_buffer_init(t, buffer_iface, new Buffer{dev, p}, size);
}

size_t buft_alignment(ggml_backend_buffer_type_t) { return QWM_ALIGN; }

bool buft_is_host(ggml_backend_buffer_type_t) { return false; }

const ggml_backend_buffer_type_i buffer_type_iface = {
    /* .get_name         = */ buft_name,
    /* .alloc_buffer     = */ buft_alloc,
    /* .alloc_buffer_n   = */ nullptr,
    /* .get_alignment    = */ buft_alignment,
    /* .get_max_size     = */ nullptr,
    /* .get_alloc_size   = */ nullptr,
    /* .get_alloc_size_n = */ nullptr,
    /* .is_host          = */ buft_is_host,
};

// ----------------------------------------------------------------- backend --

struct Backend {
    int device;
    hipStream_t stream;
    void * ws = nullptr;     // the workspace of the ops that need one (zeroed once per growth)
    size_t ws_bytes = 0;
};

const ggml_guid * backend_guid() {
    static ggml_guid g = {0x71, 0x77, 0x6d, 0x6f, 0x65, 0x2d, 0x67, 0x66, 0x78, 0x39, 0x35, 0x30, 0x2d, 0x76, 0x33, 0x01};
    return &g;
}

const char * be_name(ggml_backend_t) { return "QWMOE"; }

void be_free(ggml_backend_t be) {
    Backend * c = (Backend *)be->context;
    (void)hipSetDevice(c->device);
    (void)hip_ok(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (c->ws) (void)hip_ok(hipFree(c->ws), "hipFree");
    (void)hip_ok(hipStreamDestroy(c->stream), "hipStreamDestroy");
    delete c;
    delete be;
}

void be_set_async(ggml_backend_t be, ggml_tensor * t, const void * src, size_t off, size_t n) {
    Backend * c = (Backend *)be->context;
    (void)hip_ok(hipMemcpyAsync((uint8_t *)t->data + off, src, n, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync");
}

void be_get_async(ggml_backend_t be, const ggml_tensor * t, void * dst, size_t off, size_t n) {
    Backend * c = (Backend *)be->context;
    (void)hip_ok(hipMemcpyAsync(dst, (const uint8_t *)t->data + off, n, hipMemcpyDeviceToHost, c->stream),
                 "hipMemcpyAsync");
}

void be_sync(ggml_backend_t be) {
    Backend * c = (Backend *)be->context;
    (void)hip_ok(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

bool ensure_ws(Backend * c, size_t need) {
    if (need <= c->ws_bytes) return true;
    if (!hip_ok(hipStreamSynchronize(c->stream), "hipStreamSynchronize")) return false;
    if (c->ws) (void)hip_ok(hipFree(c->ws), "hipFree");
    c->ws = nullptr;
    c->ws_bytes = 0;
    need = (need + QWM_ALIGN - 1) / QWM_ALIGN * QWM_ALIGN;
    if (!hip_ok(hipMalloc(&c->ws, need), "hipMalloc")) return false;
    if (qwm_workspace_init(c->ws, need, c->stream) != QWM_OK) return false;
    c->ws_bytes = need;
    return true;
}

// nodes i, i + 1, i + 2 = up, gate, swiglu_split(gate, up) over the same b and
// ids, with up and gate read by nothing else: build_segB's run (runtime.cpp:4539-4541)
bool fusable_gate_up(ggml_cgraph * g, int i, int n) {
    if (i + 2 >= n) return false;
    const ggml_tensor * up = ggml_graph_node(g, i), * gate = ggml_graph_node(g, i + 1), * act = ggml_graph_node(g, i + 2);
    if (up->op != GGML_OP_MUL_MAT_ID || gate->op != GGML_OP_MUL_MAT_ID || !is_swiglu_split(act)) return false;
    if (act->src[0] != gate || act->src[1] != up || gate->src[1] != up->src[1] || gate->src[2] != up->src[2]) return false;
    if ((up->flags | gate->flags) & GGML_TENSOR_FLAG_OUTPUT) return false;
    for (int j = i + 3; j < n; ++j) {
        const ggml_tensor * t = ggml_graph_node(g, j);
        for (int s = 0; s < GGML_MAX_SRC; ++s)
            if (t->src[s] == up || t->src[s] == gate) return false;
    }
    return true;
}

ggml_status be_graph_compute(ggml_backend_t be, ggml_cgraph * g) {
    Backend * c = (Backend *)be->context;
    if (!hip_ok(hipSetDevice(c->device), "hipSetDevice")) return GGML_STATUS_FAILED;
    const int n = ggml_graph_n_nodes(g);
    for (int i = 0; i < n; ++i) {
        ggml_tensor * node = ggml_graph_node(g, i);
        if (is_view_op(node)) continue;
        int rc = QWM_ERR_UNSUPPORTED;
        const char * what = ggml_op_desc(node);
        if (node->op == GGML_OP_MUL_MAT_ID && fusable_gate_up(g, i, n)) {
            ggml_tensor * up = node, * gate = ggml_graph_node(g, i + 1), * act = ggml_graph_node(g, i + 2);
            const qwm_tensor qg = to_qwm(gate->src[0]), qu = to_qwm(up->src[0]), qb = to_qwm(gate->src[1]),
                             qi = to_qwm(gate->src[2]);
            qwm_tensor qa = to_qwm(act);
            const size_t need = qwm_mul_mat_id_swiglu_workspace_size(&qg, &qu, &qb, &qi);
            if (need) {                              // otherwise the three nodes run one by one
                if (!ensure_ws(c, need)) return GGML_STATUS_ALLOC_FAILED;
                rc = qwm_mul_mat_id_swiglu(&qg, &qu, &qb, &qi, &qa, c->ws, c->ws_bytes, c->stream);
                if (rc == QWM_OK) { i += 2; continue; }
                if (rc != QWM_ERR_UNSUPPORTED) {
                    std::fprintf(stderr, "ggml-qwmoe: %s (MUL_MAT_ID + MUL_MAT_ID + SWIGLU): %s\n", act->name,
                                 qwm_last_error());
                    return GGML_STATUS_FAILED;
                }
            }
        }
        if (node->op == GGML_OP_MUL_MAT_ID) {
            const qwm_tensor as = to_qwm(node->src[0]), b = to_qwm(node->src[1]), ids = to_qwm(node->src[2]);
            qwm_tensor dst = to_qwm(node);
            const size_t need = qwm_mul_mat_id_workspace_size(&as, &b, &ids);
            if (need && !ensure_ws(c, need)) return GGML_STATUS_ALLOC_FAILED;
            if (need) rc = qwm_mul_mat_id(&as, &b, &ids, &dst, c->ws, c->ws_bytes, c->stream);
        } else if (is_swiglu_split(node)) {
            const qwm_tensor gt = to_qwm(node->src[0]), ut = to_qwm(node->src[1]);
            qwm_tensor at = to_qwm(node);
            rc = qwm_swiglu(&gt, &ut, &at, c->stream);
        }
        if (rc != QWM_OK) {
            std::fprintf(stderr, "ggml-qwmoe: %s (%s): %s\n", node->name, what,
                         rc == QWM_ERR_UNSUPPORTED && node->op != GGML_OP_MUL_MAT_ID && !is_swiglu_split(node)
                             ? "op not supported by this backend"
                             : qwm_last_error());
            return GGML_STATUS_FAILED;
        }
    }
    return GGML_STATUS_SUCCESS;
}

void be_event_record(ggml_backend_t be, ggml_backend_event_t ev) {
    (void)hip_ok(hipEventRecord((hipEvent_t)ev->context, ((Backend *)be->context)->stream), "hipEventRecord");
}

void be_event_wait(ggml_backend_t be, ggml_backend_event_t ev) {
    (void)hip_ok(hipStreamWaitEvent(((Backend *)be->context)->stream, (hipEvent_t)ev->context, 0), "hipStreamWaitEvent");
}

const ggml_backend_i backend_iface = {
    /* .get_name            = */ be_name,
    /* .free                = */ be_free,
    /* .set_tensor_async    = */ be_set_async,
    /* .get_tensor_async    = */ be_get_async,
    /* .set_tensor_2d_async = */ nullptr,
    /* .get_tensor_2d_async = */ nullptr,
    /* .cpy_tensor_async    = */ nullptr,
    /* .synchronize         = */ be_sync,
    /* .graph_plan_create   = */ nullptr,
    /* .graph_plan_free     = */ nullptr,
    /* .graph_plan_update   = */ nullptr,
    /* .graph_plan_compute  = */ nullptr,
    /* .graph_compute       = */ be_graph_compute,
    /* .event_record        = */ be_event_record,
    /* .event_wait          = */ be_event_wait,
    /* .graph_optimize      = */ nullptr,
};

// ------------------------------------------------------------------ device --

struct Device {
    int device;
    std::string name, description;
    BufferType buft_ctx;
    ggml_backend_buffer_type buft;
};

const char * dev_name(ggml_backend_dev_t d) { return ((Device *)d->context)->name.c_str(); }
const char * dev_description(ggml_backend_dev_t d) { return ((Device *)d->context)->description.c_str(); }

void dev_memory(ggml_backend_dev_t d, size_t * free_b, size_t * total_b) {
    *free_b = *total_b = 0;
    if (hip_ok(hipSetDevice(((Device *)d->context)->device), "hipSetDevice"))
        (void)hip_ok(hipMemGetInfo(free_b, total_b), "hipMemGetInfo");
}

enum ggml_backend_dev_type dev_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }

void dev_props(ggml_backend_dev_t d, ggml_backend_dev_props * p) {
    p->name = dev_name(d);
    p->description = dev_description(d);
    p->type = GGML_BACKEND_DEVICE_TYPE_GPU;
    p->device_id = nullptr;
    dev_memory(d, &p->memory_free, &p->memory_total);
    p->caps.async = true;
    p->caps.host_buffer = false;
    p->caps.buffer_from_host_ptr = false;
    p->caps.events = true;
    p->caps.mmap_support = false;
}

ggml_backend_t dev_init_backend(ggml_backend_dev_t d, const char *) {
    const int dev = ((Device *)d->context)->device;
    if (!hip_ok(hipSetDevice(dev), "hipSetDevice")) return nullptr;
    hipStream_t s = nullptr;
    if (!hip_ok(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags")) return nullptr;
    return new ggml_backend{const_cast<ggml_guid *>(backend_guid()), backend_iface, d, new Backend{dev, s}};
}

ggml_backend_buffer_type_t dev_buffer_type(ggml_backend_dev_t d) { return &((Device *)d->context)->buft; }

bool dev_supports_op(ggml_backend_dev_t, const ggml_tensor * op) {
    if (is_view_op(op)) return true;
    if (op->op == GGML_OP_MUL_MAT_ID) {
        const qwm_tensor as = to_qwm(op->src[0]), b = to_qwm(op->src[1]), ids = to_qwm(op->src[2]);
        return qwm_mul_mat_id_workspace_size(&as, &b, &ids) > 0;
    }
    if (is_swiglu_split(op)) {
        const ggml_tensor * const ts[3] = {op->src[0], op->src[1], op};
        for (const ggml_tensor * t : ts)
            if (t->type != GGML_TYPE_F32 || !ggml_is_contiguous(t) || !ggml_are_same_shape(t, op)) return false;
        return true;
    }
    return false;
}

bool dev_supports_buft(ggml_backend_dev_t d, ggml_backend_buffer_type_t t) { return t == &((Device *)d->context)->buft; }

ggml_backend_event_t dev_event_new(ggml_backend_dev_t d) {
    if (!hip_ok(hipSetDevice(((Device *)d->context)->device), "hipSetDevice")) return nullptr;
    hipEvent_t e = nullptr;
    if (!hip_ok(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreateWithFlags")) return nullptr;
    return new ggml_backend_event{d, e};
}

void dev_event_free(ggml_backend_dev_t, ggml_backend_event_t ev) {
    (void)hip_ok(hipEventDestroy((hipEvent_t)ev->context), "hipEventDestroy");
    delete ev;
}

void dev_event_sync(ggml_backend_dev_t, ggml_backend_event_t ev) {
    (void)hip_ok(hipEventSynchronize((hipEvent_t)ev->context), "hipEventSynchronize");
}

const ggml_backend_device_i device_iface = {
    /* .get_name             = */ dev_name,
    /* .get_description      = */ dev_description,
    /* .get_memory           = */ dev_memory,
    /* .get_type             = */ dev_type,
    /* .get_props            = */ dev_props,
    /* .init_backend         = */ dev_init_backend,
    /* .get_buffer_type      = */ dev_buffer_type,
    /* .get_host_buffer_type = */ nullptr,
    /* .buffer_from_host_ptr = */ nullptr,
    /* .supports_op          = */ dev_supports_op,
    /* .supports_buft        = */ dev_supports_buft,
    /* .offload_op           = */ nullptr,
    /* .event_new            = */ dev_event_new,
    /* .event_free           = */ dev_event_free,
    /* .event_synchronize    = */ dev_event_sync,
};

// --------------------------------------------------------------------- reg --

struct Reg {
    std::vector<Device *> devices;
    std::vector<ggml_backend_device> handles;
};

const char * reg_name(ggml_backend_reg_t) { return "QWMOE"; }
size_t reg_device_count(ggml_backend_reg_t r) { return ((Reg *)r->context)->handles.size(); }
ggml_backend_dev_t reg_device(ggml_backend_reg_t r, size_t i) { return &((Reg *)r->context)->handles[i]; }

const ggml_backend_reg_i reg_iface = {
    /* .get_name         = */ reg_name,
    /* .get_device_count = */ reg_device_count,
    /* .get_device       = */ reg_device,
    /* .get_proc_address = */ nullptr,
};

}  // namespace

ggml_backend_reg_t ggml_backend_qwmoe_reg(void) {
    static ggml_backend_reg reg;
    static std::once_flag once;
    std::call_once(once, [] {
        Reg * r = new Reg;
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
        r->devices.reserve((size_t)n);
        r->handles.reserve((size_t)n);
        for (int i = 0; i < n; ++i) {
            hipDeviceProp_t prop;
            Device * d = new Device;
            d->device = i;
            d->name = "QWMOE" + std::to_string(i);
            d->description = hipGetDeviceProperties(&prop, i) == hipSuccess ? std::string(prop.name) : d->name;
            d->buft_ctx = BufferType{i, d->name};
            r->devices.push_back(d);
            r->handles.push_back(ggml_backend_device{device_iface, &reg, d});
            d->buft = ggml_backend_buffer_type{buffer_type_iface, &r->handles.back(), &d->buft_ctx};
        }
        reg = ggml_backend_reg{GGML_BACKEND_API_VERSION, reg_iface, r};
    });
    return &reg;
}

GGML_BACKEND_DL_IMPL(ggml_backend_qwmoe_reg)
