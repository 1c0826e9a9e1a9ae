// qwm_noalloc.hip -- qwm_verify_step for callers that cannot allocate device
// memory (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc): the step's scratch lives in a file-scope device array instead of
// a caller-provided workspace.
//
// The array is a host-side stand-in in host code: its device address is taken
// once per device with hipGetSymbolAddress (each GPU holds its own copy at its
// own address) and only that address is handed to kernels and fills.  Every
// call clears the part the step uses (a fill kernel, so the call stays
// capturable), which gives the step the zeroed counters it expects; calls that
// overlap on one GPU share the array and race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "qwm_internal.h"

namespace qwm {

static __device__ __align__(256) uint8_t scratch[QWM_NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
static void * g_scratch_ptr[NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

// The device address of `scratch` on the current device (looked up on the
// first call per device, with that device current).
static int scratch_address(void ** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(QWM_ERR_HIP, std::string("verify_step_noalloc: hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return fail(QWM_ERR_UNSUPPORTED, "verify_step_noalloc: device index beyond 63");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void * p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(QWM_ERR_HIP, std::string("verify_step_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return QWM_OK;
}

}  // namespace qwm

using namespace qwm;

extern "C" int qwm_verify_step_noalloc(const qwm_moe_layer * layer, int32_t layer_index, const int32_t * slot_tables,
                                       int64_t table_stride, const qwm_tensor * x, const qwm_tensor * rm,
                                       const qwm_tensor * resid, qwm_tensor * out, qwm_tensor * ids_out,
                                       qwm_tensor * w_out, const qwm_tensor * lm_head, const float * norm_w, float eps,
                                       const int32_t * drafts, int32_t * result, void * stream) {
    return guard("qwm_verify_step_noalloc", [&]() -> int {
        if (!x || !lm_head) return fail(QWM_ERR_ARG, "verify_step_noalloc: NULL argument");
        const size_t need = qwm_verify_step_workspace_size(layer, lm_head, x->ne[1]);
        if (!need)   // the shape is refused: the full call reports why, before any device work
            return qwm_verify_step(layer, layer_index, slot_tables, table_stride, x, rm, resid, out, ids_out, w_out,
                                   lm_head, norm_w, eps, drafts, result, nullptr, 0, stream);
        if (need > QWM_NOALLOC_SCRATCH_BYTES)
            return failf(QWM_ERR_UNSUPPORTED, "verify_step_noalloc: the step needs %zu bytes of scratch; the static "
                                              "array holds %zu", need, (size_t)QWM_NOALLOC_SCRATCH_BYTES);
        void * ptr = nullptr;
        int rc = scratch_address(&ptr);
        if (rc != QWM_OK) return rc;
        if ((rc = launch_fill_zero(ptr, need & ~(size_t)3, (hipStream_t)stream)) != QWM_OK) return rc;
        return qwm_verify_step(layer, layer_index, slot_tables, table_stride, x, rm, resid, out, ids_out, w_out, lm_head,
                               norm_w, eps, drafts, result, ptr, need, stream);
    });
}
