// qwm_fetch.hip -- slab gather: one launch copies every slab that a pool
// ensure call missed, reading the pinned host slabs over the host link from
// the GPU itself.
//
// The reference fills each miss with its own host-to-device copy
// (ExpertCache::fetch_slab, core/expert_cache.cpp:706-717).  On MI355X a
// 576 KiB copy engine transfer costs about 10 us of set-up on top of its
// ~11 us of data, so a verify step with ~33 missed slabs reaches half of the
// link rate.  Here the workgroups of one kernel pull 128 KiB chunks each
// with 16-byte loads from the device-visible address of the pinned host
// memory (hipHostMalloc memory is mapped into the GPU's address space) and
// write them to the pool slots: the copies overlap each other and the
// launch is paid once.  The destination bytes are the same as the copies'.
#include <hip/hip_runtime.h>

#include "qwm_internal.h"

namespace qwm {

namespace {

constexpr int GATHER_THREADS = 256;
constexpr int GATHER_UNROLL = 4;
constexpr int GATHER_CHUNK16 = 8192;   // 16-byte units per workgroup (128 KiB)

__global__ __launch_bounds__(GATHER_THREADS) void k_slab_gather(GatherArgs a) {
    const int item = (int)(blockIdx.x / (unsigned)a.wg_per_item);
    const int part = (int)(blockIdx.x % (unsigned)a.wg_per_item);
    if (item >= a.n) return;
    const GatherItem it = a.item[item];
    const int r = it.role;
    const size_t n16 = a.slab[r] / 16;
    const size_t beg = (size_t)part * GATHER_CHUNK16;
    if (beg >= n16) return;
    const size_t end = beg + GATHER_CHUNK16 < n16 ? beg + GATHER_CHUNK16 : n16;
    const size_t stride = a.src_stride[r] ? a.src_stride[r] : a.slab[r];
    const uint4 * src = reinterpret_cast<const uint4 *>(a.src[r] + (size_t)it.expert * stride);
    uint4 * dst = reinterpret_cast<uint4 *>(a.dst[r] + (size_t)it.slot * a.slab[r]);
    for (size_t i = beg + (size_t)threadIdx.x * GATHER_UNROLL; i < end; i += GATHER_THREADS * GATHER_UNROLL) {
        uint4 v[GATHER_UNROLL];
#pragma unroll
        for (int j = 0; j < GATHER_UNROLL; ++j)
            if (i + j < end) v[j] = src[i + j];
#pragma unroll
        for (int j = 0; j < GATHER_UNROLL; ++j)
            if (i + j < end) dst[i + j] = v[j];
    }
}

}  // namespace

int launch_slab_gather(const GatherArgs & a, hipStream_t s) {
    if (a.n <= 0) return QWM_OK;
    size_t max16 = 0;
    for (int r = 0; r < 3; ++r) max16 = a.slab[r] / 16 > max16 ? a.slab[r] / 16 : max16;
    GatherArgs b = a;
    b.wg_per_item = (int32_t)((max16 + GATHER_CHUNK16 - 1) / GATHER_CHUNK16);
    if (b.wg_per_item < 1) return QWM_OK;
    hipLaunchKernelGGL(k_slab_gather, dim3((unsigned)(b.wg_per_item * b.n)), dim3(GATHER_THREADS), 0, s, b);
    QWM_HIP_CHECK(hipGetLastError());
    return QWM_OK;
}

}  // namespace qwm
