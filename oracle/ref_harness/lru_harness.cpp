// C entry points over the reference header-only GPU LRU victim index
// (core/gpu_lru_index.h), compiled from the reference tree by
// oracle/Makefile into oracle/_ref/.  Test infrastructure only: it checks the
// slot-pool restatements (oracle and product) decision for decision.
#include "gpu_lru_index.h"
#include <cstdint>
#include <vector>

#define QWR_API extern "C" __attribute__((visibility("default")))

QWR_API void * qwr_lru_new(int maximum_slots) { return new questwend::GpuLruIndex((size_t) maximum_slots); }
QWR_API void qwr_lru_free(void * index) { delete static_cast<questwend::GpuLruIndex *>(index); }
QWR_API int qwr_lru_rebuild(void * index, int retained, const int32_t * keys, const uint64_t * clocks) {
    try {
        std::vector<int> k(keys, keys + retained);
        std::vector<uint64_t> c(clocks, clocks + retained);
        static_cast<questwend::GpuLruIndex *>(index)->rebuild(retained, k, c);
        return 0;
    } catch (...) { return -1; }
}
QWR_API int qwr_lru_occupy_or_touch(void * index, int slot, uint64_t clock) {
    try { static_cast<questwend::GpuLruIndex *>(index)->occupy_or_touch(slot, clock); return 0; }
    catch (...) { return -1; }
}
QWR_API int qwr_lru_release(void * index, int slot) {
    try { static_cast<questwend::GpuLruIndex *>(index)->release(slot); return 0; }
    catch (...) { return -1; }
}
QWR_API int qwr_lru_pick(void * index, const uint8_t * protected_slots) {
    return static_cast<questwend::GpuLruIndex *>(index)->pick(
        [&](int slot) { return protected_slots && protected_slots[slot] != 0; }).slot;
}
