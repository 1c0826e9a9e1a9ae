// qwm_pool.cpp -- the GPU slot pool: the RAM-tier decisions of QuestWend's
// ExpertCache (core/expert_cache.cpp) over per-role pools of expert slabs in
// HBM, with misses filled from pinned host memory on a copy stream, by
// hipMemcpyAsync per slab or by one slab-gather launch per call.  Host code,
// owner thread only.
//
// Decision rules (all restated, not copied):
//   ensure (expert_cache.cpp:1615-1645): for each id i in order, for each role
//     gate, up, down: slot_for.
//   slot_for (1465-1479): count the access; a resident key is a hit (clock
//     touch); otherwise install.
//   install (1173-1180): pick a victim (none -> "No unprotected GPU cache
//     victim"), drop its key, fetch the slab, publish the new key.
//   pick_victim (1129-1170, quotas and activation scores off): the lowest
//     free slot, else the minimum clock among unprotected occupied slots with
//     strict '<' (lowest slot wins ties; a UINT64_MAX clock never wins).
//   clock (gpu_lru_pool_hooks.h:11-25): one counter shared by every role pool;
//     each hit or publication takes clock + 1.
//   drop (hooks 68-79): slot_of[key] returns to the 0 sentinel.
//   protection (ActiveExpertGuard, expert_cache.cpp:46-59): only when the
//     demand table exists (TinyLFU admission mode): desc.protect_active.
// The indexed mode keeps an ordered (clock, slot) set and a free-slot set,
// giving the same victims as the scan in O(log n).
// Fetch: MEMCPY issues one hipMemcpyAsync per missed slab as it is
// installed (the reference's order); GATHER collects the call's misses and
// launches one slab-gather kernel for them at the end of the call.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <algorithm>
#include <limits>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

#include "qwm_internal.h"

using namespace qwm;

struct qwm_pool {
    struct Role {
        int n_slots = 0;
        uint8_t * data = nullptr;
        size_t slab = 0;
        std::vector<const uint8_t *> host;          // per layer, pinned [*, *, n_expert]
        std::vector<const uint8_t *> host_dev;      // GATHER: device-visible addresses of `host`
        std::vector<int32_t> slot2key;
        std::vector<uint64_t> clk;
        std::unordered_map<int32_t, int32_t> key2slot;
        std::vector<int32_t> slot_of;               // [n_layer * n_expert], 0 sentinel
        std::vector<int32_t> occ;                   // per layer
        std::unordered_map<int32_t, uint64_t> count;
        std::set<std::pair<uint64_t, int32_t>> lru; // indexed mode: occupied (clock, slot)
        std::set<int32_t> free_slots;               // indexed mode
    };
    int n_layer = 0, n_expert = 0;
    bool protect = false, indexed = false;
    uint64_t clock = 0;
    uint64_t hits = 0, misses = 0, evictions = 0, fetch_bytes = 0, fetches = 0;
    Role role[3];
    std::vector<uint8_t> active;                    // [n_layer * n_expert] when protect
    hipStream_t copy = nullptr;
    hipEvent_t done = nullptr;
    bool pending = false;
    bool gather = false;
    std::vector<GatherItem> batch;                  // GATHER: this call's misses

    void touch(Role & R, int32_t slot) {
        const uint64_t next = clock + 1;
        if (indexed) {
            R.lru.erase({R.clk[slot], slot});
            R.lru.insert({next, slot});
        }
        R.clk[slot] = next;
        clock = next;
    }

    int32_t pick(const Role & R) const {
        if (indexed) {
            if (!R.free_slots.empty()) return *R.free_slots.begin();
            for (const auto & cs : R.lru) {
                if (cs.first == std::numeric_limits<uint64_t>::max()) return -1;
                if (protect && active[(size_t)R.slot2key[cs.second]]) continue;
                return cs.second;
            }
            return -1;
        }
        int32_t victim = -1;
        uint64_t best = std::numeric_limits<uint64_t>::max();
        for (int32_t s = 0; s < R.n_slots; ++s) {
            const int32_t k = R.slot2key[s];
            if (k < 0) return s;
            if (protect && active[(size_t)k]) continue;
            if (R.clk[s] < best) { best = R.clk[s]; victim = s; }
        }
        return victim;
    }

    void drop(Role & R, int32_t slot) {
        const int32_t key = R.slot2key[slot];
        if (key < 0) return;
        if (indexed) {
            R.lru.erase({R.clk[slot], slot});
            R.free_slots.insert(slot);
        }
        R.occ[key / n_expert]--;
        R.slot_of[key] = 0;
        R.key2slot.erase(key);
        R.slot2key[slot] = -1;
        evictions++;
    }

    int fetch(int r, int32_t layer, int32_t expert, int32_t slot) {
        Role & R = role[r];
        if (R.host.empty() || !R.host[layer]) return QWM_OK;   // no host tier: metadata only
        if (!done) {   // created on first use, so decision-only pools need no GPU
            hipError_t e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
            if (e != hipSuccess) return fail(QWM_ERR_HIP, std::string("slab fetch: hipEventCreate: ") + hipGetErrorString(e));
        }
        if (gather) {
            // A slot filled twice in one call (its first key was evicted again
            // within the call) keeps the later slab, as stream-ordered copies do.
            bool replaced = false;
            for (GatherItem & it : batch)
                if (it.role == r && it.slot == slot) { it.expert = expert; replaced = true; }
            if (!replaced) batch.push_back(GatherItem{expert, (int16_t)slot, (int16_t)r});
        } else {
            const uint8_t * src = R.host[layer] + (size_t)expert * R.slab;
            hipError_t e = hipMemcpyAsync(R.data + (size_t)slot * R.slab, src, R.slab, hipMemcpyHostToDevice, copy);
            if (e != hipSuccess) return fail(QWM_ERR_HIP, std::string("slab fetch: ") + hipGetErrorString(e));
        }
        fetch_bytes += R.slab;
        fetches++;
        pending = true;
        return QWM_OK;
    }

    // GATHER: one launch (per GATHER_MAX misses) for the call's misses.  On a
    // launch failure the call's installs are undone (their slots are freed),
    // so no published key points at a slot that was not filled.
    int flush(int32_t layer) {
        if (batch.empty()) return QWM_OK;
        GatherArgs a{};
        for (int r = 0; r < 3; ++r) {
            a.src[r] = role[r].host_dev.empty() ? nullptr : role[r].host_dev[layer];
            a.dst[r] = role[r].data;
            a.slab[r] = role[r].slab;
        }
        int rc = QWM_OK;
        for (size_t i0 = 0; i0 < batch.size() && rc == QWM_OK; i0 += GATHER_MAX) {
            a.n = (int32_t)std::min<size_t>(GATHER_MAX, batch.size() - i0);
            for (int32_t i = 0; i < a.n; ++i) a.item[i] = batch[i0 + i];
            rc = launch_slab_gather(a, copy);
        }
        if (rc != QWM_OK)
            for (const GatherItem & it : batch) {
                Role & R = role[it.role];
                const int32_t key = R.slot2key[it.slot];
                if (key < 0) continue;
                fetch_bytes -= R.slab;
                fetches--;
                if (indexed) {
                    R.lru.erase({R.clk[it.slot], it.slot});
                    R.free_slots.insert(it.slot);
                }
                R.occ[key / n_expert]--;
                R.slot_of[key] = 0;
                R.key2slot.erase(key);
                R.slot2key[it.slot] = -1;
            }
        batch.clear();
        return rc;
    }

    void publish(Role & R, int32_t slot, int32_t key, int32_t layer) {
        R.key2slot.emplace(key, slot);
        R.slot2key[slot] = key;
        R.occ[layer]++;
        R.slot_of[key] = slot;
        if (indexed) {
            R.free_slots.erase(slot);
            R.lru.insert({R.clk[slot], slot});
        }
        touch(R, slot);
    }
};

extern "C" {

int qwm_pool_create(const qwm_pool_desc * d, void * copy_stream, qwm_pool ** out) {
    if (!d || !out) return fail(QWM_ERR_ARG, "pool_create: NULL argument");
    *out = nullptr;
    if (d->n_layer < 1 || d->n_expert < 1) return fail(QWM_ERR_ARG, "pool_create: empty pool");
    auto * p = new qwm_pool();
    p->n_layer = d->n_layer;
    p->n_expert = d->n_expert;
    p->protect = d->protect_active != 0;
    p->indexed = d->indexed != 0;
    p->copy = (hipStream_t)copy_stream;
    p->gather = d->fetch_mode == QWM_FETCH_GATHER;
    if (d->fetch_mode != QWM_FETCH_MEMCPY && d->fetch_mode != QWM_FETCH_GATHER) {
        delete p;
        return fail(QWM_ERR_ARG, "pool_create: unknown fetch_mode");
    }
    for (int r = 0; r < 3; ++r) {
        auto & R = p->role[r];
        if (d->n_slots[r] < 1) { delete p; return fail(QWM_ERR_ARG, "pool_create: a role has no slots"); }
        R.n_slots = d->n_slots[r];
        R.data = (uint8_t *)d->pool_data[r];
        R.slab = d->slab_bytes[r];
        if (d->host_slabs[r]) R.host.assign((const uint8_t * const *)d->host_slabs[r], (const uint8_t * const *)d->host_slabs[r] + d->n_layer);
        if (p->gather && !R.host.empty()) {
            if (R.slab % 16 || ((uintptr_t)R.data & 15) || R.n_slots > 32767) {
                delete p;
                return fail(QWM_ERR_ARG, "pool_create: GATHER needs 16-byte aligned pools, slab_bytes % 16 == 0 and "
                                         "at most 32767 slots per role");
            }
            R.host_dev.assign((size_t)d->n_layer, nullptr);
            for (int32_t l = 0; l < d->n_layer; ++l) {
                if (!R.host[l]) continue;
                void * dp = nullptr;
                hipError_t e = hipHostGetDevicePointer(&dp, const_cast<uint8_t *>(R.host[l]), 0);
                if (e != hipSuccess) (void)hipGetLastError();   // a refused pointer is an argument error, not sticky
                if (e != hipSuccess || ((uintptr_t)dp & 15)) {
                    delete p;
                    return fail(QWM_ERR_ARG, std::string("pool_create: GATHER needs pinned (hipHostMalloc), 16-byte "
                                                         "aligned host slabs: ") + hipGetErrorString(e));
                }
                R.host_dev[l] = (const uint8_t *)dp;
            }
        }
        R.slot2key.assign((size_t)R.n_slots, -1);
        R.clk.assign((size_t)R.n_slots, 0);
        R.slot_of.assign((size_t)d->n_layer * d->n_expert, 0);
        R.occ.assign((size_t)d->n_layer, 0);
        if (p->indexed)
            for (int32_t s = 0; s < R.n_slots; ++s) R.free_slots.insert(s);
    }
    if (p->protect) p->active.assign((size_t)d->n_layer * d->n_expert, 0);
    *out = p;
    return QWM_OK;
}

void qwm_pool_destroy(qwm_pool * p) {
    if (!p) return;
    if (p->done) {
        (void)hipEventSynchronize(p->done);
        (void)hipEventDestroy(p->done);
    }
    delete p;
}

int qwm_pool_ensure(qwm_pool * p, int32_t layer, const int32_t * ids, int32_t n,
                    int32_t * sg, int32_t * su, int32_t * sd) {
    if (!p || (!ids && n) || (n && (!sg || !su || !sd))) return fail(QWM_ERR_ARG, "pool_ensure: NULL argument");
    if (layer < 0 || layer >= p->n_layer) return fail(QWM_ERR_ARG, "pool_ensure: layer out of range");
    for (int32_t i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= p->n_expert) return fail(QWM_ERR_ARG, "pool_ensure: expert id out of range");
    std::vector<size_t> changed;
    if (p->protect)
        for (int32_t i = 0; i < n; ++i) {
            const size_t key = (size_t)layer * p->n_expert + ids[i];
            if (!p->active[key]) { p->active[key] = 1; changed.push_back(key); }
        }
    int32_t * outs[3] = {sg, su, sd};
    int rc = QWM_OK;
    for (int32_t i = 0; i < n && rc == QWM_OK; ++i) {
        const int32_t e = ids[i];
        const int32_t key = layer * p->n_expert + e;
        for (int r = 0; r < 3; ++r) {
            auto & R = p->role[r];
            R.count[key]++;
            auto it = R.key2slot.find(key);
            if (it != R.key2slot.end()) {
                p->hits++;
                p->touch(R, it->second);
                outs[r][i] = it->second;
                continue;
            }
            p->misses++;
            const int32_t victim = p->pick(R);
            if (victim < 0) { rc = fail(QWM_ERR_NO_VICTIM, "No unprotected GPU cache victim"); break; }
            p->drop(R, victim);
            if ((rc = p->fetch(r, layer, e, victim)) != QWM_OK) break;   // victim stays free on failure
            p->publish(R, victim, key, layer);
            outs[r][i] = victim;
        }
    }
    for (size_t key : changed) p->active[key] = 0;
    if (p->gather) {   // the misses installed before a NO_VICTIM failure are filled too
        const int frc = p->flush(layer);
        if (frc != QWM_OK) return frc;
    }
    if (p->pending && (rc == QWM_OK || p->gather)) {
        hipError_t e = hipEventRecord(p->done, p->copy);
        if (e != hipSuccess) return fail(QWM_ERR_HIP, std::string("pool_ensure: hipEventRecord: ") + hipGetErrorString(e));
    }
    return rc;
}

int qwm_pool_wait(qwm_pool * p, void * stream) {
    if (!p) return fail(QWM_ERR_ARG, "pool_wait: NULL pool");
    if (!p->pending) return QWM_OK;
    QWM_HIP_CHECK(hipStreamWaitEvent((hipStream_t)stream, p->done, 0));
    return QWM_OK;
}

int qwm_pool_get_stats(const qwm_pool * p, qwm_pool_stats * out) {
    if (!p || !out) return fail(QWM_ERR_ARG, "pool_get_stats: NULL argument");
    out->hits = p->hits; out->misses = p->misses; out->evictions = p->evictions;
    out->fetch_bytes = p->fetch_bytes; out->fetches = p->fetches; out->clock = p->clock;
    return QWM_OK;
}

int qwm_pool_slot_of_row(const qwm_pool * p, int32_t role, int32_t layer, int32_t * out) {
    if (!p || !out || role < 0 || role > 2 || layer < 0 || layer >= p->n_layer) return fail(QWM_ERR_ARG, "pool_slot_of_row: bad argument");
    const auto & R = p->role[role];
    for (int32_t e = 0; e < p->n_expert; ++e) out[e] = R.slot_of[(size_t)layer * p->n_expert + e];
    return QWM_OK;
}

int qwm_pool_slots(const qwm_pool * p, int32_t role, int32_t * keys, uint64_t * clocks) {
    if (!p || role < 0 || role > 2) return fail(QWM_ERR_ARG, "pool_slots: bad argument");
    const auto & R = p->role[role];
    for (int32_t s = 0; s < R.n_slots; ++s) {
        if (keys) keys[s] = R.slot2key[s];
        if (clocks) clocks[s] = R.clk[s];
    }
    return QWM_OK;
}

int qwm_slab_fetch_async(void * pool_data, size_t slab_bytes, int32_t slot, const void * pinned_src,
                         void * copy_stream, void * done_event) {
    if (!pool_data || !pinned_src || slot < 0) return fail(QWM_ERR_ARG, "slab_fetch: bad argument");
    QWM_HIP_CHECK(hipMemcpyAsync((uint8_t *)pool_data + (size_t)slot * slab_bytes, pinned_src, slab_bytes,
                                 hipMemcpyHostToDevice, (hipStream_t)copy_stream));
    if (done_event) QWM_HIP_CHECK(hipEventRecord((hipEvent_t)done_event, (hipStream_t)copy_stream));
    return QWM_OK;
}

}  // extern "C"
