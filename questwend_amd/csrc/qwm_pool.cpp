// qwm_pool.cpp -- the GPU slot pool: the RAM-tier decisions of QuestWend's
// ExpertCache (core/expert_cache.cpp) over signature pools of expert slabs
// in HBM, with misses filled from pinned host memory on a copy stream, by
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
//   signature pools (225-296): one pool per (role, type, ne0, ne1); every
//     (role, layer) is routed to one pool, which holds the keys of all the
//     layers routed to it.  qwm_pool_create makes one pool per role.
//   clock (gpu_lru_pool_hooks.h:11-25): one counter shared by every pool;
//     each hit or publication takes clock + 1.
//   drop (hooks 68-79): slot_of[key] returns to the 0 sentinel.
//   protection (ActiveExpertGuard, expert_cache.cpp:46-59): only when the
//     demand table exists (TinyLFU admission mode): desc.protect_active.
// The indexed mode keeps an ordered (clock, slot) set and a free-slot set,
// giving the same victims as the scan in O(log n).
// Fetch: MEMCPY issues one hipMemcpyAsync per missed slab as it is
// installed (the reference's order); GATHER collects the call's misses and
// launches one slab-gather kernel for them at the end of the call.
// File tier (ExpertCache::fetch_parallel's file path, expert_cache.cpp:
// 1194-1440): a (role, layer) attached to a file takes its missed slabs from
// file offset + expert * slab.  At the end of the call persistent reader
// threads pread them into a pinned staging ring, and the owner copies each
// slab to its slot on the copy stream as soon as its read is complete, in
// the order of the misses; a staging batch is reused only after its copies
// have left it.
#include <hip/hip_runtime_api.h>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstdint>
#include <cstring>
#include <algorithm>
#include <limits>
#include <memory>
#include <string>
#include <vector>

#include "qwm_internal.h"
#include "qwm_readers.h"

using namespace qwm;

namespace {

// pread until n bytes are in (0), or errno / -1 at end of file.
int read_full(int fd, uint8_t * dst, size_t n, uint64_t off) {
    while (n) {
        const ssize_t r = pread(fd, dst, n, (off_t)off);
        if (r < 0) {
            if (errno == EINTR) continue;
            return errno;
        }
        if (r == 0) return -1;
        dst += r; n -= (size_t)r; off += (uint64_t)r;
    }
    return 0;
}

struct FileJob {
    int32_t role, expert, slot;
};

}  // namespace

struct qwm_pool {
    struct Pool {                                   // one signature pool
        int role = 0;
        int n_slots = 0;
        uint8_t * data = nullptr;
        size_t slab = 0;
        std::vector<int32_t> slot2key;              // -1: free
        std::vector<uint64_t> clk;
        std::vector<int32_t> key2slot;              // [n_layer * n_expert], -1: not resident
        int32_t n_occ = 0;                          // occupied slots
        std::vector<int32_t> slot_of;               // [n_layer * n_expert], 0 sentinel
        std::vector<int32_t> occ;                   // per layer
        std::vector<uint64_t> count;                // [n_layer * n_expert]: accesses
        // indexed mode: the occupied slots in clock order (head: least
        // recently used; every touch takes a new maximum clock, so moving a
        // slot to the tail keeps the order) and the free slots as a bitmap
        // with one summary bit per word
        std::vector<int32_t> prev, next;
        int32_t head = -1, tail = -1;
        std::vector<uint64_t> free_bits, free_sum;
        std::vector<int32_t> quota;                 // per layer, after a rebalance
    };
    struct Src {                                    // where one role's slabs come from, per layer
        std::vector<const uint8_t *> host;          // pinned [*, *, n_expert]
        std::vector<const uint8_t *> host_dev;      // GATHER: device-visible addresses of `host`
        std::vector<int> fd;                        // file tier: -1 = none
        std::vector<uint64_t> foff;                 // file tier: offset of expert 0
    };
    int n_layer = 0, n_expert = 0;
    bool protect = false, indexed = false;
    bool quota_on = false;                          // per-layer quotas steer the victims (after a rebalance)
    int32_t n_used = 0;                             // the model's n_expert_used, from the last rebalance
    uint64_t clock = 0;
    uint64_t hits = 0, misses = 0, evictions = 0, fetch_bytes = 0, fetches = 0;
    std::vector<Pool> pools;
    std::vector<int32_t> lp[3];                     // pool index of (role, layer)
    Src src[3];
    std::vector<uint8_t> active;                    // [n_layer * n_expert] when protect
    hipStream_t copy = nullptr;
    hipEvent_t done = nullptr;
    bool pending = false;
    bool gather = false;
    std::vector<GatherItem> batch;                  // GATHER: this call's misses
    // file tier
    std::vector<FileJob> fjobs;                     // this call's misses from files
    bool files = false;                             // some (role, layer) is attached to a file
    Readers readers;
    int io_threads = 8, staging_slabs = 0;          // 0: as many slabs as fit in 64 MiB
    uint8_t * staging = nullptr;
    const uint8_t * staging_dev = nullptr;          // GATHER: device-visible address of the staging
    size_t staging_stride = 0;
    int staging_n = 0;
    hipEvent_t staging_free = nullptr;              // recorded after each batch's copies
    bool staging_busy = false;

    Pool & P(int r, int32_t layer) { return pools[(size_t)lp[r][(size_t)layer]]; }
    const Pool & P(int r, int32_t layer) const { return pools[(size_t)lp[r][(size_t)layer]]; }

    ~qwm_pool() {   // every flush ended with no reader inside a job
        for (auto & S : src)
            for (int f : S.fd)
                if (f >= 0) close(f);
        if (staging_free) {
            (void)hipEventSynchronize(staging_free);
            (void)hipEventDestroy(staging_free);
        }
        if (staging) (void)hipHostFree(staging);
    }

    static void lru_unlink(Pool & R, int32_t s) {
        const int32_t a = R.prev[(size_t)s], b = R.next[(size_t)s];
        (a >= 0 ? R.next[(size_t)a] : R.head) = b;
        (b >= 0 ? R.prev[(size_t)b] : R.tail) = a;
        R.prev[(size_t)s] = R.next[(size_t)s] = -1;
    }
    static void lru_push(Pool & R, int32_t s) {    // as the most recently used
        R.prev[(size_t)s] = R.tail;
        R.next[(size_t)s] = -1;
        (R.tail >= 0 ? R.next[(size_t)R.tail] : R.head) = s;
        R.tail = s;
    }
    static void mark_free(Pool & R, int32_t s, bool is_free) {
        const size_t w = (size_t)s >> 6;
        const uint64_t b = 1ull << (s & 63);
        R.free_bits[w] = is_free ? (R.free_bits[w] | b) : (R.free_bits[w] & ~b);
        const uint64_t sb = 1ull << (w & 63);
        R.free_sum[w >> 6] = R.free_bits[w] ? (R.free_sum[w >> 6] | sb) : (R.free_sum[w >> 6] & ~sb);
    }
    static int32_t first_free(const Pool & R) {
        for (size_t i = 0; i < R.free_sum.size(); ++i)
            if (R.free_sum[i]) {
                const size_t w = i * 64 + (size_t)__builtin_ctzll(R.free_sum[i]);
                return (int32_t)(w * 64 + (size_t)__builtin_ctzll(R.free_bits[w]));
            }
        return -1;
    }

    void touch(Pool & R, int32_t slot) {
        if (indexed) {
            lru_unlink(R, slot);
            lru_push(R, slot);
        }
        R.clk[slot] = ++clock;
    }

    int32_t pick(const Pool & R, int32_t layer) const {
        if (quota_on) return pick_quota(R, layer);
        if (indexed) {
            const int32_t f = first_free(R);
            if (f >= 0) return f;
            for (int32_t s = R.head; s >= 0; s = R.next[(size_t)s])
                if (!(protect && active[(size_t)R.slot2key[(size_t)s]])) return s;
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

    // pick_victim with per-layer quotas (expert_cache.cpp:1142-1170): a free
    // slot first; a layer at or over its quota recycles one of its own slots,
    // any other layer takes from a layer over its quota; least recently used
    // among those (strict <: the lowest slot on ties); none: the global LRU.
    int32_t pick_quota(const Pool & R, int32_t layer) const {
        const bool self = R.quota[layer] >= 0 && R.occ[layer] >= R.quota[layer];
        int32_t victim = -1;
        uint64_t best = std::numeric_limits<uint64_t>::max();
        for (int32_t s = 0; s < R.n_slots; ++s) {
            const int32_t k = R.slot2key[s];
            if (k < 0) return s;
            if (protect && active[(size_t)k]) continue;
            const int32_t kl = k / n_expert;
            if (self) { if (kl != layer) continue; }
            else if (R.occ[kl] <= R.quota[kl]) continue;
            if (R.clk[s] < best) { best = R.clk[s]; victim = s; }
        }
        if (victim >= 0) return victim;
        for (int32_t s = 0; s < R.n_slots; ++s) {
            const int32_t k = R.slot2key[s];
            if (protect && k >= 0 && active[(size_t)k]) continue;
            if (R.clk[s] < best) { best = R.clk[s]; victim = s; }
        }
        return victim;
    }

    void drop(Pool & R, int32_t slot) {
        const int32_t key = R.slot2key[slot];
        if (key < 0) return;
        if (indexed) {
            lru_unlink(R, slot);
            mark_free(R, slot, true);
        }
        R.occ[key / n_expert]--;
        R.slot_of[key] = 0;
        R.key2slot[key] = -1;
        R.n_occ--;
        R.slot2key[slot] = -1;
        evictions++;
    }

    int fetch(int r, int32_t layer, int32_t expert, int32_t slot) {
        Pool & R = P(r, layer);
        const Src & S = src[r];
        const bool from_file = !S.fd.empty() && S.fd[layer] >= 0;
        if (!from_file && (S.host.empty() || !S.host[layer])) return QWM_OK;   // no host tier: metadata only
        if (!done) {   // created on first use, so decision-only pools need no GPU
            hipError_t e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
            if (e != hipSuccess) return failf(QWM_ERR_HIP, "slab fetch: hipEventCreate: %s", hipGetErrorString(e));
        }
        if (from_file) {
            fjobs.push_back(FileJob{r, expert, slot});
        } else if (gather) {
            // A slot filled twice in one call (its first key was evicted again
            // within the call) keeps the later slab, as stream-ordered copies do.
            bool replaced = false;
            for (GatherItem & it : batch)
                if (it.role == r && it.slot == slot) { it.expert = expert; replaced = true; }
            if (!replaced) batch.push_back(GatherItem{expert, (int16_t)slot, (int16_t)r});
        } else {
            const uint8_t * from = S.host[layer] + (size_t)expert * R.slab;
            hipError_t e = hipMemcpyAsync(R.data + (size_t)slot * R.slab, from, R.slab, hipMemcpyHostToDevice, copy);
            if (e != hipSuccess) return failf(QWM_ERR_HIP, "slab fetch: %s", hipGetErrorString(e));
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
            a.src[r] = src[r].host_dev.empty() ? nullptr : src[r].host_dev[layer];
            a.dst[r] = P(r, layer).data;
            a.slab[r] = P(r, layer).slab;
        }
        int rc = QWM_OK;
        for (size_t i0 = 0; i0 < batch.size() && rc == QWM_OK; i0 += GATHER_MAX) {
            a.n = (int32_t)std::min<size_t>(GATHER_MAX, batch.size() - i0);
            for (int32_t i = 0; i < a.n; ++i) a.item[i] = batch[i0 + i];
            rc = launch_slab_gather(a, copy);
        }
        if (rc != QWM_OK)
            for (const GatherItem & it : batch) unpublish(it.role, layer, it.slot);
        batch.clear();
        return rc;
    }

    // Frees the slot of an install whose slab was not filled (its key no
    // longer resolves), as if the miss had not been taken.
    void unpublish(int r, int32_t layer, int32_t slot) {
        Pool & R = P(r, layer);
        const int32_t key = R.slot2key[slot];
        if (key < 0) return;
        fetch_bytes -= R.slab;
        fetches--;
        if (indexed) {
            lru_unlink(R, slot);
            mark_free(R, slot, true);
        }
        R.occ[key / n_expert]--;
        R.slot_of[key] = 0;
        R.key2slot[key] = -1;
        R.n_occ--;
        R.slot2key[slot] = -1;
    }

    // File tier: this call's misses, read by the readers into the staging ring
    // and copied to their slots in order.  On a failed read or copy the failed
    // job and every later one are unpublished.
    struct ReadCtx {
        qwm_pool * p;
        size_t b0;
        int32_t layer;
    };
    static int read_job(void * c, int j) {
        const ReadCtx & rc = *(const ReadCtx *)c;
        qwm_pool & p = *rc.p;
        const FileJob & fj = p.fjobs[rc.b0 + (size_t)j];
        const Pool & R = p.P(fj.role, rc.layer);
        const Src & S = p.src[fj.role];
        return read_full(S.fd[rc.layer], p.staging + (size_t)j * p.staging_stride, R.slab,
                         S.foff[rc.layer] + (uint64_t)fj.expert * R.slab);
    }

    int flush_files(int32_t layer) {
        if (fjobs.empty()) return QWM_OK;
        if (!staging) {   // prepare() runs before any job is queued
            for (const FileJob & j : fjobs) unpublish(j.role, layer, j.slot);
            fjobs.clear();
            return fail(QWM_ERR_STATE, "file tier: no staging ring");
        }
        int rc = QWM_OK;
        size_t bad = fjobs.size();
        for (size_t b0 = 0; b0 < fjobs.size() && rc == QWM_OK; b0 += (size_t)staging_n) {
            const int bn = (int)std::min<size_t>((size_t)staging_n, fjobs.size() - b0);
            if (staging_busy) {
                hipError_t e = hipEventSynchronize(staging_free);   // the previous batch's copies are out
                if (e != hipSuccess) { rc = failf(QWM_ERR_HIP, "file tier: %s", hipGetErrorString(e)); bad = b0; break; }
                staging_busy = false;
            }
            ReadCtx ctx{this, b0, layer};
            readers.begin(bn, &read_job, &ctx);
            // GATHER: one slab-gather launch per FILE_GATHER_GROUP completed reads
            constexpr int FILE_GATHER_GROUP = 8;
            GatherArgs ga{};
            for (int r = 0; r < 3; ++r) {
                ga.src[r] = staging_dev;
                ga.dst[r] = P(r, layer).data;
                ga.slab[r] = P(r, layer).slab;
                ga.src_stride[r] = staging_stride;
            }
            int g0 = 0;                                  // first job of the pending gather group
            auto launch_group = [&](int g1) {            // jobs [g0, g1) of this batch
                ga.n = g1 - g0;
                for (int i = 0; i < ga.n; ++i) {
                    const FileJob & gj = fjobs[b0 + (size_t)(g0 + i)];
                    ga.item[i] = GatherItem{g0 + i, (int16_t)gj.slot, (int16_t)gj.role};
                }
                const int lrc = ga.n > 0 ? launch_slab_gather(ga, copy) : QWM_OK;
                if (lrc == QWM_OK) g0 = g1;
                return lrc;
            };
            for (int j = 0; j < bn; ++j) {
                const int st = readers.wait(j);
                const FileJob & fj = fjobs[b0 + (size_t)j];
                Pool & R = P(fj.role, layer);
                if (st != 0) {
                    if (gather && launch_group(j) != QWM_OK) { rc = QWM_ERR_HIP; bad = b0 + (size_t)g0; break; }
                    rc = failf(QWM_ERR_IO, "file tier: reading the slab of expert %d (role %d, layer %d): %s",
                               (int)fj.expert, (int)fj.role, (int)layer, st < 0 ? "end of file" : strerror(st));
                    bad = b0 + (size_t)j;
                    break;
                }
                if (gather) {
                    if (j + 1 - g0 < FILE_GATHER_GROUP && j + 1 < bn) continue;
                    const int lrc = launch_group(j + 1);
                    if (lrc != QWM_OK) { rc = lrc; bad = b0 + (size_t)g0; break; }
                    continue;
                }
                hipError_t e = hipMemcpyAsync(R.data + (size_t)fj.slot * R.slab, staging + (size_t)j * staging_stride,
                                              R.slab, hipMemcpyHostToDevice, copy);
                if (e != hipSuccess) {
                    rc = failf(QWM_ERR_HIP, "file tier: %s", hipGetErrorString(e));
                    bad = b0 + (size_t)j;
                    break;
                }
            }
            readers.end();                               // no reader still writes this batch's staging
            if (hipEventRecord(staging_free, copy) == hipSuccess) staging_busy = true;
        }
        for (size_t i = bad; i < fjobs.size(); ++i) unpublish(fjobs[i].role, layer, fjobs[i].slot);
        fjobs.clear();
        return rc;
    }

    void publish(Pool & R, int32_t slot, int32_t key, int32_t layer) {
        R.key2slot[key] = slot;
        R.n_occ++;
        R.slot2key[slot] = key;
        R.occ[layer]++;
        R.slot_of[key] = slot;
        if (indexed) {
            mark_free(R, slot, false);
            lru_push(R, slot);
        }
        touch(R, slot);
    }

    // Everything a call may allocate, taken before its first change to the
    // pool: room for n_fetch more gather items and file jobs and, once a
    // file is attached, the pinned staging ring and the reader threads.
    // A failure here (an error code or an exception) leaves the pool as it
    // was.
    int prepare(size_t n_fetch) {
        if (gather) batch.reserve(batch.size() + n_fetch);
        if (!files) return QWM_OK;
        fjobs.reserve(fjobs.size() + n_fetch);
        if (!staging) {
            size_t max_slab = 0;
            for (const auto & R : pools) max_slab = std::max(max_slab, R.slab);
            staging_stride = (max_slab + 4095) & ~(size_t)4095;
            staging_n = staging_slabs > 0 ? staging_slabs : (int)std::max<size_t>(1, ((size_t)64 << 20) / staging_stride);
            uint8_t * st = nullptr;
            hipError_t e = hipHostMalloc((void **)&st, (size_t)staging_n * staging_stride, hipHostMallocDefault);
            if (e == hipSuccess && gather) {
                void * dp = nullptr;
                e = hipHostGetDevicePointer(&dp, st, 0);
                staging_dev = (const uint8_t *)dp;
            }
            if (e == hipSuccess && !staging_free) e = hipEventCreateWithFlags(&staging_free, hipEventDisableTiming);
            if (e != hipSuccess) {
                if (st) (void)hipHostFree(st);
                return failf(QWM_ERR_HIP, "file tier: pinned staging: %s", hipGetErrorString(e));
            }
            staging = st;
        }
        readers.start(io_threads);
        readers.reserve(staging_n);
        return QWM_OK;
    }
};

namespace qwm {
int32_t pool_n_layer(const qwm_pool * p) { return p->n_layer; }
int32_t pool_n_expert(const qwm_pool * p) { return p->n_expert; }
size_t pool_slab_bytes(const qwm_pool * p, int role, int32_t layer) { return p->P(role, layer).slab; }

// The layer's gate/up/down pool tensors must be the pools of its (role,
// layer) -- same base, slab stride and at least their slots -- so that every
// slot the pool hands out indexes inside the tensor the kernels read.
int pool_check_layer(const qwm_pool * p, int32_t layer, const qwm_tensor * const t[3], const char * who) {
    static const char * const names[3] = {"gate", "up", "down"};
    for (int r = 0; r < 3; ++r) {
        const auto & R = p->P(r, layer);
        if (t[r]->data != R.data || t[r]->nb[2] != R.slab || t[r]->ne[2] < R.n_slots)
            return fail(QWM_ERR_ARG, std::string(who) + ": the layer's " + names[r] + "_pool is not the pool of (" +
                                         names[r] + ", layer " + std::to_string(layer) + "): base " +
                                         (t[r]->data == R.data ? "ok" : "differs") + ", nb[2] " +
                                         std::to_string(t[r]->nb[2]) + " vs slab " + std::to_string(R.slab) +
                                         ", ne[2] " + std::to_string(t[r]->ne[2]) + " vs " +
                                         std::to_string(R.n_slots) + " slots");
    }
    return QWM_OK;
}
}  // namespace qwm

extern "C" {

// The pools, the (role, layer) routing and the host sources of a new pool
// (owned by the caller, which frees it unless this returns QWM_OK).
static int pool_init(qwm_pool * p, int32_t n_pools, const qwm_pool_sig * sig, const int32_t * layer_pool,
                     const void * const * const host_slabs[3], int32_t fetch_mode) {
    auto bad = [&](const std::string & why) { return fail(QWM_ERR_ARG, "pool_create: " + why); };
    if (fetch_mode != QWM_FETCH_MEMCPY && fetch_mode != QWM_FETCH_GATHER) return bad("unknown fetch_mode");
    p->gather = fetch_mode == QWM_FETCH_GATHER;
    if (n_pools < 3 || !sig || !layer_pool) return bad("fewer than three pools");
    p->pools.resize((size_t)n_pools);
    for (int32_t i = 0; i < n_pools; ++i) {
        auto & R = p->pools[(size_t)i];
        if (sig[i].role < 0 || sig[i].role > 2) return bad("a pool's role is not 0, 1 or 2");
        if (sig[i].n_slots < 1) return bad("a pool has no slots");
        R.role = sig[i].role;
        R.n_slots = sig[i].n_slots;
        R.data = (uint8_t *)sig[i].pool_data;
        R.slab = sig[i].slab_bytes;
        const size_t keys = (size_t)p->n_layer * p->n_expert;
        R.slot2key.assign((size_t)R.n_slots, -1);
        R.clk.assign((size_t)R.n_slots, 0);
        R.key2slot.assign(keys, -1);
        R.slot_of.assign(keys, 0);
        R.count.assign(keys, 0);
        R.occ.assign((size_t)p->n_layer, 0);
        R.quota.assign((size_t)p->n_layer, -1);     // no quota until a rebalance computes them
        if (p->indexed) {
            R.prev.assign((size_t)R.n_slots, -1);
            R.next.assign((size_t)R.n_slots, -1);
            R.free_bits.assign(((size_t)R.n_slots + 63) / 64, 0);
            R.free_sum.assign((R.free_bits.size() + 63) / 64, 0);
            for (int32_t s = 0; s < R.n_slots; ++s) qwm_pool::mark_free(R, s, true);
        }
    }
    for (int r = 0; r < 3; ++r) {
        p->lp[r].assign(layer_pool + (size_t)r * p->n_layer, layer_pool + (size_t)(r + 1) * p->n_layer);
        for (int32_t l = 0; l < p->n_layer; ++l) {
            const int32_t i = p->lp[r][(size_t)l];
            if (i < 0 || i >= n_pools || p->pools[(size_t)i].role != r)
                return bad("layer_pool routes (role " + std::to_string(r) + ", layer " + std::to_string(l) +
                           ") to a pool out of range or of another role");
        }
    }
    for (int r = 0; r < 3; ++r) {
        auto & S = p->src[r];
        if (!host_slabs[r]) continue;
        S.host.assign((const uint8_t * const *)host_slabs[r], (const uint8_t * const *)host_slabs[r] + p->n_layer);
        if (!p->gather) continue;
        S.host_dev.assign((size_t)p->n_layer, nullptr);
        for (int32_t l = 0; l < p->n_layer; ++l) {
            if (!S.host[l]) continue;
            const auto & R = p->P(r, l);
            if (R.slab % 16 || ((uintptr_t)R.data & 15) || R.n_slots > 32767)
                return bad("GATHER needs 16-byte aligned pools, slab_bytes % 16 == 0 and at most 32767 slots per pool");
            void * dp = nullptr;
            hipError_t e = hipHostGetDevicePointer(&dp, const_cast<uint8_t *>(S.host[l]), 0);
            if (e != hipSuccess) (void)hipGetLastError();   // a refused pointer is an argument error, not sticky
            if (e != hipSuccess || ((uintptr_t)dp & 15))
                return bad(std::string("GATHER needs pinned (hipHostMalloc), 16-byte aligned host slabs: ") +
                           hipGetErrorString(e));
            S.host_dev[l] = (const uint8_t *)dp;
        }
    }
    if (p->protect) p->active.assign((size_t)p->n_layer * p->n_expert, 0);
    return QWM_OK;
}

int qwm_pool_create(const qwm_pool_desc * d, void * copy_stream, qwm_pool ** out) {
    return guard("qwm_pool_create", [&]() -> int {
        if (!d || !out) return fail(QWM_ERR_ARG, "pool_create: NULL argument");
        *out = nullptr;
        if (d->n_layer < 1 || d->n_expert < 1) return fail(QWM_ERR_ARG, "pool_create: empty pool");
        qwm_pool_sig sig[3] = {};
        std::vector<int32_t> lp((size_t)3 * d->n_layer);
        for (int r = 0; r < 3; ++r) {
            sig[r].role = r;
            sig[r].n_slots = d->n_slots[r];
            sig[r].pool_data = d->pool_data[r];
            sig[r].slab_bytes = d->slab_bytes[r];
            for (int32_t l = 0; l < d->n_layer; ++l) lp[(size_t)r * d->n_layer + l] = r;
        }
        std::unique_ptr<qwm_pool> p(new qwm_pool());
        p->n_layer = d->n_layer;
        p->n_expert = d->n_expert;
        p->protect = d->protect_active != 0;
        p->indexed = d->indexed != 0;
        p->copy = (hipStream_t)copy_stream;
        const int rc = pool_init(p.get(), 3, sig, lp.data(), d->host_slabs, d->fetch_mode);
        if (rc == QWM_OK) *out = p.release();
        return rc;
    });
}

int qwm_pool_create_sig(const qwm_pool_sig_desc * d, void * copy_stream, qwm_pool ** out) {
    return guard("qwm_pool_create_sig", [&]() -> int {
        if (!d || !out || !d->pools || !d->layer_pool) return fail(QWM_ERR_ARG, "pool_create_sig: NULL argument");
        *out = nullptr;
        if (d->n_layer < 1 || d->n_expert < 1) return fail(QWM_ERR_ARG, "pool_create_sig: empty pool");
        std::unique_ptr<qwm_pool> p(new qwm_pool());
        p->n_layer = d->n_layer;
        p->n_expert = d->n_expert;
        p->protect = d->protect_active != 0;
        p->indexed = d->indexed != 0;
        p->copy = (hipStream_t)copy_stream;
        const int rc = pool_init(p.get(), d->n_pools, d->pools, d->layer_pool, d->host_slabs, d->fetch_mode);
        if (rc == QWM_OK) *out = p.release();
        return rc;
    });
}

// The signatures of ExpertCache's constructor (expert_cache.cpp:225-251) and
// the uniform residency fraction that sizes their pools (253-287).
int qwm_pool_plan_sigs(int32_t n_layer, int32_t n_expert, const qwm_tensor * experts, uint64_t vram_bytes,
                       int32_t n_used, qwm_pool_sig * sigs, int32_t max_sigs, int32_t * n_sigs,
                       int32_t * layer_pool, double * frac_out) {
    return guard("qwm_pool_plan_sigs", [&]() -> int {
        if (!experts || !sigs || !n_sigs || !layer_pool || n_layer < 1 || n_expert < 1 || n_used < 1 || max_sigs < 1)
            return fail(QWM_ERR_ARG, "pool_plan_sigs: bad argument");
        int32_t ns = 0;
        for (int r = 0; r < 3; ++r)
            for (int32_t l = 0; l < n_layer; ++l) {
                const qwm_tensor & t = experts[(size_t)r * n_layer + l];
                if (t.ne[2] != n_expert || t.ne[0] < 1 || t.ne[1] < 1 || t.nb[2] == 0)
                    return fail(QWM_ERR_ARG, "pool_plan_sigs: expert tensor of role " + std::to_string(r) + ", layer " +
                                                 std::to_string(l) + " is not [ne0, ne1, n_expert]");
                int32_t idx = -1;
                for (int32_t s = 0; s < ns; ++s)
                    if (sigs[s].role == r && sigs[s].type == t.type && sigs[s].ne0 == t.ne[0] && sigs[s].ne1 == t.ne[1]) {
                        idx = s;
                        break;
                    }
                if (idx < 0) {
                    if (ns >= max_sigs) return fail(QWM_ERR_ARG, "pool_plan_sigs: more than max_sigs signatures");
                    idx = ns++;
                    sigs[idx] = qwm_pool_sig{};
                    sigs[idx].role = r;
                    sigs[idx].type = t.type;
                    sigs[idx].ne0 = t.ne[0];
                    sigs[idx].ne1 = t.ne[1];
                    sigs[idx].slab_bytes = t.nb[2];
                }
                sigs[idx].n_layers++;
                layer_pool[(size_t)r * n_layer + l] = idx;
            }
        uint64_t total = 0;
        for (int32_t s = 0; s < ns; ++s) total += (uint64_t)sigs[s].slab_bytes * (uint64_t)sigs[s].n_layers * (uint64_t)n_expert;
        double frac = total ? (double)vram_bytes / (double)total : 1.0;
        if (frac > 1.0) frac = 1.0;
        for (int32_t s = 0; s < ns; ++s) {
            const int32_t cap = sigs[s].n_layers * n_expert;
            int32_t n = (int32_t)(frac * cap);
            if (n < n_used) n = n_used;
            if (n > cap) n = cap;
            if (n <= n_used)
                return fail(QWM_ERR_ARG, "pool_plan_sigs: pool " + std::to_string(s) + " would hold " + std::to_string(n) +
                                             " slots, no more than n_used (the reference's \"GPU pool cannot fit "
                                             "transient workspace plus retained experts\")");
            sigs[s].n_slots = n;
        }
        *n_sigs = ns;
        if (frac_out) *frac_out = frac;
        return QWM_OK;
    });
}

int qwm_pool_layer_pool(const qwm_pool * p, int32_t role, int32_t layer) {
    return guard("qwm_pool_layer_pool", [&]() -> int {
        if (!p || role < 0 || role > 2 || layer < 0 || layer >= p->n_layer) return fail(QWM_ERR_ARG, "pool_layer_pool: bad argument");
        return p->lp[role][(size_t)layer];
    });
}

void qwm_pool_destroy(qwm_pool * p) {
    guard_void("qwm_pool_destroy", [&]() {
        if (!p) return;
        if (p->done) {
            (void)hipEventSynchronize(p->done);
            (void)hipEventDestroy(p->done);
        }
        delete p;
    });
}

int qwm_pool_ensure(qwm_pool * p, int32_t layer, const int32_t * ids, int32_t n,
                    int32_t * sg, int32_t * su, int32_t * sd) {
    return guard("qwm_pool_ensure", [&]() -> int {
        if (!p || (!ids && n) || (n && (!sg || !su || !sd))) return fail(QWM_ERR_ARG, "pool_ensure: NULL argument");
        if (layer < 0 || layer >= p->n_layer) return fail(QWM_ERR_ARG, "pool_ensure: layer out of range");
        for (int32_t i = 0; i < n; ++i)
            if (ids[i] < 0 || ids[i] >= p->n_expert) return fail(QWM_ERR_ARG, "pool_ensure: expert id out of range");
        // every allocation of the call, before its first change to the pool
        std::vector<size_t> changed;
        if (p->protect) changed.reserve((size_t)n);
        int rc = p->prepare(3 * (size_t)n);
        if (rc != QWM_OK) return rc;
        if (p->protect)
            for (int32_t i = 0; i < n; ++i) {
                const size_t key = (size_t)layer * p->n_expert + ids[i];
                if (!p->active[key]) { p->active[key] = 1; changed.push_back(key); }
            }
        int32_t * outs[3] = {sg, su, sd};
        for (int32_t i = 0; i < n && rc == QWM_OK; ++i) {
            const int32_t e = ids[i];
            const int32_t key = layer * p->n_expert + e;
            for (int r = 0; r < 3; ++r) {
                auto & R = p->P(r, layer);
                R.count[key]++;
                const int32_t hit = R.key2slot[key];
                if (hit >= 0) {
                    p->hits++;
                    p->touch(R, hit);
                    outs[r][i] = hit;
                    continue;
                }
                p->misses++;
                const int32_t victim = p->pick(R, layer);
                if (victim < 0) { rc = fail(QWM_ERR_NO_VICTIM, "No unprotected GPU cache victim"); break; }
                p->drop(R, victim);
                if ((rc = p->fetch(r, layer, e, victim)) != QWM_OK) break;   // victim stays free on failure
                p->publish(R, victim, key, layer);
                outs[r][i] = victim;
            }
        }
        for (size_t key : changed) p->active[key] = 0;
        // the misses installed before a NO_VICTIM failure are filled too
        const int grc = p->gather ? p->flush(layer) : QWM_OK;
        const int frc = p->flush_files(layer);
        if (p->pending) {   // covers every copy issued so far, also after a failure
            hipError_t e = hipEventRecord(p->done, p->copy);
            if (e != hipSuccess) return failf(QWM_ERR_HIP, "pool_ensure: hipEventRecord: %s", hipGetErrorString(e));
        }
        if (grc != QWM_OK) return grc;
        if (frc != QWM_OK) return frc;
        return rc;
    });
}

int qwm_pool_wait(qwm_pool * p, void * stream) {
    return guard("qwm_pool_wait", [&]() -> int {
        if (!p) return fail(QWM_ERR_ARG, "pool_wait: NULL pool");
        if (!p->pending) return QWM_OK;
        QWM_HIP_CHECK(hipStreamWaitEvent((hipStream_t)stream, p->done, 0));
        return QWM_OK;
    });
}

int qwm_pool_get_stats(const qwm_pool * p, qwm_pool_stats * out) {
    return guard("qwm_pool_get_stats", [&]() -> int {
        if (!p || !out) return fail(QWM_ERR_ARG, "pool_get_stats: NULL argument");
        out->hits = p->hits; out->misses = p->misses; out->evictions = p->evictions;
        out->fetch_bytes = p->fetch_bytes; out->fetches = p->fetches; out->clock = p->clock;
        return QWM_OK;
    });
}

int qwm_pool_slot_of_row(const qwm_pool * p, int32_t role, int32_t layer, int32_t * out) {
    return guard("qwm_pool_slot_of_row", [&]() -> int {
        if (!p || !out || role < 0 || role > 2 || layer < 0 || layer >= p->n_layer) return fail(QWM_ERR_ARG, "pool_slot_of_row: bad argument");
        const auto & R = p->P(role, layer);
        for (int32_t e = 0; e < p->n_expert; ++e) out[e] = R.slot_of[(size_t)layer * p->n_expert + e];
        return QWM_OK;
    });
}

int qwm_pool_resident_bits(const qwm_pool * p, int32_t layer, uint32_t * bits) {
    return guard("qwm_pool_resident_bits", [&]() -> int {
        if (!p || !bits || layer < 0 || layer >= p->n_layer) return fail(QWM_ERR_ARG, "pool_resident_bits: bad argument");
        const int32_t words = (p->n_expert + 31) / 32;
        for (int32_t w = 0; w < words; ++w) bits[w] = 0u;
        for (int32_t e = 0; e < p->n_expert; ++e) {
            const int32_t key = layer * p->n_expert + e;
            bool all = true;
            for (int r = 0; r < 3 && all; ++r) all = p->P(r, layer).key2slot[key] >= 0;
            if (all) bits[e >> 5] |= 1u << (e & 31);
        }
        return QWM_OK;
    });
}

int qwm_pool_touch(qwm_pool * p, int32_t layer, const int32_t * ids, int32_t n) {
    return guard("qwm_pool_touch", [&]() -> int {
        if (!p || (!ids && n) || layer < 0 || layer >= p->n_layer) return fail(QWM_ERR_ARG, "pool_touch: bad argument");
        for (int32_t i = 0; i < n; ++i)
            if (ids[i] < 0 || ids[i] >= p->n_expert) return fail(QWM_ERR_ARG, "pool_touch: expert id out of range");
        for (int32_t i = 0; i < n; ++i) {
            const int32_t key = layer * p->n_expert + ids[i];
            for (int r = 0; r < 3; ++r) {
                auto & R = p->P(r, layer);
                const int32_t slot = R.key2slot[key];
                if (slot < 0) continue;
                R.count[key]++;
                p->touch(R, slot);
                p->hits++;
            }
        }
        return QWM_OK;
    });
}

// ExpertCache::capacity (expert_cache.cpp:478-491): the fewest slots the
// layer may hold in the pools of its three roles before it recycles its own
// -- its quota (at least n_used) while quotas are on and computed, else the
// pool size.
int qwm_pool_capacity(const qwm_pool * p, int32_t layer) {
    return guard("qwm_pool_capacity", [&]() -> int {
        if (!p || layer < 0 || layer >= p->n_layer) return fail(QWM_ERR_ARG, "pool_capacity: bad argument");
        int32_t m = INT32_MAX;
        for (int r = 0; r < 3; ++r) {
            const auto & R = p->P(r, layer);
            const int32_t q = R.quota[(size_t)layer];
            m = std::min(m, p->quota_on && q >= 0 ? std::max(q, p->n_used) : R.n_slots);
        }
        return m;
    });
}

// ExpertCache::quota_of (expert_cache.cpp:493-501): the layer's quota (min
// over the pools of its roles), or the pool size where none was computed.
int qwm_pool_quota_of(const qwm_pool * p, int32_t layer) {
    return guard("qwm_pool_quota_of", [&]() -> int {
        if (!p || layer < 0 || layer >= p->n_layer) return fail(QWM_ERR_ARG, "pool_quota_of: bad argument");
        int32_t m = INT32_MAX;
        for (int r = 0; r < 3; ++r) {
            const auto & R = p->P(r, layer);
            const int32_t q = R.quota[(size_t)layer];
            m = std::min(m, q >= 0 ? q : R.n_slots);
        }
        return m;
    });
}

int qwm_pool_quotas_active(const qwm_pool * p) {
    return guard("qwm_pool_quotas_active", [&]() -> int {
        if (!p) return fail(QWM_ERR_ARG, "pool_quotas_active: NULL pool");
        return p->quota_on ? 1 : 0;
    });
}

// ExpertCache::set_quotas (expert_cache.h:162).  The indexed mode's shortcut
// is off while quotas steer the victims.
int qwm_pool_set_quotas(qwm_pool * p, int32_t on) {
    return guard("qwm_pool_set_quotas", [&]() -> int {
        if (!p) return fail(QWM_ERR_ARG, "pool_set_quotas: NULL pool");
        p->quota_on = on != 0;
        return QWM_OK;
    });
}

// plan_slices (runtime.cpp:4639-4687): the layer's expert union over the
// batch; quotas on when the union fits the layer's quota - 8, off otherwise;
// then slices of consecutive tokens, cut before a token whose new experts
// would take the slice's union past max(n_used, capacity - 8) or whose slice
// reached max_slice tokens (QWEN_SEGB_SLICE, 1024 by default).
int qwm_pool_plan_slices(qwm_pool * p, int32_t layer, const int32_t * sel, int32_t T, int32_t n_used,
                         int32_t max_slice, int32_t * slices, int32_t * n_slices, int32_t * union_out) {
    return guard("qwm_pool_plan_slices", [&]() -> int {
        if (!p || !sel || !slices || !n_slices || T < 1 || n_used < 1 || max_slice < 0 || layer < 0 ||
            layer >= p->n_layer)
            return fail(QWM_ERR_ARG, "pool_plan_slices: bad argument");
        const int32_t E = p->n_expert;
        for (int64_t i = 0; i < (int64_t)T * n_used; ++i)
            if (sel[i] < 0 || sel[i] >= E) return fail(QWM_ERR_ARG, "pool_plan_slices: expert id out of range");
        if (max_slice == 0) max_slice = 1024;
        std::vector<uint8_t> seen((size_t)E, 0);
        int32_t uni = 0;
        for (int64_t i = 0; i < (int64_t)T * n_used; ++i)
            if (!seen[(size_t)sel[i]]) { seen[(size_t)sel[i]] = 1; ++uni; }
        p->quota_on = uni <= qwm_pool_quota_of(p, layer) - 8;
        const int32_t cap = std::max(n_used, qwm_pool_capacity(p, layer) - 8);
        std::fill(seen.begin(), seen.end(), 0);
        int32_t ns = 0, distinct = 0, t0 = 0;
        for (int32_t t = 0; t < T; ++t) {
            int32_t nnew = 0;
            for (int32_t j = 0; j < n_used; ++j) {
                const int32_t e = sel[(size_t)t * n_used + j];
                if (!seen[(size_t)e]) { seen[(size_t)e] = 1; ++nnew; }
            }
            if ((distinct + nnew > cap || t - t0 >= max_slice) && t > t0) {
                slices[2 * ns] = t0; slices[2 * ns + 1] = t - t0; ++ns;
                std::fill(seen.begin(), seen.end(), 0);
                distinct = 0; nnew = 0;
                for (int32_t j = 0; j < n_used; ++j) {
                    const int32_t e = sel[(size_t)t * n_used + j];
                    if (!seen[(size_t)e]) { seen[(size_t)e] = 1; ++nnew; }
                }
                t0 = t;
            }
            distinct += nnew;
        }
        slices[2 * ns] = t0; slices[2 * ns + 1] = T - t0; ++ns;
        *n_slices = ns;
        if (union_out) *union_out = uni;
        return QWM_OK;
    });
}

int qwm_pool_slots(const qwm_pool * p, int32_t pool, int32_t * keys, uint64_t * clocks) {
    return guard("qwm_pool_slots", [&]() -> int {
        if (!p || pool < 0 || pool >= (int32_t)p->pools.size()) return fail(QWM_ERR_ARG, "pool_slots: bad argument");
        const auto & R = p->pools[(size_t)pool];
        for (int32_t s = 0; s < R.n_slots; ++s) {
            if (keys) keys[s] = R.slot2key[s];
            if (clocks) clocks[s] = R.clk[s];
        }
        return QWM_OK;
    });
}

// ExpertCache::save_profile (expert_cache.cpp:1485-1500): the same text
// format; pools in order (each line carries its pool's role), keys ascending
// within a pool.
int qwm_pool_save_profile(const qwm_pool * p, const char * path) {
    return guard("qwm_pool_save_profile", [&]() -> int {
        if (!p || !path) return fail(QWM_ERR_ARG, "pool_save_profile: NULL argument");
        FILE * f = std::fopen(path, "wb");
        if (!f) return fail(QWM_ERR_IO, std::string("pool_save_profile: ") + path + ": " + strerror(errno));
        bool ok = std::fprintf(f, "QWENEXPCACHE 1\n%d %d\n", p->n_layer, p->n_expert) > 0;
        for (const auto & R : p->pools)
            for (size_t key = 0; key < R.count.size() && ok; ++key)
                if (R.count[key])
                    ok = std::fprintf(f, "%d %d %d %llu\n", R.role, (int)(key / (size_t)p->n_expert),
                                      (int)(key % (size_t)p->n_expert), (unsigned long long)R.count[key]) > 0;
        ok = (std::fclose(f) == 0) && ok;
        if (!ok) return fail(QWM_ERR_IO, std::string("pool_save_profile: writing ") + path + " failed");
        return QWM_OK;
    });
}

// ExpertCache::load_prefetch (expert_cache.cpp:1502-1538): a missing or
// incompatible profile is a cold start (nothing installed, QWM_OK).  The
// in-range entries, largest count first (equal counts in file order), are
// installed while the pool of their (role, layer) has a free slot and the
// key is not resident; the slabs are fetched as ensure fetches misses.
int qwm_pool_load_profile(qwm_pool * p, const char * path, int64_t * n_installed) {
    return guard("qwm_pool_load_profile", [&]() -> int {
        if (!p || !path) return fail(QWM_ERR_ARG, "pool_load_profile: NULL argument");
        if (n_installed) *n_installed = 0;
        FILE * f = std::fopen(path, "rb");
        if (!f) return QWM_OK;
        int ver = 0, nl = 0, ne = 0;
        if (std::fscanf(f, "QWENEXPCACHE %d", &ver) != 1 || ver != 1 || std::fscanf(f, "%d %d", &nl, &ne) != 2 ||
            nl != p->n_layer || ne != p->n_expert) {
            std::fclose(f);
            return QWM_OK;
        }
        struct Ent { int r, l, e; unsigned long long c; };
        std::vector<Ent> ents;
        Ent en;
        while (std::fscanf(f, "%d %d %d %llu", &en.r, &en.l, &en.e, &en.c) == 4)
            if (en.r >= 0 && en.r < 3 && en.l >= 0 && en.l < p->n_layer && en.e >= 0 && en.e < p->n_expert) ents.push_back(en);
        std::fclose(f);
        std::stable_sort(ents.begin(), ents.end(), [](const Ent & a, const Ent & b) { return a.c > b.c; });
        int rc = p->prepare(ents.size());   // the call's allocations, before its first change to the pool
        if (rc != QWM_OK) return rc;
        int cur = -1;
        int64_t n = 0;
        auto flush_layer = [&](int layer) {          // the fetch batches are per layer
            if (layer < 0) return QWM_OK;
            const int grc = p->gather ? p->flush(layer) : QWM_OK;
            const int frc = p->flush_files(layer);
            return grc != QWM_OK ? grc : frc;
        };
        for (const Ent & x : ents) {
            auto & R = p->P(x.r, x.l);
            if (R.n_occ >= R.n_slots) continue;
            const int32_t key = x.l * p->n_expert + x.e;
            if (R.key2slot[key] >= 0) continue;
            if (x.l != cur) {
                if ((rc = flush_layer(cur)) != QWM_OK) break;
                cur = x.l;
            }
            const int32_t slot = p->pick(R, x.l);    // the lowest free slot
            if ((rc = p->fetch(x.r, x.l, x.e, slot)) != QWM_OK) break;
            p->publish(R, slot, key, x.l);
            ++n;
        }
        const int lrc = flush_layer(cur);
        if (rc == QWM_OK) rc = lrc;
        if (p->pending) QWM_HIP_CHECK(hipEventRecord(p->done, p->copy));
        if (n_installed) *n_installed = n;
        return rc;
    });
}

// ExpertCache::compute_quota and rebalance (expert_cache.cpp:509-625): one
// quota per layer from the counts summed over the pools (entries by count,
// then key, both descending).  A layer's expert takes one slot in each of
// the pools of its three roles, while all three have one left: first every
// layer up to n_used experts, then greedily one more expert per entry beyond
// its layer's first n_used.  Each of the layer's pools gets that quota.
// The quotas then steer every later victim (pick_quota), and the hottest
// experts within each layer's quota are installed, all three roles
// together, up to fill_budget experts.  Everything is computed, and the
// call's allocations taken, before the first change to the pool.
int qwm_pool_rebalance(qwm_pool * p, int32_t n_used, int64_t fill_budget, int32_t * quota_out, int64_t * n_filled) {
    return guard("qwm_pool_rebalance", [&]() -> int {
        if (!p || n_used < 1 || fill_budget < 0) return fail(QWM_ERR_ARG, "pool_rebalance: bad argument");
        if (n_filled) *n_filled = 0;
        const int32_t L = p->n_layer, E = p->n_expert;
        std::vector<uint64_t> cnt((size_t)L * E, 0);
        for (const auto & R : p->pools)
            for (size_t key = 0; key < cnt.size(); ++key) cnt[key] += R.count[key];
        std::vector<std::pair<uint64_t, int32_t>> ents;   // (count, key) of every counted key
        for (size_t key = 0; key < cnt.size(); ++key)
            if (cnt[key]) ents.emplace_back(cnt[key], (int32_t)key);
        std::sort(ents.begin(), ents.end(), std::greater<std::pair<uint64_t, int32_t>>());
        std::vector<int32_t> quota((size_t)L, 0);
        if (!ents.empty()) {
            std::vector<int64_t> rem(p->pools.size());
            for (size_t i = 0; i < p->pools.size(); ++i) rem[i] = p->pools[i].n_slots;
            auto take = [&](int32_t l) {
                for (int r = 0; r < 3; ++r)
                    if (rem[(size_t)p->lp[r][(size_t)l]] <= 0) return false;
                for (int r = 0; r < 3; ++r) rem[(size_t)p->lp[r][(size_t)l]]--;
                return true;
            };
            for (int32_t l = 0; l < L; ++l)
                while (quota[l] < n_used && take(l)) quota[l]++;
            std::vector<int32_t> seen((size_t)L, 0);
            for (const auto & e : ents) {
                const int32_t l = e.second / E;
                if (seen[l]++ < n_used) continue;
                if (quota[l] >= E) continue;
                if (!take(l)) continue;
                quota[l]++;
            }
        }
        std::vector<int32_t> seen((size_t)L, 0);
        int rc = p->prepare(3 * (size_t)std::min<int64_t>(fill_budget, (int64_t)ents.size()));
        if (rc != QWM_OK) return rc;
        for (int32_t l = 0; l < L; ++l)
            for (int r = 0; r < 3; ++r) p->P(r, l).quota[(size_t)l] = quota[l];
        p->quota_on = true;
        p->n_used = n_used;
        if (quota_out) std::copy(quota.begin(), quota.end(), quota_out);
        int cur = -1;
        int64_t filled = 0;
        auto flush_layer = [&](int layer) {
            if (layer < 0) return QWM_OK;
            const int grc = p->gather ? p->flush(layer) : QWM_OK;
            const int frc = p->flush_files(layer);
            return grc != QWM_OK ? grc : frc;
        };
        for (const auto & e : ents) {
            if (filled >= fill_budget) break;
            const int32_t key = e.second, l = key / E, ex = key % E;
            if (seen[l] >= quota[l]) continue;
            seen[l]++;
            bool all = true;
            for (int r = 0; r < 3; ++r) all = all && p->P(r, l).key2slot[key] >= 0;
            if (all) continue;
            if (l != cur) {
                if ((rc = flush_layer(cur)) != QWM_OK) break;
                cur = l;
            }
            for (int r = 0; r < 3 && rc == QWM_OK; ++r) {
                auto & R = p->P(r, l);
                if (R.key2slot[key] >= 0) continue;
                const int32_t victim = p->pick(R, l);
                if (victim < 0) { rc = fail(QWM_ERR_NO_VICTIM, "No unprotected GPU cache victim"); break; }
                p->drop(R, victim);
                if ((rc = p->fetch(r, l, ex, victim)) != QWM_OK) break;
                p->publish(R, victim, key, l);
            }
            if (rc != QWM_OK) break;
            ++filled;
        }
        const int lrc = flush_layer(cur);
        if (rc == QWM_OK) rc = lrc;
        if (p->pending) QWM_HIP_CHECK(hipEventRecord(p->done, p->copy));
        if (n_filled) *n_filled = filled;
        return rc;
    });
}

// ExpertCache::clear_counts (expert_cache.cpp:557-559).
int qwm_pool_clear_counts(qwm_pool * p) {
    return guard("qwm_pool_clear_counts", [&]() -> int {
        if (!p) return fail(QWM_ERR_ARG, "pool_clear_counts: NULL pool");
        for (auto & R : p->pools) std::fill(R.count.begin(), R.count.end(), 0);
        return QWM_OK;
    });
}

int qwm_pool_attach_file(qwm_pool * p, int32_t role, int32_t layer, const char * path, uint64_t offset) {
    return guard("qwm_pool_attach_file", [&]() -> int {
        if (!p || !path || role < 0 || role > 2 || layer < 0 || layer >= p->n_layer)
            return fail(QWM_ERR_ARG, "pool_attach_file: bad argument");
        const auto & R = p->P(role, layer);
        auto & S = p->src[role];
        if (!R.data) return fail(QWM_ERR_ARG, "pool_attach_file: the (role, layer) has no device pool");
        if (p->gather && (R.slab % 16 || ((uintptr_t)R.data & 15) || R.n_slots > 32767))
            return fail(QWM_ERR_ARG, "pool_attach_file: GATHER needs 16-byte aligned pools, slab_bytes % 16 == 0 and at "
                                     "most 32767 slots per pool");
        if (S.fd.empty()) {   // allocated before the file is opened, so an exception leaks no descriptor
            S.fd.assign((size_t)p->n_layer, -1);
            S.foff.assign((size_t)p->n_layer, 0);
        }
        const int fd = open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) return failf(QWM_ERR_IO, "pool_attach_file: %s: %s", path, strerror(errno));
        struct stat st;
        const uint64_t need = offset + (uint64_t)p->n_expert * R.slab;
        if (fstat(fd, &st) != 0 || (uint64_t)st.st_size < need) {
            close(fd);
            return failf(QWM_ERR_ARG, "pool_attach_file: %s is shorter than offset + n_expert * slab_bytes", path);
        }
        if (S.fd[layer] >= 0) close(S.fd[layer]);
        S.fd[layer] = fd;
        S.foff[layer] = offset;
        p->files = true;
        return QWM_OK;
    });
}

int qwm_pool_set_io(qwm_pool * p, int32_t n_threads, int32_t staging_slabs) {
    return guard("qwm_pool_set_io", [&]() -> int {
        if (!p || n_threads < 1 || n_threads > 64 || staging_slabs < 0) return fail(QWM_ERR_ARG, "pool_set_io: bad argument");
        p->io_threads = n_threads;
        if (staging_slabs != p->staging_slabs && p->staging) {   // re-sized on the next miss
            if (p->staging_busy) QWM_HIP_CHECK(hipEventSynchronize(p->staging_free));
            p->staging_busy = false;
            QWM_HIP_CHECK(hipHostFree(p->staging));
            p->staging = nullptr;
        }
        p->staging_slabs = staging_slabs;
        return QWM_OK;
    });
}

int qwm_slab_fetch_async(void * pool_data, size_t slab_bytes, int32_t slot, const void * pinned_src,
                         void * copy_stream, void * done_event) {
    return guard("qwm_slab_fetch_async", [&]() -> int {
        if (!pool_data || !pinned_src || slot < 0) return fail(QWM_ERR_ARG, "slab_fetch: bad argument");
        QWM_HIP_CHECK(hipMemcpyAsync((uint8_t *)pool_data + (size_t)slot * slab_bytes, pinned_src, slab_bytes,
                                     hipMemcpyHostToDevice, (hipStream_t)copy_stream));
        if (done_event) QWM_HIP_CHECK(hipEventRecord((hipEvent_t)done_event, (hipStream_t)copy_stream));
        return QWM_OK;
    });
}

}  // extern "C"
