// pool_fault_test.cpp -- fault injection over libqwmoe's slot pool through
// the C ABI, in the manner of the reference's tests/gpu_lru_index_test.cpp
// (an operator new override that makes a chosen allocation throw).
//
// For each operation (ensure, touch, plan_slices, rebalance, load_profile,
// clear_counts, set_quotas, save_profile, create) and each allocation index
// N = 1, 2, ...: the N-th allocation inside the call throws std::bad_alloc.
// Every call must then
//   - return QWM_ERR_NOMEM with a message naming the entry point, and
//   - leave the pool exactly as it was (keys, clocks, slot_of rows, stats,
//     capacity, quota_of, quota mode, saved profile text),
// until N passes the call's allocation count; then the call must give the
// same result and state as the same call on a twin pool that never failed.
// Decision-only pools (no host slabs, no device memory): no GPU is used.
// Prints "ok <faults injected>" and exits 0, or names the failure and exits 1.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <random>
#include <string>
#include <vector>

#include "../include/qwmoe.h"

static long g_countdown = 0;   // > 0: allocations left before the one that throws
static long g_injected = 0;

// Throwing allocations count down; the nothrow forms (std::stable_sort's
// temporary buffer) are left alone, since their callers cope with NULL.
static void * take(size_t n, bool nothrow) {
    if (!nothrow && g_countdown > 0 && --g_countdown == 0) {
        ++g_injected;
        throw std::bad_alloc();
    }
    void * p = std::malloc(n ? n : 1);
    if (!p && !nothrow) throw std::bad_alloc();
    return p;
}
void * operator new(size_t n) { return take(n, false); }
void * operator new[](size_t n) { return take(n, false); }
void * operator new(size_t n, const std::nothrow_t &) noexcept { return take(n, true); }
void * operator new[](size_t n, const std::nothrow_t &) noexcept { return take(n, true); }
void operator delete(void * p) noexcept { std::free(p); }
void operator delete[](void * p) noexcept { std::free(p); }
void operator delete(void * p, size_t) noexcept { std::free(p); }
void operator delete[](void * p, size_t) noexcept { std::free(p); }

static int g_fail = 0;
#define CHECK(cond, ...)                                    \
    do {                                                    \
        if (!(cond)) {                                      \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);              \
            std::fprintf(stderr, "\n");                     \
            g_fail = 1;                                     \
        }                                                   \
    } while (0)

constexpr int L = 4, E = 32, N_USED = 4;
static const int32_t POOL_SLOTS[4] = {40, 40, 20, 16};     // gate, up (all layers), down A, down B
static const int32_t POOL_ROLE[4] = {0, 1, 2, 2};
static const int32_t LAYER_POOL[3 * L] = {0, 0, 0, 0, 1, 1, 1, 1, 2, 3, 3, 2};

static qwm_pool * make(int indexed, int protect, int gather) {
    qwm_pool_sig sig[4];
    std::memset(sig, 0, sizeof sig);
    for (int i = 0; i < 4; ++i) {
        sig[i].role = POOL_ROLE[i];
        sig[i].n_slots = POOL_SLOTS[i];
    }
    qwm_pool_sig_desc d;
    std::memset(&d, 0, sizeof d);
    d.n_layer = L;
    d.n_expert = E;
    d.n_pools = 4;
    d.pools = sig;
    d.layer_pool = LAYER_POOL;
    d.indexed = indexed;
    d.protect_active = protect;
    d.fetch_mode = gather ? QWM_FETCH_GATHER : QWM_FETCH_MEMCPY;
    qwm_pool * p = nullptr;
    if (qwm_pool_create_sig(&d, nullptr, &p) != QWM_OK) {
        std::fprintf(stderr, "create: %s\n", qwm_last_error());
        std::exit(1);
    }
    return p;
}

static std::string slurp(const char * path) {
    std::string s;
    FILE * f = std::fopen(path, "rb");
    if (!f) return s;
    char buf[4096];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) s.append(buf, n);
    std::fclose(f);
    return s;
}

// Everything the C ABI shows of a pool.
static std::string state(const qwm_pool * p, const char * tmp) {
    std::string s;
    char line[128];
    for (int i = 0; i < 4; ++i) {
        std::vector<int32_t> k((size_t)POOL_SLOTS[i]);
        std::vector<uint64_t> c((size_t)POOL_SLOTS[i]);
        qwm_pool_slots(p, i, k.data(), c.data());
        for (int t = 0; t < POOL_SLOTS[i]; ++t) {
            std::snprintf(line, sizeof line, "%d:%d:%llu ", i, k[(size_t)t], (unsigned long long)c[(size_t)t]);
            s += line;
        }
    }
    std::vector<int32_t> row(E);
    for (int r = 0; r < 3; ++r)
        for (int l = 0; l < L; ++l) {
            qwm_pool_slot_of_row(p, r, l, row.data());
            for (int e = 0; e < E; ++e) s += std::to_string(row[(size_t)e]) + ",";
        }
    for (int l = 0; l < L; ++l)
        s += " cap" + std::to_string(qwm_pool_capacity(p, l)) + " q" + std::to_string(qwm_pool_quota_of(p, l));
    s += " on" + std::to_string(qwm_pool_quotas_active(p));
    qwm_pool_stats st;
    qwm_pool_get_stats(p, &st);
    std::snprintf(line, sizeof line, " h%llu m%llu e%llu c%llu", (unsigned long long)st.hits,
                  (unsigned long long)st.misses, (unsigned long long)st.evictions, (unsigned long long)st.clock);
    s += line;
    qwm_pool_save_profile(p, tmp);
    s += slurp(tmp);
    return s;
}

// Runs op on `a` with the N-th allocation failing, N = 1, 2, ..., checking
// NOMEM + unchanged state each time, until op returns something else; then
// runs op on the twin `b` and checks that both agree.  Returns the number of
// injected failures.
template <class Op>
static int sweep(const char * name, qwm_pool * a, qwm_pool * b, const char * tmp, Op op) {
    const std::string before = state(a, tmp);
    int faults = 0;
    for (long n = 1; n < 100000; ++n) {
        const long injected0 = g_injected;
        g_countdown = n;
        const int rc = op(a);
        g_countdown = 0;
        if (g_injected == injected0) {     // the call made fewer than n allocations: done
            const int rb = op(b);
            CHECK(rc == rb, "%s: rc %d on the faulted pool, %d on its twin", name, rc, rb);
            CHECK(state(a, tmp) == state(b, tmp), "%s: state differs from the twin after the call", name);
            return faults;
        }
        ++faults;
        CHECK(rc == QWM_ERR_NOMEM, "%s: allocation %ld failed, rc %d (%s)", name, n, rc, qwm_last_error());
        CHECK(std::strstr(qwm_last_error(), "bad_alloc") != nullptr, "%s: message '%s'", name, qwm_last_error());
        CHECK(state(a, tmp) == before, "%s: allocation %ld failed and the pool changed", name, n);
        if (g_fail) return faults;
    }
    CHECK(false, "%s: never completed", name);
    return faults;
}

int main(int argc, char ** argv) {
    const std::string dir = argc > 1 ? argv[1] : "/tmp";
    const std::string tmp = dir + "/fault_state.prof", prof = dir + "/fault_load.prof";
    std::mt19937 rng(7);
    int total = 0;
    for (int mode = 0; mode < 3; ++mode) {
        const int indexed = mode >= 1, protect = mode == 2, gather = mode == 2;
        qwm_pool * a = make(indexed, protect, gather);
        qwm_pool * b = make(indexed, protect, gather);
        auto draw = [&](int layer, int n) {   // n distinct experts, skewed towards low ids
            std::vector<int32_t> ids;
            while ((int)ids.size() < n) {
                const int32_t e = (int32_t)(rng() % (uint32_t)(1 + rng() % E));
                bool dup = false;
                for (int32_t x : ids) dup = dup || x == e;
                if (!dup) ids.push_back(e);
            }
            (void)layer;
            return ids;
        };
        for (int step = 0; step < 60; ++step) {
            const int l = (int)(rng() % L);
            std::vector<int32_t> ids = draw(l, N_USED);
            std::vector<int32_t> more = draw(l, N_USED);
            ids.insert(ids.end(), more.begin(), more.end());
            std::vector<int32_t> s(3 * ids.size());
            const int32_t n = (int32_t)ids.size();
            total += sweep("ensure", a, b, tmp.c_str(), [&](qwm_pool * p) {
                return qwm_pool_ensure(p, l, ids.data(), n, s.data(), s.data() + n, s.data() + 2 * n);
            });
            if (step % 6 == 5) {
                std::vector<int32_t> t = draw(l, N_USED);
                total += sweep("touch", a, b, tmp.c_str(),
                               [&](qwm_pool * p) { return qwm_pool_touch(p, l, t.data(), N_USED); });
            }
            if (step % 9 == 8) {
                int32_t sl[2 * 2], ns, uni;
                total += sweep("plan_slices", a, b, tmp.c_str(), [&](qwm_pool * p) {
                    return qwm_pool_plan_slices(p, l, ids.data(), 2, N_USED, 0, sl, &ns, &uni);
                });
            }
            if (step == 30) {
                int32_t q[L];
                int64_t nf;
                total += sweep("rebalance", a, b, tmp.c_str(),
                               [&](qwm_pool * p) { return qwm_pool_rebalance(p, N_USED, 12, q, &nf); });
            }
            if (g_fail) break;
        }
        total += sweep("save_profile", a, b, tmp.c_str(),
                       [&](qwm_pool * p) { return qwm_pool_save_profile(p, prof.c_str()); });
        total += sweep("set_quotas", a, b, tmp.c_str(), [&](qwm_pool * p) { return qwm_pool_set_quotas(p, 0); });
        // a profile loaded into fresh pools
        qwm_pool * c = make(indexed, protect, gather);
        qwm_pool * d = make(indexed, protect, gather);
        int64_t ni;
        total += sweep("load_profile", c, d, tmp.c_str(),
                       [&](qwm_pool * p) { return qwm_pool_load_profile(p, prof.c_str(), &ni); });
        total += sweep("clear_counts", a, b, tmp.c_str(), [&](qwm_pool * p) { return qwm_pool_clear_counts(p); });
        qwm_pool_destroy(a);
        qwm_pool_destroy(b);
        qwm_pool_destroy(c);
        qwm_pool_destroy(d);
        if (g_fail) break;
    }
    // create: every failing allocation returns NOMEM and no pool
    for (long n = 1; n < 100000 && !g_fail; ++n) {
        qwm_pool_sig sig[4];
        std::memset(sig, 0, sizeof sig);
        for (int i = 0; i < 4; ++i) {
            sig[i].role = POOL_ROLE[i];
            sig[i].n_slots = POOL_SLOTS[i];
        }
        qwm_pool_sig_desc dsc;
        std::memset(&dsc, 0, sizeof dsc);
        dsc.n_layer = L;
        dsc.n_expert = E;
        dsc.n_pools = 4;
        dsc.pools = sig;
        dsc.layer_pool = LAYER_POOL;
        dsc.indexed = 1;
        static int sentinel;
        qwm_pool * p = reinterpret_cast<qwm_pool *>(&sentinel);   // must come back NULL on failure
        const long injected0 = g_injected;
        g_countdown = n;
        const int rc = qwm_pool_create_sig(&dsc, nullptr, &p);
        g_countdown = 0;
        if (g_injected == injected0) {
            CHECK(rc == QWM_OK && p, "create: rc %d", rc);
            qwm_pool_destroy(p);
            break;
        }
        ++total;
        CHECK(rc == QWM_ERR_NOMEM && p == nullptr, "create: allocation %ld failed, rc %d", n, rc);
    }
    if (g_fail) return 1;
    std::printf("ok %d\n", total);
    return 0;
}
