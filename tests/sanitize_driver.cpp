// sanitize_driver.cpp -- libqwmoe's host code under the sanitizers, built by
// tests/test_sanitizers.py from the library's own sources (no GPU is used):
//   pool            random signature-pool traces in every index mode:
//                   ensure, touch, plan_slices, rebalance, profiles, the
//                   argument errors (AddressSanitizer + UndefinedBehavior-
//                   Sanitizer build);
//   gguf <files..>  the GGUF index over every file given -- valid, truncated
//                   and corrupted ones -- with tensor lookups and the expert
//                   attach (same build);
//   readers         the file tier's reader threads over many batches,
//                   thread-count changes and batches ended early
//                   (ThreadSanitizer build, QWM_SAN_READERS_ONLY).
// Exits 0 when every run completed and its checks held; the sanitizers abort
// the process on the first report.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "../questwend_amd/csrc/qwm_readers.h"

#ifndef QWM_SAN_READERS_ONLY
#include "../questwend_amd/csrc/qwm_internal.h"

// The slab-gather launcher lives in the kernel library; decision-only pools
// never launch it.
namespace qwm {
int launch_slab_gather(const GatherArgs &, hipStream_t) { return fail(QWM_ERR_HIP, "no GPU in this build"); }
}  // namespace qwm
#endif

#define CHECK(cond)                                                               \
    do {                                                                          \
        if (!(cond)) {                                                            \
            std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            std::exit(1);                                                         \
        }                                                                         \
    } while (0)

#ifndef QWM_SAN_READERS_ONLY
static int run_pool(const char * dir) {
    std::mt19937 rng(11);
    const std::string prof = std::string(dir) + "/san.prof";
    for (int mode = 0; mode < 4; ++mode) {
        const int L = 5, E = 48, k = 6;
        // gate and up shared by every layer; down split over two pools
        qwm_pool_sig sig[4];
        std::memset(sig, 0, sizeof sig);
        const int32_t slots[4] = {60, 60, 30, 19}, roles[4] = {0, 1, 2, 2};
        for (int i = 0; i < 4; ++i) {
            sig[i].role = roles[i];
            sig[i].n_slots = slots[i];
        }
        const int32_t lp[3 * L] = {0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 2, 3, 2, 3, 2};
        qwm_pool_sig_desc d;
        std::memset(&d, 0, sizeof d);
        d.n_layer = L;
        d.n_expert = E;
        d.n_pools = 4;
        d.pools = sig;
        d.layer_pool = lp;
        d.indexed = mode & 1;
        d.protect_active = mode >= 2;
        d.fetch_mode = mode == 3 ? QWM_FETCH_GATHER : QWM_FETCH_MEMCPY;
        qwm_pool * p = nullptr;
        CHECK(qwm_pool_create_sig(&d, nullptr, &p) == QWM_OK);
        std::vector<int32_t> ids, s;
        for (int step = 0; step < 3000; ++step) {
            const int l = (int)(rng() % L);
            const int T = 1 + (int)(rng() % 3);
            ids.clear();
            for (int t = 0; t < T; ++t) {
                int got = 0;
                while (got < k) {
                    const int32_t e = (int32_t)(rng() % (uint32_t)(1 + rng() % E));
                    bool dup = false;
                    for (int j = 0; j < got; ++j) dup = dup || ids[(size_t)(t * k + j)] == e;
                    if (!dup) { ids.push_back(e); ++got; }
                }
            }
            const int32_t n = (int32_t)ids.size();
            s.assign(3 * (size_t)n, -1);
            switch (step % 11) {
                case 3: CHECK(qwm_pool_touch(p, l, ids.data(), n) == QWM_OK); break;
                case 5: {
                    std::vector<int32_t> sl(2 * (size_t)T);
                    int32_t ns = 0, uni = 0;
                    CHECK(qwm_pool_plan_slices(p, l, ids.data(), T, k, 0, sl.data(), &ns, &uni) == QWM_OK);
                    CHECK(ns >= 1 && ns <= T);
                    break;
                }
                case 7:
                    if (step % 500 == 7) {
                        std::vector<int32_t> q(L);
                        int64_t nf = 0;
                        CHECK(qwm_pool_rebalance(p, k, 20, q.data(), &nf) == QWM_OK);
                    }
                    break;
                case 9:
                    if (step % 700 == 9) {
                        CHECK(qwm_pool_save_profile(p, prof.c_str()) == QWM_OK);
                        qwm_pool * q = nullptr;
                        CHECK(qwm_pool_create_sig(&d, nullptr, &q) == QWM_OK);
                        int64_t ni = 0;
                        CHECK(qwm_pool_load_profile(q, prof.c_str(), &ni) == QWM_OK);
                        qwm_pool_destroy(q);
                    }
                    break;
                default: {
                    const int rc = qwm_pool_ensure(p, l, ids.data(), n, s.data(), s.data() + n, s.data() + 2 * n);
                    CHECK(rc == QWM_OK || rc == QWM_ERR_NO_VICTIM);
                    if (rc == QWM_OK)
                        for (int r = 0; r < 3; ++r)
                            for (int i = 0; i < n; ++i)
                                CHECK(s[(size_t)(r * n + i)] >= 0 &&
                                      s[(size_t)(r * n + i)] < slots[lp[r * L + l]]);
                }
            }
            if (step % 101 == 0) {   // argument errors
                int32_t bad = E;
                CHECK(qwm_pool_ensure(p, l, &bad, 1, s.data(), s.data(), s.data()) == QWM_ERR_ARG);
                CHECK(qwm_pool_ensure(p, L, ids.data(), 1, s.data(), s.data(), s.data()) == QWM_ERR_ARG);
                CHECK(qwm_pool_slots(p, 4, nullptr, nullptr) == QWM_ERR_ARG);
                std::vector<uint32_t> bits((E + 31) / 32);
                CHECK(qwm_pool_resident_bits(p, l, bits.data()) == QWM_OK);
            }
        }
        qwm_pool_destroy(p);
    }
    return 0;
}

static int run_gguf(int n, char ** files) {
    static const char * const names[] = {"blk.0.ffn_gate_exps.weight", "blk.1.ffn_down_exps.weight",
                                         "token_embd.weight", "output_norm.weight", "not.there"};
    int ok = 0;
    for (int i = 0; i < n; ++i) {
        for (const char * name : names) {
            qwm_gguf_tensor t;
            if (qwm_gguf_find_tensor(files[i], name, &t) == QWM_OK) ++ok;
        }
        // the expert attach on a pool whose device addresses are never
        // touched (no ensure runs on it)
        qwm_pool_desc d;
        std::memset(&d, 0, sizeof d);
        d.n_layer = 2;
        d.n_expert = 4;
        for (int r = 0; r < 3; ++r) {
            d.n_slots[r] = 4;
            d.pool_data[r] = reinterpret_cast<void *>((uintptr_t)0x100000 * (r + 1));
            d.slab_bytes[r] = 73728;   // one Q4_K [512, 256] (or [256, 512]) expert
        }
        qwm_pool * p = nullptr;
        CHECK(qwm_pool_create(&d, nullptr, &p) == QWM_OK);
        (void)qwm_pool_attach_gguf(p, files[i], 0);
        qwm_pool_destroy(p);
    }
    std::printf("gguf lookups found %d\n", ok);
    return 0;
}
#endif

struct ReadBatch {
    std::vector<int> out;
    int round;
};
static int job(void * c, int j) {
    ReadBatch & b = *(ReadBatch *)c;
    b.out[(size_t)j] = j * 7 + b.round;
    return (j % 13 == 12) ? 5 : 0;   // a few jobs report an error status
}

static int run_readers() {
    std::mt19937 rng(3);
    qwm::Readers rd;
    for (int round = 0; round < 400; ++round) {
        const int nt = 1 + round / 40 % 6;   // the thread count changes every 40 batches
        rd.start(nt);
        rd.reserve(64);
        ReadBatch b;
        const int bn = 1 + (int)(rng() % 64);
        b.out.assign((size_t)bn, -1);
        b.round = round;
        rd.begin(bn, &job, &b);
        const int upto = (round % 5 == 4) ? (int)(rng() % (uint32_t)bn) : bn;   // some batches end early
        for (int j = 0; j < upto; ++j) {
            const int st = rd.wait(j);
            CHECK(st == ((j % 13 == 12) ? 5 : 0));
            CHECK(b.out[(size_t)j] == j * 7 + round);
        }
        rd.end();   // no reader is inside a job of this batch from here on: b may go
    }
    std::printf("readers ok\n");
    return 0;
}

int main(int argc, char ** argv) {
    if (argc < 2) return 2;
    const std::string mode = argv[1];
    if (mode == "readers") return run_readers();
#ifndef QWM_SAN_READERS_ONLY
    if (mode == "pool") return run_pool(argc > 2 ? argv[2] : "/tmp");
    if (mode == "gguf") return run_gguf(argc - 2, argv + 2);
#endif
    return 2;
}
