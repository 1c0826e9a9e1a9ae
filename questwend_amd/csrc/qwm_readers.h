// qwm_readers.h -- the persistent reader threads of the slot pool's file
// tier (the role of the reference's PersistentExpertIO workers,
// core/expert_io_workers.h): a fixed set of threads that claim the jobs of
// one batch at a time.
#pragma once

#include <condition_variable>
#include <cstdint>
#include <mutex>
#include <thread>
#include <vector>

namespace qwm {

// Persistent reader threads.  begin(n, fn, ctx) hands out jobs 0..n-1 (each
// run once, by whichever reader claims it, as fn(ctx, j)); wait(j) returns
// job j's status once it has run; end() returns when no reader is inside a
// job of the batch.  start() and reserve() take every allocation, so that
// begin() with n <= the reserved count allocates nothing.
class Readers {
public:
    using Job = int (*)(void * ctx, int j);
    ~Readers() { stop_all(); }
    void start(int n) {
        if ((int)th_.size() == n) return;
        stop_all();
        stop_ = false;
        th_.reserve((size_t)n);
        for (int i = 0; i < n; ++i) th_.emplace_back([this] { loop(); });
    }
    void reserve(int n) { status_.reserve((size_t)n); }
    void begin(int n, Job fn, void * ctx) {
        std::lock_guard<std::mutex> lk(mu_);
        fn_ = fn;
        ctx_ = ctx;
        n_ = n;
        next_ = 0;
        status_.assign((size_t)n, PENDING);
        ++gen_;
        go_.notify_all();
    }
    int wait(int j) {
        std::unique_lock<std::mutex> lk(mu_);
        done_.wait(lk, [&] { return status_[(size_t)j] != PENDING; });
        return status_[(size_t)j];
    }
    void end() {
        std::unique_lock<std::mutex> lk(mu_);
        next_ = n_;                                   // unclaimed jobs are not run
        done_.wait(lk, [&] { return active_ == 0; });
    }

private:
    static constexpr int PENDING = -2;
    void loop() {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            go_.wait(lk, [&] { return stop_ || gen_ != seen; });
            if (stop_) return;
            seen = gen_;
            ++active_;
            while (next_ < n_) {
                const int j = next_++;
                lk.unlock();
                const int st = fn_(ctx_, j);
                lk.lock();
                status_[(size_t)j] = st;
                done_.notify_all();
            }
            --active_;
            done_.notify_all();
        }
    }
    void stop_all() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        go_.notify_all();
        for (auto & t : th_) t.join();
        th_.clear();
    }
    std::mutex mu_;
    std::condition_variable go_, done_;
    std::vector<std::thread> th_;
    Job fn_ = nullptr;
    void * ctx_ = nullptr;
    std::vector<int> status_;
    int n_ = 0, next_ = 0, active_ = 0;
    uint64_t gen_ = 0;
    bool stop_ = false;
};

}  // namespace qwm
