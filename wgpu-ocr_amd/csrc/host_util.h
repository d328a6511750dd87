// Host-side helpers shared by the page pipelines: a worker thread pool and pinned buffers.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "common.h"

namespace ocr {

using Clock = std::chrono::steady_clock;
inline double ms_since(Clock::time_point t) { return std::chrono::duration<double, std::milli>(Clock::now() - t).count(); }

// A fixed pool of host worker threads with a FIFO of tasks.
class Workers {
  public:
    explicit Workers(int n) {
        for (int i = 0; i < n; i++) threads_.emplace_back([this] { loop(); });
    }
    ~Workers() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : threads_) t.join();
    }
    void submit(std::function<void()> f) {
        {
            std::lock_guard<std::mutex> lk(mu_);
            q_.push_back(std::move(f));
        }
        cv_.notify_one();
    }

  private:
    void loop() {
        for (;;) {
            std::function<void()> f;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [this] { return stop_ || !q_.empty(); });
                if (q_.empty()) return;
                f = std::move(q_.front());
                q_.pop_front();
            }
            f();
        }
    }
    std::vector<std::thread> threads_;
    std::deque<std::function<void()>> q_;
    std::mutex mu_;
    std::condition_variable cv_;
    bool stop_ = false;
};

// A process-wide pool of host threads for data-parallel loops. run(n, fn, prio) calls fn(i)
// for every i in [0, n) on the calling thread and on whichever pool threads are free, and
// returns when all are done. Pool threads take items of the loop with the lowest prio first
// (then the oldest), so the page needed first gets the free cores first. Items are claimed one
// at a time under the lock: loops here have tens to hundreds of items of tens of microseconds.
class LoopPool {
  public:
    // Four cores fewer than the host has: the threads that call run() (a page's layout each,
    // whose serial steps run there) keep cores of their own.
    static LoopPool &get() {
        static LoopPool pool(std::max(1, int(std::thread::hardware_concurrency()) - 4));
        return pool;
    }
    template <class F> void run(int n, F &&fn, int prio = 0) {
        if (n <= 0) return;
        if (n == 1 || threads_.empty()) {
            for (int i = 0; i < n; i++) fn(i);
            return;
        }
        Job job;
        job.n = n;
        job.prio = prio;
        job.fn = [&fn](int i) { fn(i); };
        {
            std::lock_guard<std::mutex> lk(mu_);
            job.seq = seq_++;
            jobs_.push_back(&job);
        }
        cv_.notify_all();
        for (;;) {
            int i;
            {
                std::lock_guard<std::mutex> lk(mu_);
                if (job.next >= n) break;
                i = job.next++;
                if (job.next == n) unlist(&job);
            }
            job.fn(i);
            finish(job);
        }
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return job.done == n; });
    }
    ~LoopPool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : threads_) t.join();
    }

  private:
    struct Job {
        int n = 0, next = 0, done = 0, prio = 0;
        long seq = 0;
        std::function<void(int)> fn;
    };
    explicit LoopPool(int n) {
        for (int i = 0; i < n; i++) threads_.emplace_back([this] { loop(); });
    }
    void unlist(Job *j) { jobs_.erase(std::remove(jobs_.begin(), jobs_.end(), j), jobs_.end()); }
    void finish(Job &j) {
        std::lock_guard<std::mutex> lk(mu_);
        if (++j.done == j.n) done_cv_.notify_all();
    }
    void loop() {
        for (;;) {
            Job *j = nullptr;
            int i = 0;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [this] { return stop_ || !jobs_.empty(); });
                if (stop_) return;
                for (Job *c : jobs_)
                    if (!j || c->prio < j->prio || (c->prio == j->prio && c->seq < j->seq)) j = c;
                i = j->next++;
                if (j->next == j->n) unlist(j);
            }
            j->fn(i);
            finish(*j);
        }
    }
    std::vector<std::thread> threads_;
    std::vector<Job *> jobs_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    long seq_ = 0;
    bool stop_ = false;
};

// Page-locked host memory, reused across runs.
struct Pinned {
    void *p = nullptr;
    size_t bytes = 0;
    Pinned() = default;
    Pinned(const Pinned &) = delete;
    Pinned &operator=(const Pinned &) = delete;
    Pinned(Pinned &&o) noexcept : p(o.p), bytes(o.bytes) { o.p = nullptr, o.bytes = 0; }
    Pinned &operator=(Pinned &&o) noexcept {
        std::swap(p, o.p);
        std::swap(bytes, o.bytes);
        return *this;
    }
    void ensure(size_t n) {
        if (n <= bytes) return;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        host_malloc(&p, n);
        // Touch every page now: the first CPU access to a page of it faults it in (about 2 GB/s
        // where later accesses run at memory speed), which would otherwise land on a run.
        std::memset(p, 0, n);
        bytes = n;
    }
    ~Pinned() {
        if (p) (void)hipHostFree(p);
    }
};


// Host worker threads: the request, else the hardware's threads, at most 16.
inline int worker_count(int requested) {
    if (requested > 0) return requested;
    const int hc = int(std::thread::hardware_concurrency());
    return std::max(1, std::min(hc > 0 ? hc : 4, 16));
}

}  // namespace ocr
