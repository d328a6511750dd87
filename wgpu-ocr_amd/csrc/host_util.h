// Host-side helpers shared by the page pipelines: a worker thread pool and pinned buffers.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <condition_variable>
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
        OCR_HIP(hipHostMalloc(&p, n, hipHostMallocDefault));
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
