// Device context: the GPU, its stream and the scratch pool (the reference's Gpu, src/gpu.rs:825-1056).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <deque>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "wait.h"

namespace ocr {

// As device_malloc (common.h), but returns the error instead of failing (the pool retries after a trim).
hipError_t try_device_malloc(void **p, size_t bytes);
uint64_t device_allocations();
uint64_t host_allocations();
// Bounded waits (wait.h) for an event or for all work of a stream; `what` names it, with the
// event or stream, in the error a deadline raises.
void wait_event(hipEvent_t ev, const std::string &what, bool spin = false);
void wait_stream(hipStream_t s, const std::string &what, bool spin = true);
// For destructors, which cannot fail: a bounded wait as above; past the deadline the stall is
// reported on stderr and the wait goes on (the buffers the stream uses must not be reused before
// it ends). GPU errors are ignored here.
void drain_stream(hipStream_t s, const std::string &what) noexcept;
// Whether an event's work has finished, for callers that only poll (no error is raised here):
// hipErrorNotReady reads as false, any other error as on_error, and such an error is cleared
// from the thread's last error when it is the one this query left (a later launch check would
// otherwise report it as its own).
inline bool event_query(hipEvent_t e, bool on_error) {
    const hipError_t r = hipEventQuery(e);
    if (r == hipSuccess) return true;
    if (r == hipErrorNotReady) return false;
    if (hipPeekAtLastError() == r) (void)hipGetLastError();
    return on_error;
}

// 64 zero bytes on the current device (allocated once per device, kept until the process ends):
// the kernels' source for out-of-range taps.
const void *zero_block64();

// Size-classed, stream-ordered pool of device buffers (gpu.rs:938-966). hipMalloc is slow and
// synchronising, so scratch buffers are reused. Every buffer has a home stream, the stream its
// last holder queued work on; other streams that touched it are named when it is given back,
// and an event is recorded on each of them then. A buffer is handed out again only for work on
// its home stream (stream order covers its uses there; the recorded events are waited for on
// the GPU, not the host), or once its home stream is retired (synchronised, about to go).
// Sizes are rounded up to classes (2^k and 1.5 * 2^k above 64 KiB) so varied batch shapes share
// buffers; the pool keeps at most `cap` bytes and frees the rest (POOLMB, gpu.rs:919), which
// waits for the device.
class Pool {
  public:
    explicit Pool(size_t cap_bytes) : cap_(cap_bytes) {}
    ~Pool();
    // A buffer of at least `bytes` for work queued on stream s.
    void *get(size_t bytes, hipStream_t s);
    // Gives p back; its holder queued work on `home` and, if given, on the `extra` streams.
    void put(void *p, hipStream_t home, const hipStream_t *extra = nullptr, int nextra = 0);
    // Stream s has finished all its work and is about to be destroyed: buffers given back from
    // it need no wait any more.
    void retire_stream(hipStream_t s);
    void trim();  // free everything held
    size_t held() const { return held_; }
    size_t live() const { return live_; }
    size_t cap() const { return cap_; }
    static size_t size_class(size_t bytes);

  private:
    struct Block {
        void *p;
        hipStream_t home;  // null: no work queued on it anywhere
        std::vector<hipEvent_t> pending;  // recorded on other streams that used the buffer
    };
    hipEvent_t event();
    std::map<size_t, std::vector<Block>> free_;
    std::unordered_map<void *, size_t> size_of_;
    std::vector<hipEvent_t> spare_;
    size_t cap_, held_ = 0, live_ = 0;
    std::mutex mu_;
};

class Ctx;

// Kernel timing with HIP events, for measurement (the role of the reference's OPPROFILE,
// src/gpu.rs:1247-1368, without its waits): while a kernel family is being probed, each launch
// of it is bracketed by two events recorded on the launch's own stream, and its algorithmic
// FLOPs and bytes are added up. Process-wide; families are "conv_igemm", "conv_mfma", "gru", "conv_transpose",
// "conv_direct", "maxpool", "mask_up", "grey_resize", "line_crop", "avgpool_t", "argmax", "copy".
class Probe {
  public:
    static Probe &get();
    void start(const std::string &family);
    // Waits for the recorded events; returns false if the family was not being probed.
    bool stop(const std::string &family, uint32_t *calls, double *ms, double *flops, double *bytes);
    bool active(const char *family);
    void record(const char *family, hipStream_t s, bool begin, double flops, double bytes);

  private:
    struct Fam {
        std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
        double flops = 0, bytes = 0;
        hipEvent_t open = nullptr;
    };
    std::map<std::string, Fam> fams_;
    std::vector<hipEvent_t> spare_;
    std::mutex mu_;
    std::atomic<bool> any_{false};
    hipEvent_t take();
};

// Brackets one launch when its family is probed (no cost otherwise beyond a flag check).
class ProbeScope {
  public:
    ProbeScope(const char *family, hipStream_t s, double flops, double bytes) : fam_(family), s_(s) {
        on_ = Probe::get().active(family);
        if (on_) Probe::get().record(fam_, s_, true, flops, bytes);
    }
    ~ProbeScope() {
        if (on_) Probe::get().record(fam_, s_, false, 0, 0);
    }

  private:
    const char *fam_;
    hipStream_t s_;
    bool on_ = false;
};

// A pooled device buffer owned by one holder; goes back to the pool when destroyed. Its work
// is queued on `stream` (the context's stream unless given); used_on() names another stream
// that reads or writes it, so the pool orders the buffer's next use after that stream's work.
class DBuf {
  public:
    DBuf() = default;
    DBuf(Ctx *ctx, size_t bytes);
    DBuf(Ctx *ctx, size_t bytes, hipStream_t stream);
    DBuf(DBuf &&o) noexcept { *this = std::move(o); }
    DBuf &operator=(DBuf &&o) noexcept;
    DBuf(const DBuf &) = delete;
    DBuf &operator=(const DBuf &) = delete;
    ~DBuf() { reset(); }
    void reset();
    void used_on(hipStream_t s);
    template <class T> T *as() const { return static_cast<T *>(p_); }
    void *get() const { return p_; }
    size_t bytes() const { return bytes_; }
    explicit operator bool() const { return p_ != nullptr; }

  private:
    Ctx *ctx_ = nullptr;
    void *p_ = nullptr;
    size_t bytes_ = 0;
    hipStream_t home_ = nullptr;
    hipStream_t extra_[2] = {nullptr, nullptr};
    int nextra_ = 0;
};

// A weight buffer uploaded once at load time (not pooled).
struct DevWeights {
    void *p = nullptr;
    size_t bytes = 0;
};

class Ctx {
  public:
    Ctx(int device, uint32_t lines, size_t pool_mb);
    ~Ctx();
    int device() const { return device_; }
    // The stream work is queued on: the context's own, unless a StreamScope on the calling
    // thread names another.
    hipStream_t stream() const;
    hipStream_t own_stream() const { return stream_; }
    uint32_t lines() const { return lines_; }
    Pool &pool() { return pool_; }
    void bind() const;  // make this context's device current on the calling thread
    void sync();        // waits for stream()

    // Weights live until the context is destroyed.
    template <class T> const T *upload_weights(const T *data, size_t count) {
        return static_cast<const T *>(upload_raw(data, count * sizeof(T)));
    }
    // Async on stream(): src is copied into a pinned staging ring first, so the call returns
    // at once and src may be reused (a copy from pageable memory would wait for the stream).
    void h2d(void *dst, const void *src, size_t bytes);
    void d2h(void *dst, const void *src, size_t bytes);  // synchronous: waits for stream()

  private:
    const void *upload_raw(const void *data, size_t bytes);
    int device_;
    uint32_t lines_;
    hipStream_t stream_ = nullptr;
    Pool pool_;
    std::vector<void *> weights_;
    // Pinned staging ring of h2d: regions still read by a copy on the stream, oldest first.
    struct Staged {
        size_t begin, end;
        hipEvent_t done;
    };
    char *ring_ = nullptr;
    size_t ring_head_ = 0;
    std::deque<Staged> staged_;
    std::vector<hipEvent_t> spare_events_;
    std::mutex ring_mu_;
};

// While alive, ctx.stream() on this thread is s: everything the models and graphs queue (and
// the pooled buffers they take) goes to s instead of the context's own stream.
class StreamScope {
  public:
    StreamScope(const Ctx &ctx, hipStream_t s);
    ~StreamScope();
    StreamScope(const StreamScope &) = delete;
    StreamScope &operator=(const StreamScope &) = delete;

  private:
    const Ctx *prev_ctx_;
    hipStream_t prev_stream_;
};

}  // namespace ocr
