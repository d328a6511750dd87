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

namespace ocr {

// Size-classed, stream-ordered pool of device buffers (gpu.rs:938-966). hipMalloc is slow and
// synchronising, so scratch buffers are reused: a buffer given back is handed out again for
// later work on the same stream, which stream order makes safe without any wait. Sizes are
// rounded up to classes (2^k and 1.5 * 2^k above 64 KiB) so varied batch shapes share buffers;
// the pool keeps at most `cap` bytes and frees the rest (POOLMB, gpu.rs:919).
class Pool {
  public:
    explicit Pool(size_t cap_bytes) : cap_(cap_bytes) {}
    ~Pool();
    void *get(size_t bytes);
    void put(void *p);
    void trim();  // free everything held
    size_t held() const { return held_; }
    size_t live() const { return live_; }
    static size_t size_class(size_t bytes);

  private:
    std::map<size_t, std::vector<void *>> free_;
    std::unordered_map<void *, size_t> size_of_;
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

// A pooled device buffer owned by one holder; goes back to the pool when destroyed.
class DBuf {
  public:
    DBuf() = default;
    DBuf(Ctx *ctx, size_t bytes);
    DBuf(DBuf &&o) noexcept { *this = std::move(o); }
    DBuf &operator=(DBuf &&o) noexcept;
    DBuf(const DBuf &) = delete;
    DBuf &operator=(const DBuf &) = delete;
    ~DBuf() { reset(); }
    void reset();
    template <class T> T *as() const { return static_cast<T *>(p_); }
    void *get() const { return p_; }
    size_t bytes() const { return bytes_; }
    explicit operator bool() const { return p_ != nullptr; }

  private:
    Ctx *ctx_ = nullptr;
    void *p_ = nullptr;
    size_t bytes_ = 0;
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
    hipStream_t stream() const { return stream_; }
    uint32_t lines() const { return lines_; }
    Pool &pool() { return pool_; }
    void bind() const;  // make this context's device current on the calling thread
    void sync();

    // Weights live until the context is destroyed.
    template <class T> const T *upload_weights(const T *data, size_t count) {
        return static_cast<const T *>(upload_raw(data, count * sizeof(T)));
    }
    // Async on the stream: src is copied into a pinned staging ring first, so the call returns
    // at once and src may be reused (a copy from pageable memory would wait for the stream).
    void h2d(void *dst, const void *src, size_t bytes);
    void d2h(void *dst, const void *src, size_t bytes);  // synchronous: waits for the stream

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

}  // namespace ocr
