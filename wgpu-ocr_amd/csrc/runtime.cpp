#include "runtime.h"

#include <cstdio>
#include <cstring>

namespace ocr {

void fail(const std::string &msg) { throw Error(msg); }

Probe &Probe::get() {
    static Probe p;
    return p;
}

hipEvent_t Probe::take() {
    if (!spare_.empty()) {
        hipEvent_t e = spare_.back();
        spare_.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    OCR_HIP(hipEventCreate(&e));
    return e;
}

void Probe::start(const std::string &family) {
    std::lock_guard<std::mutex> lk(mu_);
    Fam &f = fams_[family];
    for (auto &pr : f.ev) spare_.push_back(pr.first), spare_.push_back(pr.second);
    f = Fam{};
    any_ = true;
}

bool Probe::active(const char *family) {
    if (!any_) return false;
    std::lock_guard<std::mutex> lk(mu_);
    return fams_.count(family) > 0;
}

void Probe::record(const char *family, hipStream_t s, bool begin, double flops, double bytes) {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = fams_.find(family);
    if (it == fams_.end()) return;
    Fam &f = it->second;
    hipEvent_t e = take();
    OCR_HIP(hipEventRecord(e, s));
    if (begin) {
        f.open = e;
        f.flops += flops;
        f.bytes += bytes;
    } else if (f.open) {
        f.ev.push_back({f.open, e});
        f.open = nullptr;
    }
}

bool Probe::stop(const std::string &family, uint32_t *calls, double *ms, double *flops, double *bytes) {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = fams_.find(family);
    if (it == fams_.end()) return false;
    Fam &f = it->second;
    double total = 0;
    for (auto &pr : f.ev) {
        OCR_HIP(hipEventSynchronize(pr.second));
        float t = 0;
        OCR_HIP(hipEventElapsedTime(&t, pr.first, pr.second));
        total += t;
        spare_.push_back(pr.first);
        spare_.push_back(pr.second);
    }
    if (calls) *calls = uint32_t(f.ev.size());
    if (ms) *ms = total;
    if (flops) *flops = f.flops;
    if (bytes) *bytes = f.bytes;
    fams_.erase(it);
    any_ = !fams_.empty();
    return true;
}

size_t Pool::size_class(size_t bytes) {
    bytes = (bytes + 255) & ~size_t(255);
    if (bytes <= (64u << 10)) return bytes ? bytes : 256;
    size_t p = 1;
    while (p < bytes) p <<= 1;
    size_t mid = p / 2 + p / 4;  // 1.5 * 2^(k-1)
    return mid >= bytes ? mid : p;
}

Pool::~Pool() { trim(); }

void *Pool::get(size_t bytes) {
    size_t sz = size_class(bytes);
    {
        std::lock_guard<std::mutex> lk(mu_);
        auto it = free_.find(sz);
        if (it != free_.end() && !it->second.empty()) {
            void *p = it->second.back();
            it->second.pop_back();
            held_ -= sz;
            live_ += sz;
            return p;
        }
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) {
        // Out of memory: give back what the pool holds and try once more.
        trim();
        OCR_HIP(hipMalloc(&p, sz));
    }
    std::lock_guard<std::mutex> lk(mu_);
    size_of_[p] = sz;
    live_ += sz;
    return p;
}

void Pool::put(void *p) {
    if (!p) return;
    std::lock_guard<std::mutex> lk(mu_);
    auto it = size_of_.find(p);
    if (it == size_of_.end()) return;
    size_t sz = it->second;
    live_ -= sz;
    if (held_ + sz > cap_) {
        size_of_.erase(it);
        // hipFree waits for the device to finish with the buffer.
        (void)hipFree(p);
        return;
    }
    held_ += sz;
    free_[sz].push_back(p);
}

void Pool::trim() {
    std::lock_guard<std::mutex> lk(mu_);
    for (auto &kv : free_)
        for (void *p : kv.second) {
            (void)hipFree(p);
            size_of_.erase(p);
        }
    free_.clear();
    held_ = 0;
}

DBuf::DBuf(Ctx *ctx, size_t bytes) : ctx_(ctx), bytes_(bytes) { p_ = ctx->pool().get(bytes); }

DBuf &DBuf::operator=(DBuf &&o) noexcept {
    if (this != &o) {
        reset();
        ctx_ = o.ctx_;
        p_ = o.p_;
        bytes_ = o.bytes_;
        o.p_ = nullptr;
        o.ctx_ = nullptr;
        o.bytes_ = 0;
    }
    return *this;
}

void DBuf::reset() {
    if (p_ && ctx_) ctx_->pool().put(p_);
    p_ = nullptr;
    ctx_ = nullptr;
    bytes_ = 0;
}

Ctx::Ctx(int device, uint32_t lines, size_t pool_mb) : device_(device), lines_(lines), pool_(pool_mb << 20) {
    int count = 0;
    OCR_HIP(hipGetDeviceCount(&count));
    if (device < 0 || device >= count)
        fail("device " + std::to_string(device) + " not present (" + std::to_string(count) + " visible)");
    OCR_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    OCR_HIP(hipGetDeviceProperties(&prop, device));
    if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0)
        fail(std::string("this library is built for gfx950; device is ") + prop.gcnArchName);
    OCR_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
}

Ctx::~Ctx() {
    (void)hipSetDevice(device_);
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (const Staged &st : staged_) (void)hipEventDestroy(st.done);
    for (hipEvent_t e : spare_events_) (void)hipEventDestroy(e);
    if (ring_) (void)hipHostFree(ring_);
    pool_.trim();
    for (void *p : weights_) (void)hipFree(p);
    if (stream_) (void)hipStreamDestroy(stream_);
}

void Ctx::bind() const { OCR_HIP(hipSetDevice(device_)); }

void Ctx::sync() { OCR_HIP(hipStreamSynchronize(stream_)); }

const void *Ctx::upload_raw(const void *data, size_t bytes) {
    void *p = nullptr;
    OCR_HIP(hipMalloc(&p, bytes ? bytes : 16));
    weights_.push_back(p);
    if (bytes) OCR_HIP(hipMemcpy(p, data, bytes, hipMemcpyHostToDevice));
    return p;
}

namespace {
constexpr size_t RING_BYTES = size_t(32) << 20;
}

void Ctx::h2d(void *dst, const void *src, size_t bytes) {
    if (!bytes) return;
    if (bytes > RING_BYTES / 4) {
        // Large uploads (whole pages, inputs) go straight from the caller's memory.
        OCR_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream_));
        return;
    }
    std::lock_guard<std::mutex> lk(ring_mu_);
    if (!ring_) {
        OCR_HIP(hipHostMalloc(reinterpret_cast<void **>(&ring_), RING_BYTES, hipHostMallocDefault));
        // Fault every page in now (a page's first CPU write runs at about 2 GB/s, later ones at
        // memory speed), not while a run stages its tables.
        std::memset(ring_, 0, RING_BYTES);
    }
    const size_t need = (bytes + 255) & ~size_t(255);
    if (ring_head_ + need > RING_BYTES) ring_head_ = 0;
    const size_t b = ring_head_, e = b + need;
    // Copies that have finished give their regions back; a region still being read by a copy
    // on the stream is waited for (oldest first) before it is written again.
    while (!staged_.empty() && hipEventQuery(staged_.front().done) == hipSuccess) {
        spare_events_.push_back(staged_.front().done);
        staged_.pop_front();
    }
    auto overlaps = [&] {
        for (const Staged &st : staged_)
            if (st.begin < e && b < st.end) return true;
        return false;
    };
    while (overlaps()) {
        OCR_HIP(hipEventSynchronize(staged_.front().done));
        spare_events_.push_back(staged_.front().done);
        staged_.pop_front();
    }
    std::memcpy(ring_ + b, src, bytes);
    OCR_HIP(hipMemcpyAsync(dst, ring_ + b, bytes, hipMemcpyHostToDevice, stream_));
    hipEvent_t ev = nullptr;
    if (!spare_events_.empty()) {
        ev = spare_events_.back();
        spare_events_.pop_back();
    } else {
        OCR_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    }
    OCR_HIP(hipEventRecord(ev, stream_));
    staged_.push_back({b, e, ev});
    ring_head_ = e;
}

void Ctx::d2h(void *dst, const void *src, size_t bytes) {
    if (bytes) OCR_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream_));
    OCR_HIP(hipStreamSynchronize(stream_));
}

}  // namespace ocr
