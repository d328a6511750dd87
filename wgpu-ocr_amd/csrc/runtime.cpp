#include "runtime.h"

#include <cstdio>
#include <cstring>

namespace ocr {

namespace {
std::atomic<uint64_t> g_device_allocs{0}, g_host_allocs{0};
}  // namespace

hipError_t try_device_malloc(void **p, size_t bytes) {
    g_device_allocs.fetch_add(1, std::memory_order_relaxed);
    return hipMalloc(p, bytes);
}

void device_malloc(void **p, size_t bytes) { OCR_HIP(try_device_malloc(p, bytes)); }

void host_malloc(void **p, size_t bytes) {
    g_host_allocs.fetch_add(1, std::memory_order_relaxed);
    OCR_HIP(hipHostMalloc(p, bytes, hipHostMallocDefault));
}

uint64_t device_allocations() { return g_device_allocs.load(std::memory_order_relaxed); }
uint64_t host_allocations() { return g_host_allocs.load(std::memory_order_relaxed); }

void wait_event(hipEvent_t ev, const std::string &what, bool spin) {
    wait_until(
        [&] {
            const hipError_t e = hipEventQuery(ev);
            if (e == hipSuccess) return true;
            if (e != hipErrorNotReady) OCR_HIP(e);
            return false;
        },
        [&] {
            char b[48];
            std::snprintf(b, sizeof b, " (event %p)", static_cast<void *>(ev));
            return what + b;
        },
        spin);
}

void wait_stream(hipStream_t s, const std::string &what, bool spin) {
    wait_until(
        [&] {
            const hipError_t e = hipStreamQuery(s);
            if (e == hipSuccess) return true;
            if (e != hipErrorNotReady) OCR_HIP(e);
            return false;
        },
        [&] {
            char b[48];
            std::snprintf(b, sizeof b, " (stream %p)", static_cast<void *>(s));
            return what + b;
        },
        spin);
}

void drain_stream(hipStream_t s, const std::string &what) noexcept {
    try {
        wait_stream(s, what);
        return;
    } catch (const WaitTimeout &e) {
        std::fprintf(stderr, "ocrhip: %s; still waiting\n", e.what());
        std::fflush(stderr);
    } catch (...) {
    }
    (void)hipStreamSynchronize(s);
}

const void *zero_block64() {
    constexpr int MAX_DEV = 64;
    static std::mutex mu;
    static void *blocks[MAX_DEV] = {};
    int dev = 0;
    OCR_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEV) fail("zero block: device index " + std::to_string(dev));
    std::lock_guard<std::mutex> lk(mu);
    if (!blocks[dev]) {
        void *z = nullptr;
        device_malloc(&z, 64);
        OCR_HIP(hipMemset(z, 0, 64));
        blocks[dev] = z;
    }
    return blocks[dev];
}

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
        wait_event(pr.second, "the end of a probed " + family + " launch", true);
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

Pool::~Pool() {
    trim();
    for (hipEvent_t e : spare_) (void)hipEventDestroy(e);
}

hipEvent_t Pool::event() {
    if (!spare_.empty()) {
        hipEvent_t e = spare_.back();
        spare_.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    OCR_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    return e;
}

void *Pool::get(size_t bytes, hipStream_t s) {
    size_t sz = size_class(bytes);
    {
        std::lock_guard<std::mutex> lk(mu_);
        auto it = free_.find(sz);
        if (it != free_.end() && !it->second.empty()) {
            std::vector<Block> &v = it->second;
            // The newest buffer whose home is s (stream order covers its earlier uses there) and
            // whose uses on other streams have finished, else the newest whose home is s (s then
            // waits for those uses on the GPU), else the newest idle one. A buffer still homed on
            // another stream is not taken: an event recorded on that stream now would also wait
            // for everything queued there since, and serialise the streams.
            auto settled = [](const Block &b) {
                for (hipEvent_t e : b.pending)
                    if (!event_query(e, false)) return false;
                return true;
            };
            long pick = -1;
            for (size_t k = v.size(); k-- > 0;)
                if (v[k].home == s && settled(v[k])) {
                    pick = long(k);
                    break;
                }
            if (pick < 0)
                for (size_t k = v.size(); k-- > 0;)
                    if (v[k].home == s) {
                        pick = long(k);
                        break;
                    }
            if (pick < 0)
                for (size_t k = v.size(); k-- > 0;)
                    if (v[k].home == nullptr) {
                        pick = long(k);
                        break;
                    }
            if (pick >= 0) {
                Block b = std::move(v[size_t(pick)]);
                v.erase(v.begin() + pick);
                for (hipEvent_t e : b.pending) {
                    OCR_HIP(hipStreamWaitEvent(s, e, 0));
                    spare_.push_back(e);  // reusable: the wait above captured its state
                }
                held_ -= sz;
                live_ += sz;
                return b.p;
            }
        }
    }
    void *p = nullptr;
    hipError_t e = try_device_malloc(&p, sz);
    if (e != hipSuccess) {
        // Out of memory: give back what the pool holds and try once more.
        (void)hipGetLastError();
        trim();
        device_malloc(&p, sz);
    }
    std::lock_guard<std::mutex> lk(mu_);
    size_of_[p] = sz;
    live_ += sz;
    return p;
}

void Pool::put(void *p, hipStream_t home, const hipStream_t *extra, int nextra) {
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
    Block b{p, home, {}};
    for (int k = 0; k < nextra; k++) {
        if (!extra[k] || extra[k] == home) continue;
        hipEvent_t e = event();
        OCR_HIP(hipEventRecord(e, extra[k]));
        b.pending.push_back(e);
    }
    held_ += sz;
    free_[sz].push_back(std::move(b));
}

void Pool::retire_stream(hipStream_t s) {
    std::lock_guard<std::mutex> lk(mu_);
    for (auto &kv : free_)
        for (Block &b : kv.second)
            if (b.home == s) b.home = nullptr;
}

void Pool::trim() {
    std::lock_guard<std::mutex> lk(mu_);
    for (auto &kv : free_)
        for (Block &b : kv.second) {
            (void)hipFree(b.p);
            size_of_.erase(b.p);
            for (hipEvent_t e : b.pending) spare_.push_back(e);
        }
    free_.clear();
    held_ = 0;
}

DBuf::DBuf(Ctx *ctx, size_t bytes) : DBuf(ctx, bytes, ctx->stream()) {}

DBuf::DBuf(Ctx *ctx, size_t bytes, hipStream_t stream) : ctx_(ctx), bytes_(bytes), home_(stream) {
    p_ = ctx->pool().get(bytes, stream);
}

DBuf &DBuf::operator=(DBuf &&o) noexcept {
    if (this != &o) {
        reset();
        ctx_ = o.ctx_;
        p_ = o.p_;
        bytes_ = o.bytes_;
        home_ = o.home_;
        nextra_ = o.nextra_;
        extra_[0] = o.extra_[0], extra_[1] = o.extra_[1];
        o.p_ = nullptr;
        o.ctx_ = nullptr;
        o.bytes_ = 0;
        o.nextra_ = 0;
    }
    return *this;
}

void DBuf::used_on(hipStream_t s) {
    if (s == home_) return;
    for (int k = 0; k < nextra_; k++)
        if (extra_[k] == s) return;
    if (nextra_ == 2) fail("DBuf::used_on: more than two extra streams");
    extra_[nextra_++] = s;
}

void DBuf::reset() {
    if (p_ && ctx_) ctx_->pool().put(p_, home_, extra_, nextra_);
    p_ = nullptr;
    ctx_ = nullptr;
    bytes_ = 0;
    nextra_ = 0;
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
    if (stream_) drain_stream(stream_, "the context's stream before it is destroyed");
    for (const Staged &st : staged_) (void)hipEventDestroy(st.done);
    for (hipEvent_t e : spare_events_) (void)hipEventDestroy(e);
    if (ring_) (void)hipHostFree(ring_);
    pool_.trim();
    for (void *p : weights_) (void)hipFree(p);
    if (stream_) (void)hipStreamDestroy(stream_);
}

namespace {
thread_local const Ctx *tl_ctx = nullptr;
thread_local hipStream_t tl_stream = nullptr;
}  // namespace

hipStream_t Ctx::stream() const { return tl_ctx == this && tl_stream ? tl_stream : stream_; }

StreamScope::StreamScope(const Ctx &ctx, hipStream_t s) : prev_ctx_(tl_ctx), prev_stream_(tl_stream) {
    tl_ctx = &ctx;
    tl_stream = s;
}

StreamScope::~StreamScope() {
    tl_ctx = prev_ctx_;
    tl_stream = prev_stream_;
}

void Ctx::bind() const { OCR_HIP(hipSetDevice(device_)); }

void Ctx::sync() { wait_stream(stream(), "the context's work on device " + std::to_string(device_)); }

const void *Ctx::upload_raw(const void *data, size_t bytes) {
    void *p = nullptr;
    device_malloc(&p, bytes ? bytes : 16);
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
        OCR_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream()));
        return;
    }
    std::lock_guard<std::mutex> lk(ring_mu_);
    if (!ring_) {
        void *ring = nullptr;
        host_malloc(&ring, RING_BYTES);
        ring_ = static_cast<char *>(ring);
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
        wait_event(staged_.front().done, "an upload still reading the staging ring", true);
        spare_events_.push_back(staged_.front().done);
        staged_.pop_front();
    }
    std::memcpy(ring_ + b, src, bytes);
    const hipStream_t st = stream();
    OCR_HIP(hipMemcpyAsync(dst, ring_ + b, bytes, hipMemcpyHostToDevice, st));
    hipEvent_t ev = nullptr;
    if (!spare_events_.empty()) {
        ev = spare_events_.back();
        spare_events_.pop_back();
    } else {
        OCR_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    }
    OCR_HIP(hipEventRecord(ev, st));
    staged_.push_back({b, e, ev});
    ring_head_ = e;
}

void Ctx::d2h(void *dst, const void *src, size_t bytes) {
    const hipStream_t st = stream();
    if (bytes) OCR_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st));
    wait_stream(st, "a device-to-host copy of " + std::to_string(bytes) + " bytes");
}

}  // namespace ocr
