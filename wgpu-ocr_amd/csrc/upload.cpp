#include "upload.h"

#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>
#if !defined(__HIP_DEVICE_COMPILE__)
#include <immintrin.h>
#endif

#include "host_util.h"

namespace ocr {

namespace {

// Pinned staging of pages handed over in pageable host memory: SLOTS buffers of SLOT_BYTES,
// each reused once the copy out of it has finished.
constexpr int SLOTS = 6;
constexpr size_t SLOT_BYTES = size_t(8) << 20;
// Threads that help the stager thread copy a slot (the pipeline's own: the shared loop pool's
// threads run the page layouts, and a copy queued behind their chunks left PCIe idle).
constexpr int COPY_HELPERS = 2;

// memcpy with non-temporal stores (no read of the destination's lines into the cache: 34 GB/s
// a thread against 25 on the MI355X host), for 32-byte aligned destinations on AVX2 hosts.
#if defined(__HIP_DEVICE_COMPILE__)
void stream_copy(void *dst, const void *src, size_t n) { std::memcpy(dst, src, n); }
#else
__attribute__((target("avx2"))) void stream_copy_avx2(char *d, const char *s, size_t n) {
    size_t i = 0;
    for (; i + 128 <= n; i += 128) {
        const __m256i a = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(s + i));
        const __m256i b = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(s + i + 32));
        const __m256i c = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(s + i + 64));
        const __m256i e = _mm256_loadu_si256(reinterpret_cast<const __m256i *>(s + i + 96));
        _mm256_stream_si256(reinterpret_cast<__m256i *>(d + i), a);
        _mm256_stream_si256(reinterpret_cast<__m256i *>(d + i + 32), b);
        _mm256_stream_si256(reinterpret_cast<__m256i *>(d + i + 64), c);
        _mm256_stream_si256(reinterpret_cast<__m256i *>(d + i + 96), e);
    }
    std::memcpy(d + i, s + i, n - i);
    _mm_sfence();  // the stores are visible before the copy engine is told to read them
}
void stream_copy(void *dst, const void *src, size_t n) {
    static const bool avx2 = __builtin_cpu_supports("avx2");
    if (avx2 && (reinterpret_cast<uintptr_t>(dst) & 31) == 0)
        stream_copy_avx2(static_cast<char *>(dst), static_cast<const char *>(src), n);
    else
        std::memcpy(dst, src, n);
}
#endif

// The stager thread and COPY_HELPERS threads of its own copy one buffer in as many pieces
// (64-byte aligned cuts); copy() returns when every piece is done.
class CopyCrew {
  public:
    explicit CopyCrew(int helpers) : parts_(helpers + 1) {
        for (int k = 1; k <= helpers; k++) th_.emplace_back([this, k] { loop(k); });
    }
    ~CopyCrew() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : th_) t.join();
    }
    void copy(void *dst, const void *src, size_t n) {
        {
            std::lock_guard<std::mutex> lk(mu_);
            dst_ = static_cast<char *>(dst), src_ = static_cast<const char *>(src), n_ = n;
            left_ = parts_ - 1;
            gen_++;
        }
        cv_.notify_all();
        piece(0);
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return left_ == 0; });
    }

  private:
    void piece(int k) {
        auto cut = [&](int j) { return j == parts_ ? n_ : (n_ * size_t(j) / size_t(parts_)) & ~size_t(63); };
        const size_t a = cut(k), b = cut(k + 1);
        if (b > a) stream_copy(dst_ + a, src_ + a, b - a);
    }
    void loop(int k) {
        long seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            piece(k);
            std::lock_guard<std::mutex> lk(mu_);
            if (--left_ == 0) done_cv_.notify_all();
        }
    }
    std::vector<std::thread> th_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    long gen_ = 0;
    int left_ = 0;
    const int parts_;
    bool stop_ = false;
    char *dst_ = nullptr;
    const char *src_ = nullptr;
    size_t n_ = 0;
};

}  // namespace

// True when p is page-locked host memory (hipHostMalloc), which a copy engine reads directly.
bool host_pinned(const void *p) {
    hipPointerAttribute_t a{};
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();  // pageable memory is not known to HIP: not an error
        return false;
    }
    return a.type == hipMemoryTypeHost;
}

struct PageUploader::Impl {
    CopyCrew crew{COPY_HELPERS};
    Pinned slot[SLOTS];
    hipEvent_t slot_ev[SLOTS] = {};
    bool slot_used[SLOTS] = {};
    int next_slot = 0;
};

PageUploader::PageUploader(Ctx &ctx) : ctx_(ctx), impl_(new Impl) {
    ctx_.bind();
    OCR_HIP(hipStreamCreateWithFlags(&up_, hipStreamNonBlocking));
    for (hipEvent_t &e : impl_->slot_ev) OCR_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
}

PageUploader::~PageUploader() {
    if (up_) {
        drain_stream(up_, "the upload stream");
        ctx_.pool().retire_stream(up_);
        (void)hipStreamDestroy(up_);
    }
    for (hipEvent_t e : impl_->slot_ev)
        if (e) (void)hipEventDestroy(e);
}

void PageUploader::upload(uint8_t *dst, const uint8_t *src, size_t bytes, bool pinned) {
    if (pinned) {
        OCR_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, up_));
        return;
    }
    Impl &I = *impl_;
    for (size_t off = 0; off < bytes; off += SLOT_BYTES) {
        const size_t n = std::min(SLOT_BYTES, bytes - off);
        const int k = I.next_slot;
        I.next_slot = (I.next_slot + 1) % SLOTS;
        I.slot[k].ensure(SLOT_BYTES);
        if (I.slot_used[k]) wait_event(I.slot_ev[k], "the upload reading staging slot " + std::to_string(k), true);
        uint8_t *stage = static_cast<uint8_t *>(I.slot[k].p);
        I.crew.copy(stage, src + off, n);
        OCR_HIP(hipMemcpyAsync(dst + off, stage, n, hipMemcpyHostToDevice, up_));
        OCR_HIP(hipEventRecord(I.slot_ev[k], up_));
        I.slot_used[k] = true;
    }
}

}  // namespace ocr
