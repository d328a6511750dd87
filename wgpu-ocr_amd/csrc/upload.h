// Uploads of page images handed over in host memory (the pages the reference's `run` receives,
// src/bin/ocr-bench.rs:458-585): page-locked memory goes straight to the device; pageable memory
// through a ring of page-locked staging slots, the host copy split between the calling thread and
// two helper threads of the uploader's own, each slot's copy to the device queued on the
// uploader's stream as soon as the slot is filled.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <memory>

#include "runtime.h"

namespace ocr {

// True when p is page-locked host memory (hipHostMalloc), which a copy engine reads directly.
bool host_pinned(const void *p);

class PageUploader {
  public:
    explicit PageUploader(Ctx &ctx);
    ~PageUploader();
    PageUploader(const PageUploader &) = delete;
    PageUploader &operator=(const PageUploader &) = delete;
    // Copies bytes of host memory to dst on stream(); returns once src may be reused (for
    // pageable memory: once its bytes are in the staging slots).
    void upload(uint8_t *dst, const uint8_t *src, size_t bytes, bool pinned);
    hipStream_t stream() const { return up_; }

  private:
    struct Impl;
    Ctx &ctx_;
    hipStream_t up_ = nullptr;
    std::unique_ptr<Impl> impl_;
};

}  // namespace ocr
