// Shared definitions of the ocrhip host library: errors and the activation tensor view.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace ocr {

// Every failure inside the library is an ocr::Error; the C ABI turns it into a status code and
// a thread-local message (the reference returns Result<_, String> everywhere, src/gpu.rs).
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] void fail(const std::string &msg);

// Every device and page-locked host allocation the library makes goes through these two, so
// they can be counted (ocr_memory_stats): callers that must not allocate can check a path.
void device_malloc(void **p, size_t bytes);
void host_malloc(void **p, size_t bytes);

#define OCR_HIP(call)                                                                              \
    do {                                                                                           \
        hipError_t e_ = (call);                                                                    \
        if (e_ != hipSuccess)                                                                      \
            ::ocr::fail(std::string(#call) + ": " + hipGetErrorString(e_));                        \
    } while (0)

// An activation tensor on the device: NHWC float32, possibly a channel slice of a wider buffer
// (the producers of a Concat write straight into their channel range). Pixel (n, y, x) starts
// at p + ((n * h + y) * w + x) * cs.
struct Act {
    float *p = nullptr;
    int n = 0, h = 0, w = 0, c = 0;
    int cs = 0;  // pixel stride in floats, >= c
    size_t pixels() const { return size_t(n) * h * w; }
    size_t count() const { return pixels() * c; }
};

// Activation functions of the epilogues (gpu.rs:28-34): 0 none, 1 ReLU, 2 sigmoid, 3 GELU, 4 SiLU.
enum ActKind : int { ACT_NONE = 0, ACT_RELU = 1, ACT_SIGMOID = 2, ACT_GELU = 3, ACT_SILU = 4 };

}  // namespace ocr
