// The GPU word boxes without any device allocation (ocr_word_rects_gpu_noalloc): the labelling
// kernels of ccl.hip run on one fixed device array of this file instead of pooled buffers, for
// callers that cannot call hipMalloc (serving loops, harnesses that forbid it).
//
// Each GPU holds its own copy of `scratch` at its own address. The address is looked up once
// per device, with that device current, when a context is created on it (noalloc_init), and
// only that address is handed to HIP calls and kernels afterwards: in host code the array's
// name is a host-side stand-in, not a device address. Calls on one device share the array, so
// they are serialised by a per-device lock here (two calls that overlapped would race on it).
// Every kernel writes what it later reads (row offsets and totals by the count and scan passes,
// run records by the run pass, slots by the component pass), so nothing needs clearing between
// calls and a call never sees the previous call's contents.
#include <hip/hip_runtime.h>

#include <exception>
#include <mutex>
#include <string>
#include <vector>

#include "../geometry.h"
#include "../kernels.h"
#include "../noalloc.h"
#include "../runtime.h"

namespace ocr {

namespace {

constexpr size_t round256(size_t b) { return (b + 255) & ~size_t(255); }

// Region offsets inside the array (each 256-byte aligned).
constexpr size_t OFF_BITS = 0;
constexpr size_t OFF_ROWOFF = OFF_BITS + round256(NOALLOC_MAX_WORDS * 4);
constexpr size_t OFF_TOTAL = OFF_ROWOFF + round256(size_t(NOALLOC_MAX_H + 1) * 4);
constexpr size_t OFF_X0 = OFF_TOTAL + round256(16);
constexpr size_t OFF_X1 = OFF_X0 + round256(size_t(NOALLOC_RUNS) * 2);
constexpr size_t OFF_RY = OFF_X1 + round256(size_t(NOALLOC_RUNS) * 2);
constexpr size_t OFF_ROOT = OFF_RY + round256(size_t(NOALLOC_RUNS) * 2);
constexpr size_t OFF_CBOT = OFF_ROOT + round256(size_t(NOALLOC_RUNS) * 4);
constexpr size_t OFF_COMPS = OFF_CBOT + round256(size_t(NOALLOC_RUNS) * 4);
constexpr size_t OFF_XMIN = OFF_COMPS + round256(size_t(NOALLOC_COMPS) * 16);
constexpr size_t OFF_XMAX = OFF_XMIN + round256(size_t(NOALLOC_SLOTS) * 4);
constexpr size_t SCRATCH_BYTES = OFF_XMAX + round256(size_t(NOALLOC_SLOTS) * 4);
static_assert(SCRATCH_BYTES == NOALLOC_SCRATCH_BYTES, "scratch layout and its stated size disagree");

static __device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_init_mu;
void *g_scratch[MAX_DEVICES];       // the array's device address on each device (null: not set up)
std::mutex g_call_mu[MAX_DEVICES];  // one call at a time per device

// Leaving a call by an exception after its kernels were queued: wait for the stream before the
// device's lock is released, or the next call would overwrite the array under those kernels.
struct SyncOnUnwind {
    hipStream_t st;
    int uncaught = std::uncaught_exceptions();
    ~SyncOnUnwind() {
        if (std::uncaught_exceptions() <= uncaught) return;
        try {
            wait_stream(st, "the labelling kernels of a failed allocation-free call");
        } catch (...) {
        }
    }
};

}  // namespace

void noalloc_init(int device) {
    if (device < 0 || device >= MAX_DEVICES) fail("noalloc scratch: device index " + std::to_string(device));
    std::lock_guard<std::mutex> lk(g_init_mu);
    if (g_scratch[device]) return;
    int cur = -1;
    OCR_HIP(hipGetDevice(&cur));
    if (cur != device) fail("noalloc scratch: set up with device " + std::to_string(cur) + " current, not " +
                            std::to_string(device));
    void *p = nullptr;
    OCR_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) fail("noalloc scratch: no device address");
    g_scratch[device] = p;
}

std::vector<RRect> word_rects_gpu_noalloc(Ctx &c, const uint32_t *bits, int w, int h) {
    if (w < 1 || h < 1 || w > 65536) fail("ocr_word_rects_gpu_noalloc: mask size");
    if (h > NOALLOC_MAX_H)
        fail("ocr_word_rects_gpu_noalloc: " + std::to_string(h) + " rows exceed the fixed scratch's " +
             std::to_string(NOALLOC_MAX_H));
    const size_t words = size_t(w + 31) / 32 * size_t(h);
    if (words > NOALLOC_MAX_WORDS)
        fail("ocr_word_rects_gpu_noalloc: a mask of " + std::to_string(words) + " words exceeds the fixed scratch's " +
             std::to_string(NOALLOC_MAX_WORDS));
    const int dev = c.device();
    void *base = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_init_mu);
        if (dev >= 0 && dev < MAX_DEVICES) base = g_scratch[dev];
    }
    if (!base) fail("ocr_word_rects_gpu_noalloc: scratch not set up on device " + std::to_string(dev));
    std::lock_guard<std::mutex> call(g_call_mu[dev]);
    c.bind();
    unsigned char *s = static_cast<unsigned char *>(base);
    const hipStream_t st = c.stream();
    SyncOnUnwind drain{st};
    OCR_HIP(hipMemcpyAsync(s + OFF_BITS, bits, words * 4, hipMemcpyHostToDevice, st));
    CclPage pg{};
    pg.bits = reinterpret_cast<const uint32_t *>(s + OFF_BITS), pg.w = w, pg.h = h;
    pg.row_off = reinterpret_cast<int32_t *>(s + OFF_ROWOFF);
    pg.total = reinterpret_cast<int32_t *>(s + OFF_TOTAL);
    pg.x0 = reinterpret_cast<uint16_t *>(s + OFF_X0), pg.x1 = reinterpret_cast<uint16_t *>(s + OFF_X1);
    pg.ry = reinterpret_cast<uint16_t *>(s + OFF_RY);
    pg.root = reinterpret_cast<int32_t *>(s + OFF_ROOT), pg.cbot = reinterpret_cast<int32_t *>(s + OFF_CBOT);
    pg.comps = reinterpret_cast<int32_t *>(s + OFF_COMPS);
    pg.xmin = reinterpret_cast<uint32_t *>(s + OFF_XMIN), pg.xmax = reinterpret_cast<uint32_t *>(s + OFF_XMAX);
    pg.cap = NOALLOC_RUNS, pg.ccap = NOALLOC_COMPS, pg.scap = NOALLOC_SLOTS;
    ccl_runs(&pg, 1, st);
    int32_t tot[4] = {0, 0, 0, 0};
    OCR_HIP(hipMemcpyAsync(tot, pg.total, 16, hipMemcpyDeviceToHost, st));
    wait_stream(st, "the allocation-free labelling of a " + std::to_string(w) + " x " + std::to_string(h) + " mask");
    // More runs, components or row slots than the array holds: the host labels the mask from
    // the bits (the same rectangles; see word_rects_from_rows).
    if (tot[0] > NOALLOC_RUNS || tot[1] > NOALLOC_COMPS || tot[2] > NOALLOC_SLOTS) return word_rects(bits, w, h);
    const size_t nc = size_t(tot[1]), ns = size_t(tot[2]);
    std::vector<int32_t> comps(nc * 4);
    std::vector<uint32_t> xmin(ns), xmax(ns);
    if (nc) {
        OCR_HIP(hipMemcpyAsync(comps.data(), pg.comps, nc * 16, hipMemcpyDeviceToHost, st));
        OCR_HIP(hipMemcpyAsync(xmin.data(), pg.xmin, ns * 4, hipMemcpyDeviceToHost, st));
        OCR_HIP(hipMemcpyAsync(xmax.data(), pg.xmax, ns * 4, hipMemcpyDeviceToHost, st));
        wait_stream(st, "the copies of the allocation-free labelling's records");
    }
    return word_rects_from_rows(bits, w, h, comps.data(), int(nc), xmin.data(), xmax.data(), int(ns));
}

}  // namespace ocr
