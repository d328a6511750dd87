// The allocation-free GPU word boxes (kernels/ccl_noalloc.hip): limits of its fixed device array.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "geometry.h"

namespace ocr {

class Ctx;

// Largest mask: 2^19 words of 32 pixels (2 MiB; a 4096 x 4096 page) and 16384 rows. Runs,
// components and row slots the array holds (past them the host labels the mask instead).
constexpr size_t NOALLOC_MAX_WORDS = size_t(1) << 19;
constexpr int NOALLOC_MAX_H = 16384;
constexpr int NOALLOC_RUNS = 1 << 17, NOALLOC_COMPS = 16384, NOALLOC_SLOTS = 65536;
// The array: mask, row offsets, totals, 14 B a run, 16 B a component, 8 B a row slot.
constexpr size_t NOALLOC_SCRATCH_BYTES = 4784640;  // 4.56 MiB

// Looks up the array's address on `device` (the current device); once per device, when a
// context is created on it.
void noalloc_init(int device);

// word_rects_gpu's rectangles with the labelling in the fixed array: no device allocation.
// Fails for masks larger than the array holds.
std::vector<RRect> word_rects_gpu_noalloc(Ctx &c, const uint32_t *bits, int w, int h);

}  // namespace ocr
