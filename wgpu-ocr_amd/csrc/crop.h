// Descriptor of one line image cut on the GPU (kernels/crop.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"
#include "geometry.h"

namespace ocr {

struct CropLine {
    const uint8_t *rgb;  // the page's RGB bytes (device)
    int pw, ph;          // page size
    int left, top, bw, bh, out_w;  // crop box on the page and the resized width (LineGeom)
    int row_base;        // index of this line's first row offset in the row_off array
    float *dst;          // the line's slot in its batch: [64][wb] floats (device)
    int wb;              // batch width
};

// All lines in one launch; row_off holds every line's (bh + 1) span offsets (already rebased
// into the shared spans array).
void line_crop(const CropLine *d_lines, int nlines, const int *d_row_off, const int *d_spans, int max_wb,
               hipStream_t s);

}  // namespace ocr
