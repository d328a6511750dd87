// Descriptor of one line image cut on the GPU (kernels/crop.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "common.h"
#include "geometry.h"
#include "runtime.h"

namespace ocr {

struct CropLine {
    const uint8_t *rgb;  // the page's RGB bytes (device)
    int pw, ph;          // page size
    int left, top, bw, bh, out_w;  // crop box on the page and the resized width (LineGeom)
    int row_base;        // index of this line's first row offset in the row_off array
    float *dst;          // the line's slot in its batch: [64][wb] floats (device)
    int wb;              // batch width
    // Set by line_crop: output tiles of tr rows x tc columns, ntx across the slot, the line's
    // first block.
    int tr = 0, tc = 0, ntx = 0, blk0 = 0;
};

// All lines in one launch; row_off (host memory) holds every line's (bh + 1) span offsets
// (already rebased into the shared spans array). The descriptors, a block-to-line map, the row
// offsets and the spans go to the device as one upload through the context's staging ring.
void line_crop(Ctx &ctx, std::vector<CropLine> &lines, const std::vector<int32_t> &row_off,
               const std::vector<int32_t> &spans, hipStream_t s);

// One PP-OCR line image (ppocr::line_input, src/ppocr.rs:42-62, and ppocr::batch, ppocr.rs:64-78).
struct PpCropLine {
    const uint8_t *rgb;  // the page's RGB bytes (device)
    int pw, ph;          // page size
    int left, top, cw, ch, out_w;  // crop box and resized width (PpLine)
    float *dst;          // the line's slot in its batch: [3][48][wb] floats (device)
    int wb;              // batch width
};
void pp_line_crop(const PpCropLine *d_lines, int nlines, int max_wb, hipStream_t s);

}  // namespace ocr
