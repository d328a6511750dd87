// PNG pages to 8-bit RGB: the reference's page decode, image::open(p)?.into_rgb8()
// (src/bin/ocr-bench.rs:424, src/bin/stages.rs:94, src/bin/ppocr-bench.rs:69).
#pragma once

#include <cstddef>
#include <cstdint>

namespace ocr {

struct PngHeader {
    uint32_t w = 0, h = 0;
    int depth = 0;      // bits per sample: 1, 2, 4, 8 or 16
    int color = 0;      // 0 grey, 2 RGB, 3 palette, 4 grey + alpha, 6 RGB + alpha
    int interlace = 0;  // 0 none, 1 Adam7
};

// The signature and the IHDR chunk only (checked, CRC included).
PngHeader png_header(const uint8_t *data, size_t n);

// The whole image as w * h RGB triples, row by row, at out (cap bytes, at least w * h * 3).
// Thread-safe: no state is shared between calls.
PngHeader png_decode_rgb(const uint8_t *data, size_t n, uint8_t *out, size_t cap);

}  // namespace ocr
