// Line images for the recogniser, cut on the GPU straight from the page's RGB bytes in HBM: the
// role of ocrs' prepare_recognition_input (called at src/bin/ocr-bench.rs:378) and of the batch
// assembly after it (ocr-bench.rs:388-404). For each line: the pixels inside its polygon (row
// spans computed on the host) take the ocrs grey value of the page (the same formula as the
// detector front end, src/gpu.rs:542), everything else is black (-0.5); that crop is resized to
// 64 rows and out_w columns bilinearly with half-pixel centres, clamped (rten's resize_image),
// and written into the line's slot of its batch, padded with black to the batch width.
#include <hip/hip_runtime.h>

#include "../crop.h"
#include "../runtime.h"

namespace ocr {

namespace {

// mix as the reference states it, each operation rounded on its own (no contraction).
__device__ inline float mixf(float a, float b, float t) {
#pragma clang fp contract(off)
    return a * (1.f - t) + b * t;
}

__device__ inline float grey_px(const uint8_t *rgb, int w, int h, int x, int y) {
#pragma clang fp contract(off)
    if (x < 0 || y < 0 || x >= w || y >= h) return -0.5f;
    const uint8_t *q = rgb + (size_t(y) * w + x) * 3;
    float g = -0.5f + float(q[0]) * (0.299f / 255.f);
    g = g + float(q[1]) * (0.587f / 255.f);
    return g + float(q[2]) * (0.114f / 255.f);
}

// One thread per output pixel, a workgroup per 256 columns of one output row: the row's source
// rows, their polygon spans and the vertical weight are the same for the whole workgroup.
__global__ __launch_bounds__(256) void line_crop_kernel(const CropLine *lines, const int *row_off, const int *spans) {
#pragma clang fp contract(off)
    const CropLine L = lines[blockIdx.z];
    const int oy = blockIdx.y, ox = blockIdx.x * 256 + threadIdx.x;
    if (ox >= L.wb) return;
    float v = -0.5f;
    if (ox < L.out_w) {
        const float sy = float(L.bh) / float(LINE_H), sx = float(L.bw) / float(L.out_w);
        const float iy = fminf(fmaxf(sy * (float(oy) + 0.5f) - 0.5f, 0.f), float(L.bh) - 1.f);
        const int y1 = int(iy), y2 = min(y1 + 1, L.bh - 1);
        const float fy = iy - float(y1);
        // Crop pixel (cx, cy): the page's grey inside the row's spans, black elsewhere.
        auto px = [&](int cx, int cy) -> float {
            const int s0 = row_off[L.row_base + cy], s1 = row_off[L.row_base + cy + 1];
            for (int s = s0; s < s1; s += 2)
                if (cx >= spans[s] && cx < spans[s + 1]) return grey_px(L.rgb, L.pw, L.ph, L.left + cx, L.top + cy);
            return -0.5f;
        };
        const float ix = fminf(fmaxf(sx * (float(ox) + 0.5f) - 0.5f, 0.f), float(L.bw) - 1.f);
        const int x1 = int(ix), x2 = min(x1 + 1, L.bw - 1);
        const float fx = ix - float(x1);
        const float top = mixf(px(x1, y1), px(x2, y1), fx);
        const float bot = mixf(px(x1, y2), px(x2, y2), fx);
        v = mixf(top, bot, fy);
    }
    L.dst[size_t(oy) * L.wb + ox] = v;
}

// PP-OCR line images: the crop resized to 48 rows x out_w columns bilinearly (half-pixel,
// clamped) and rounded to bytes (the reference resizes to an 8-bit image), then per channel
// (v / 255 - 0.5) / 0.5 in RGB order, zero past out_w. Page pixels outside the page read as 0.
__global__ void pp_line_crop_kernel(const PpCropLine *lines) {
#pragma clang fp contract(off)
    const PpCropLine L = lines[blockIdx.y];
    const int total = PP_LINE_H * L.wb;
    const float sy = float(L.ch) / float(PP_LINE_H), sx = float(L.cw) / float(L.out_w);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int ox = i % L.wb, oy = i / L.wb;
        float v[3] = {0.f, 0.f, 0.f};
        if (ox < L.out_w) {
            const float iy = fminf(fmaxf(sy * (float(oy) + 0.5f) - 0.5f, 0.f), float(L.ch) - 1.f);
            const float ix = fminf(fmaxf(sx * (float(ox) + 0.5f) - 0.5f, 0.f), float(L.cw) - 1.f);
            const int y1 = int(iy), x1 = int(ix);
            const int y2 = min(y1 + 1, L.ch - 1), x2 = min(x1 + 1, L.cw - 1);
            const float fy = iy - float(y1), fx = ix - float(x1);
            auto px = [&](int cx, int cy, int c) -> float {
                const int x = L.left + cx, y = L.top + cy;
                if (x < 0 || y < 0 || x >= L.pw || y >= L.ph) return 0.f;
                return float(L.rgb[(size_t(y) * L.pw + x) * 3 + c]);
            };
            for (int c = 0; c < 3; c++) {
                const float top = mixf(px(x1, y1, c), px(x2, y1, c), fx);
                const float bot = mixf(px(x1, y2, c), px(x2, y2, c), fx);
                const float q = floorf(mixf(top, bot, fy) + 0.5f);
                v[c] = (q / 255.f - 0.5f) / 0.5f;
            }
        }
        for (int c = 0; c < 3; c++) L.dst[(size_t(c) * PP_LINE_H + oy) * L.wb + ox] = v[c];
    }
}

}  // namespace

void pp_line_crop(const PpCropLine *d_lines, int nlines, int max_wb, hipStream_t s) {
    if (nlines <= 0) return;
    if (nlines > 65535) fail("pp_line_crop: more than 65535 lines");
    const int per_line = (PP_LINE_H * max_wb + 255) / 256;
    dim3 grid(unsigned(per_line < 64 ? per_line : 64), unsigned(nlines));
    ProbeScope probe("line_crop", s, 0, 12.0 * double(nlines) * PP_LINE_H * max_wb);
    hipLaunchKernelGGL(pp_line_crop_kernel, grid, dim3(256), 0, s, d_lines);
    OCR_HIP(hipGetLastError());
}

void line_crop(const CropLine *d_lines, int nlines, const int *d_row_off, const int *d_spans, int max_wb,
               hipStream_t s) {
    if (nlines <= 0) return;
    if (nlines > 65535) fail("line_crop: more than 65535 lines");
    dim3 grid(unsigned((max_wb + 255) / 256), LINE_H, unsigned(nlines));
    ProbeScope probe("line_crop", s, 0, 4.0 * double(nlines) * LINE_H * max_wb);
    hipLaunchKernelGGL(line_crop_kernel, grid, dim3(256), 0, s, d_lines, d_row_off, d_spans);
    OCR_HIP(hipGetLastError());
}

}  // namespace ocr
