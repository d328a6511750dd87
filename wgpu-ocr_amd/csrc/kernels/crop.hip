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

__device__ inline float crop_px(const CropLine &L, const int *row_off, const int *spans, int cx, int cy) {
    const int s0 = row_off[L.row_base + cy], s1 = row_off[L.row_base + cy + 1];
    for (int s = s0; s < s1; s += 2)
        if (cx >= spans[s] && cx < spans[s + 1]) return grey_px(L.rgb, L.pw, L.ph, L.left + cx, L.top + cy);
    return -0.5f;
}

__global__ void line_crop_kernel(const CropLine *lines, const int *row_off, const int *spans) {
#pragma clang fp contract(off)
    const CropLine L = lines[blockIdx.y];
    const int total = LINE_H * L.wb;
    const float sy = float(L.bh) / float(LINE_H), sx = float(L.bw) / float(L.out_w);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
        const int ox = i % L.wb, oy = i / L.wb;
        float v = -0.5f;
        if (ox < L.out_w) {
            const float iy = fminf(fmaxf(sy * (float(oy) + 0.5f) - 0.5f, 0.f), float(L.bh) - 1.f);
            const float ix = fminf(fmaxf(sx * (float(ox) + 0.5f) - 0.5f, 0.f), float(L.bw) - 1.f);
            const int y1 = int(iy), x1 = int(ix);
            const int y2 = min(y1 + 1, L.bh - 1), x2 = min(x1 + 1, L.bw - 1);
            const float fy = iy - float(y1), fx = ix - float(x1);
            const float top = mixf(crop_px(L, row_off, spans, x1, y1), crop_px(L, row_off, spans, x2, y1), fx);
            const float bot = mixf(crop_px(L, row_off, spans, x1, y2), crop_px(L, row_off, spans, x2, y2), fx);
            v = mixf(top, bot, fy);
        }
        L.dst[size_t(oy) * L.wb + ox] = v;
    }
}

}  // namespace

void line_crop(const CropLine *d_lines, int nlines, const int *d_row_off, const int *d_spans, int max_wb,
               hipStream_t s) {
    if (nlines <= 0) return;
    const int per_line = (LINE_H * max_wb + 255) / 256;
    dim3 grid(unsigned(per_line < 64 ? per_line : 64), unsigned(nlines));
    ProbeScope probe("line_crop", s, 0, 4.0 * double(nlines) * LINE_H * max_wb);
    hipLaunchKernelGGL(line_crop_kernel, grid, dim3(256), 0, s, d_lines, d_row_off, d_spans);
    OCR_HIP(hipGetLastError());
}

}  // namespace ocr
