// Line images for the recogniser, cut on the GPU straight from the page's RGB bytes in HBM: the
// role of ocrs' prepare_recognition_input (called at src/bin/ocr-bench.rs:378) and of the batch
// assembly after it (ocr-bench.rs:388-404). For each line: the pixels inside its polygon (row
// spans computed on the host) take the ocrs grey value of the page (the same formula as the
// detector front end, src/gpu.rs:542), everything else is black (-0.5); that crop is resized to
// 64 rows and out_w columns bilinearly with half-pixel centres, clamped (rten's resize_image),
// and written into the line's slot of its batch, padded with black to the batch width.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>

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

// Four 32-bit words read from a 4-byte boundary (the 16 bytes around a run of 4 RGB pixels).
typedef unsigned u32x4a __attribute__((ext_vector_type(4), aligned(4)));

constexpr int CROP_WIN = 6144;   // grey values of a block's source window in LDS
constexpr int CROP_SPANS = 512;  // polygon span bounds of the window's rows in LDS
constexpr int CROP_ROWS = 256;   // window rows

// Source coordinate of output coordinate o (half-pixel centres, clamped): the lower tap, the
// upper tap and the weight of the upper one.
struct Tap {
    int a, b;
    float f;
};
__device__ inline Tap tap(float scale, int o, int n) {
#pragma clang fp contract(off)
    const float i = fminf(fmaxf(scale * (float(o) + 0.5f) - 0.5f, 0.f), float(n) - 1.f);
    const int a = int(i);
    return {a, min(a + 1, n - 1), i - float(a)};
}

// A workgroup per output tile (tr rows x tc columns) of one line. The tile's source window (the
// crop rows and columns its taps touch) is first made grey in LDS, each source pixel once:
// inside the row's polygon spans the page's grey, else black; then every output pixel reads its
// four taps from LDS. A window too large for LDS (only possible for a tile shape the host did not
// size) is read straight from the page instead, with the same arithmetic.
__global__ __launch_bounds__(256) void line_crop_kernel(const CropLine *lines, const int *map, const int *row_off,
                                                        const int *spans) {
#pragma clang fp contract(off)
    __shared__ float s_grey[CROP_WIN];
    __shared__ int s_span[CROP_SPANS];
    __shared__ int s_roff[CROP_ROWS + 1];
    const CropLine L = lines[map[blockIdx.x]];
    const int t = int(blockIdx.x) - L.blk0;
    const int band = t / L.ntx, chunk = t - band * L.ntx;
    const int oy0 = band * L.tr, ox0 = chunk * L.tc;
    const int nr = min(L.tr, LINE_H - oy0), nc = min(L.tc, L.wb - ox0);
    const int ncw = min(nc, L.out_w - ox0);  // columns of the tile inside the resized crop
    const float sy = float(L.bh) / float(LINE_H), sx = float(L.bw) / float(L.out_w);
    const int tid = threadIdx.x;
    // The window: crop rows wy0 .. wy1, columns wx0 .. wx1.
    int wy0 = 0, wx0 = 0, wr = 0, wc = 0;
    if (ncw > 0) {
        wy0 = tap(sy, oy0, L.bh).a;
        wx0 = tap(sx, ox0, L.bw).a;
        wr = tap(sy, oy0 + nr - 1, L.bh).b - wy0 + 1;
        wc = tap(sx, ox0 + ncw - 1, L.bw).b - wx0 + 1;
    }
    const int sp0 = ncw > 0 ? row_off[L.row_base + wy0] : 0;
    const int nsp = ncw > 0 ? row_off[L.row_base + wy0 + wr] - sp0 : 0;
    const bool staged = ncw > 0 && wr * wc <= CROP_WIN && wr <= CROP_ROWS && nsp <= CROP_SPANS;
    if (staged) {
        for (int i = tid; i <= wr; i += 256) s_roff[i] = row_off[L.row_base + wy0 + i] - sp0;
        for (int i = tid; i < nsp; i += 256) s_span[i] = spans[sp0 + i];
        __syncthreads();
        // Grey of the window in items of four neighbouring pixels of one row, IPT items a thread
        // with all their loads issued before any is used. An item whose 12 bytes lie inside the
        // page row and inside the buffer is one 16-byte load from the 4-byte boundary at or below
        // its first byte, realigned with alignbyte; any other item reads its pixels one by one.
        constexpr int IPT = 6;
        const int nq = (wc + 3) >> 2, n = wr * nq;
        const uintptr_t buf0 = reinterpret_cast<uintptr_t>(L.rgb);
        const uintptr_t buf1 = buf0 + size_t(L.pw) * L.ph * 3;
        for (int j0 = 0; j0 < n; j0 += IPT * 256) {
            u32x4a raw[IPT];
            int off[IPT];
            bool fast[IPT];
#pragma unroll
            for (int k = 0; k < IPT; k++) {
                const int j = j0 + k * 256 + tid;
                const int r = j / nq, c = 4 * (j - r * nq);
                const int x0 = L.left + wx0 + c, y = L.top + wy0 + r;
                const uintptr_t a = buf0 + (size_t(y) * L.pw + x0) * 3, al = a & ~uintptr_t(3);
                fast[k] = j < n && y >= 0 && y < L.ph && x0 >= 0 && x0 + 4 <= L.pw && al >= buf0 && al + 16 <= buf1;
                off[k] = int(a & 3);
                raw[k] = fast[k] ? *reinterpret_cast<const u32x4a *>(al) : u32x4a{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int k = 0; k < IPT; k++) {
                const int j = j0 + k * 256 + tid;
                if (j >= n) break;
                const int r = j / nq, c = 4 * (j - r * nq);
                float g[4];
                if (fast[k]) {
                    const unsigned s = unsigned(off[k]);
                    const unsigned b[3] = {__builtin_amdgcn_alignbyte(raw[k].y, raw[k].x, s),
                                           __builtin_amdgcn_alignbyte(raw[k].z, raw[k].y, s),
                                           __builtin_amdgcn_alignbyte(raw[k].w, raw[k].z, s)};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int m0 = 3 * e, m1 = m0 + 1, m2 = m0 + 2;
                        const float cr = float((b[m0 >> 2] >> (8 * (m0 & 3))) & 255u);
                        const float cg = float((b[m1 >> 2] >> (8 * (m1 & 3))) & 255u);
                        const float cb = float((b[m2 >> 2] >> (8 * (m2 & 3))) & 255u);
                        float v = -0.5f + cr * (0.299f / 255.f);  // as grey_px, term by term
                        v = v + cg * (0.587f / 255.f);
                        g[e] = v + cb * (0.114f / 255.f);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        g[e] = grey_px(L.rgb, L.pw, L.ph, L.left + wx0 + c + e, L.top + wy0 + r);
                }
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (c + e >= wc) break;
                    const int cx = wx0 + c + e;
                    bool in = false;
                    for (int q = s_roff[r]; q < s_roff[r + 1]; q += 2) in = in || (cx >= s_span[q] && cx < s_span[q + 1]);
                    s_grey[r * wc + c + e] = in ? g[e] : -0.5f;
                }
            }
        }
        __syncthreads();
    }
    // Crop pixel (cx, cy) read straight from the page: the page's grey inside the row's spans,
    // black elsewhere.
    auto px = [&](int cx, int cy) -> float {
        const int s0 = row_off[L.row_base + cy], s1 = row_off[L.row_base + cy + 1];
        for (int q = s0; q < s1; q += 2)
            if (cx >= spans[q] && cx < spans[q + 1]) return grey_px(L.rgb, L.pw, L.ph, L.left + cx, L.top + cy);
        return -0.5f;
    };
    for (int i = tid; i < nr * nc; i += 256) {
        const int r = i / nc, c = i - r * nc;
        const int oy = oy0 + r, ox = ox0 + c;
        float v = -0.5f;
        if (ox < L.out_w) {
            const Tap ty = tap(sy, oy, L.bh), tx = tap(sx, ox, L.bw);
            float p11, p21, p12, p22;
            if (staged) {
                const int r1 = (ty.a - wy0) * wc, r2 = (ty.b - wy0) * wc, c1 = tx.a - wx0, c2 = tx.b - wx0;
                p11 = s_grey[r1 + c1];
                p21 = s_grey[r1 + c2];
                p12 = s_grey[r2 + c1];
                p22 = s_grey[r2 + c2];
            } else {
                p11 = px(tx.a, ty.a);
                p21 = px(tx.b, ty.a);
                p12 = px(tx.a, ty.b);
                p22 = px(tx.b, ty.b);
            }
            const float top = mixf(p11, p21, tx.f);
            const float bot = mixf(p12, p22, tx.f);
            v = mixf(top, bot, ty.f);
        }
        L.dst[size_t(oy) * L.wb + ox] = v;
    }
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

void line_crop(Ctx &ctx, std::vector<CropLine> &lines, const std::vector<int32_t> &row_off,
               const std::vector<int32_t> &spans, hipStream_t s) {
    if (lines.empty()) return;
    // Tile shape per line: 16 rows x 256 columns, narrowed until the source window (at most
    // (tr - 1) sy + 3 rows by (tc - 1) sx + 3 columns) fits in LDS.
    std::vector<int> map;
    double bytes = 0;
    for (size_t i = 0; i < lines.size(); i++) {
        CropLine &L = lines[i];
        if (L.wb < 1 || L.out_w < 1 || L.out_w > L.wb || L.bw < 1 || L.bh < 1) fail("line_crop: line box or width");
        const double sy = double(L.bh) / LINE_H, sx = double(L.bw) / L.out_w;
        auto win = [&](int tr, int tc) { return (std::floor((tr - 1) * sy) + 3) * (std::floor((tc - 1) * sx) + 3); };
        int tr = 16, tc = 256;
        while (win(tr, tc) > CROP_WIN && tc > 64) tc /= 2;
        while (win(tr, tc) > CROP_WIN && tr > 1) tr /= 2;
        while (win(tr, tc) > CROP_WIN && tc > 1) tc /= 2;
        L.tr = tr;
        L.tc = tc;
        L.ntx = (L.wb + tc - 1) / tc;
        L.blk0 = int(map.size());
        const long long nb = (long long)((LINE_H + tr - 1) / tr) * L.ntx;
        if (double(map.size()) + double(nb) > 2147483647.0) fail("line_crop: grid too large");
        map.insert(map.end(), size_t(nb), int(i));
        bytes += 4.0 * LINE_H * L.wb + 3.0 * double(L.bw) * L.bh;
    }
    // One block: descriptors, map, row offsets, spans (each from a 16-byte boundary).
    auto up16 = [](size_t b) { return (b + 15) & ~size_t(15); };
    const size_t o_map = up16(lines.size() * sizeof(CropLine)), o_roff = o_map + up16(map.size() * 4),
                 o_spans = o_roff + up16(row_off.size() * 4), total = o_spans + up16(std::max<size_t>(spans.size(), 1) * 4);
    std::vector<char> blk(total, 0);
    std::memcpy(blk.data(), lines.data(), lines.size() * sizeof(CropLine));
    std::memcpy(blk.data() + o_map, map.data(), map.size() * 4);
    if (!row_off.empty()) std::memcpy(blk.data() + o_roff, row_off.data(), row_off.size() * 4);
    if (!spans.empty()) std::memcpy(blk.data() + o_spans, spans.data(), spans.size() * 4);
    DBuf d(&ctx, total);
    ctx.h2d(d.get(), blk.data(), total);
    char *b = d.as<char>();
    ProbeScope probe("line_crop", s, 0, bytes);
    hipLaunchKernelGGL(line_crop_kernel, dim3(unsigned(map.size())), dim3(256), 0, s, reinterpret_cast<CropLine *>(b),
                       reinterpret_cast<int *>(b + o_map), reinterpret_cast<const int *>(b + o_roff),
                       reinterpret_cast<const int *>(b + o_spans));
    OCR_HIP(hipGetLastError());
}

}  // namespace ocr
