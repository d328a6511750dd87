/*
 * ORACLE - test infrastructure only. A plain-C, float32 CPU restatement of the reference's
 * GPU path (huppiflupp/wgpu-ocr, src/gpu.rs): the oracle the tests compare the HIP kernels with and, timed,
 * as the CPU baseline. Nothing in the product links or calls this file.
 *
 * Layout is ONNX's: NCHW float32. Each function cites the reference code it restates.
 * Pinning (the check in tests/test_oracle.py that fixes each function):
 *   orc_conv2d            torch conv2d golden vectors (pads, strides, groups, cin = 1, wide)
 *   orc_conv_transpose2d  torch conv_transpose2d golden vectors (2x2, 2x3, 3x3 stride 1)
 *   orc_pool2d            torch max_pool2d / avg_pool2d golden vectors
 *   orc_gru               torch GRU golden vectors (gates reordered), truncated-run lengths,
 *                         and a planted gate swap that must fail
 *   orc_grey_resize       torch bilinear (half-pixel) golden of the padded grey page
 *   orc_mask_up_prob      torch bilinear golden of the valid region; valid-region closed form
 *   orc_pack_bits         bit layout closed form
 *   orc_line_crop         torch bilinear golden of span-masked grey crops
 *   orc_activate          sigmoid closed form via the conv golden; ReLU by the conv goldens
 *   orc_det_prep          torch bilinear (half-pixel) golden of the BGR-normalised page
 *   orc_pp_line_input     torch bilinear golden of a page box, rounded to bytes and normalised
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* gpu.rs:20-34: 0 none, 1 ReLU, 2 sigmoid, 3 GELU (A&S 7.1.26 erf), 4 SiLU. */
static float erf_as(float v) {
    float s = v < 0.f ? -1.f : (v > 0.f ? 1.f : 0.f);
    float a = fabsf(v);
    float t = 1.f / (1.f + 0.3275911f * a);
    float poly = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) * t;
    return s * (1.f - poly * expf(-a * a));
}

float orc_activate(float v, int act) {
    switch (act) {
    case 1: return v > 0.f ? v : 0.f;
    case 2: return 1.f / (1.f + expf(-v));
    case 3: return 0.5f * v * (1.f + erf_as(v * 0.70710678118654752f));
    case 4: return v / (1.f + expf(-v));
    default: return v;
    }
}

/* Conv (ONNX semantics; gpu.rs:37-69 and 1255-1265 for the epilogue y = act(acc + b[c]), then
 * + res when given). Grouped: cin_g = cin / group input channels per group. pads are
 * top, left, bottom, right. Output [n][cout][oh][ow]. */
void orc_conv2d(const float *x, int n, int cin, int h, int w, const float *wt, int cout, int kh, int kw,
                const float *b, int pt, int pl, int pb, int pr, int sh, int sw, int group, int act,
                const float *res, float *y) {
    int oh = (h + pt + pb - kh) / sh + 1, ow = (w + pl + pr - kw) / sw + 1;
    int cin_g = cin / group, cout_g = cout / group;
#pragma omp parallel for collapse(2) schedule(static)
    for (int nb = 0; nb < n; nb++) {
        for (int co = 0; co < cout; co++) {
            int g = co / cout_g;
            float *yo = y + ((size_t)nb * cout + co) * oh * ow;
            for (int i = 0; i < oh * ow; i++) yo[i] = 0.f;
            for (int cg = 0; cg < cin_g; cg++) {
                int ci = g * cin_g + cg;
                const float *xi = x + ((size_t)nb * cin + ci) * h * w;
                for (int ky = 0; ky < kh; ky++) {
                    for (int kx = 0; kx < kw; kx++) {
                        float wv = wt[(((size_t)co * cin_g + cg) * kh + ky) * kw + kx];
                        for (int oy = 0; oy < oh; oy++) {
                            int iy = oy * sh - pt + ky;
                            if (iy < 0 || iy >= h) continue;
                            float *yr = yo + (size_t)oy * ow;
                            const float *xr = xi + (size_t)iy * w;
                            /* ox range with 0 <= ox * sw - pl + kx < w */
                            int lo = pl - kx > 0 ? (pl - kx + sw - 1) / sw : 0;
                            int hi = (w - 1 + pl - kx) >= 0 ? (w - 1 + pl - kx) / sw + 1 : 0;
                            if (hi > ow) hi = ow;
                            if (sw == 1) {
                                const float *xs = xr - pl + kx;
                                for (int ox = lo; ox < hi; ox++) yr[ox] += wv * xs[ox];
                            } else {
                                for (int ox = lo; ox < hi; ox++) yr[ox] += wv * xr[ox * sw - pl + kx];
                            }
                        }
                    }
                }
            }
            float bv = b ? b[co] : 0.f;
            const float *ro = res ? res + ((size_t)nb * cout + co) * oh * ow : NULL;
            for (int i = 0; i < oh * ow; i++) {
                float r = orc_activate(yo[i] + bv, act);
                yo[i] = ro ? r + ro[i] : r;
            }
        }
    }
}

/* ConvTranspose, group 1, no pads or output padding (gpu.rs:424-460, 1184-1191, 1283-1290):
 * oh = (h - 1) * s + kh. Weights [cin][cout][kh][kw]. y = act(sum + b). */
void orc_conv_transpose2d(const float *x, int n, int cin, int h, int w, const float *wt, int cout, int kh,
                          int kw, const float *b, int sh, int sw, int act, float *y) {
    int oh = (h - 1) * sh + kh, ow = (w - 1) * sw + kw;
#pragma omp parallel for collapse(2) schedule(static)
    for (int nb = 0; nb < n; nb++) {
        for (int co = 0; co < cout; co++) {
            float *yo = y + ((size_t)nb * cout + co) * oh * ow;
            for (int i = 0; i < oh * ow; i++) yo[i] = 0.f;
            for (int ci = 0; ci < cin; ci++) {
                const float *xi = x + ((size_t)nb * cin + ci) * h * w;
                for (int ky = 0; ky < kh; ky++)
                    for (int kx = 0; kx < kw; kx++) {
                        float wv = wt[(((size_t)ci * cout + co) * kh + ky) * kw + kx];
                        for (int iy = 0; iy < h; iy++)
                            for (int ix = 0; ix < w; ix++)
                                yo[(size_t)(iy * sh + ky) * ow + ix * sw + kx] += wv * xi[(size_t)iy * w + ix];
                    }
            }
            float bv = b ? b[co] : 0.f;
            for (int i = 0; i < oh * ow; i++) yo[i] = orc_activate(yo[i] + bv, act);
        }
    }
}

/* MaxPool / AveragePool without padding, floor output size (gpu.rs:462-482, 1291-1297;
 * nd.rs:246-275 for avg). x is [nc][h][w]. */
void orc_pool2d(const float *x, int nc, int h, int w, int kh, int kw, int sh, int sw, int avg, float *y) {
    int oh = (h - kh) / sh + 1, ow = (w - kw) / sw + 1;
#pragma omp parallel for schedule(static)
    for (int c = 0; c < nc; c++)
        for (int oy = 0; oy < oh; oy++)
            for (int ox = 0; ox < ow; ox++) {
                float m = -3.4e38f, s = 0.f;
                for (int ky = 0; ky < kh; ky++)
                    for (int kx = 0; kx < kw; kx++) {
                        float v = x[((size_t)c * h + oy * sh + ky) * w + ox * sw + kx];
                        m = v > m ? v : m;
                        s += v;
                    }
                y[((size_t)c * oh + oy) * ow + ox] = avg ? s / (float)(kh * kw) : m;
            }
}

static float sigm(float v) { return 1.f / (1.f + expf(-v)); }

/* ONNX GRU with linear_before_reset = 1, gate order [z, r, h] (gpu.rs:680-819):
 *   z = s(Wz x + Wbz + Rz h + Rbz), r = s(Wr x + Wbr + Rr h + Rbr),
 *   c = tanh(Wh x + Wbh + r * (Rh h + Rbh)), h' = (1 - z) c + z h, h0 = 0.
 * X [T][N][I], W [D][3H][I], R [D][3H][H], B [D][6H] = [Wb | Rb], Y [T][D][N][H].
 * Direction 1 runs t = len - 1 - s (gpu.rs:692, 768). lens NULL means T for every line; steps
 * at or past a line's length are written as 0 (ONNX). */
void orc_gru(const float *X, int T, int N, int I, const float *W, const float *R, const float *B, int H, int D,
             const int *lens, float *Y) {
    memset(Y, 0, sizeof(float) * (size_t)T * D * N * H);
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int d = 0; d < D; d++) {
        for (int nb = 0; nb < N; nb++) {
            const float *Wd = W + (size_t)d * 3 * H * I, *Rd = R + (size_t)d * 3 * H * H, *Bd = B + (size_t)d * 6 * H;
            float *h = calloc((size_t)H, sizeof(float)), *hn = calloc((size_t)H, sizeof(float));
            int len = lens ? lens[nb] : T;
            for (int s = 0; s < len; s++) {
                int t = d == 0 ? s : len - 1 - s;
                const float *x = X + ((size_t)t * N + nb) * I;
                for (int j = 0; j < H; j++) {
                    float g[3], rh[3];
                    for (int q = 0; q < 3; q++) {
                        const float *wr = Wd + (size_t)(q * H + j) * I, *rr = Rd + (size_t)(q * H + j) * H;
                        float a = 0.f, c = 0.f;
                        for (int i = 0; i < I; i++) a += wr[i] * x[i];
                        for (int k = 0; k < H; k++) c += rr[k] * h[k];
                        g[q] = a + Bd[q * H + j];
                        rh[q] = c + Bd[3 * H + q * H + j];
                    }
                    float z = sigm(g[0] + rh[0]), r = sigm(g[1] + rh[1]);
                    float c = tanhf(g[2] + r * rh[2]);
                    hn[j] = (1.f - z) * c + z * h[j];
                }
                memcpy(h, hn, sizeof(float) * (size_t)H);
                memcpy(Y + (((size_t)t * D + d) * N + nb) * H, h, sizeof(float) * (size_t)H);
            }
            free(h);
            free(hn);
        }
    }
}

/* WGSL mix(a, b, t) = a * (1 - t) + b * t. */
static float mixf(float a, float b, float t) { return a * (1.f - t) + b * t; }

/* gpu.rs:530-561: ocrs grey of the RGB page, black (-0.5) outside the w x h page inside the
 * padded pw x ph canvas, resized bilinearly (half-pixel, clamped, x then y) to ow x oh. */
static float grey_px(const uint8_t *rgb, int w, int h, int x, int yy) {
    if (x >= w || yy >= h) return -0.5f;
    const uint8_t *p = rgb + ((size_t)yy * w + x) * 3;
    return -0.5f + (float)p[0] * (0.299f / 255.f) + (float)p[1] * (0.587f / 255.f) + (float)p[2] * (0.114f / 255.f);
}

void orc_grey_resize(const uint8_t *rgb, int w, int h, int pw, int ph, int ow, int oh, float sx, float sy, float *y) {
#pragma omp parallel for schedule(static)
    for (int oy = 0; oy < oh; oy++)
        for (int ox = 0; ox < ow; ox++) {
            float iy = fminf(fmaxf(sy * ((float)oy + 0.5f) - 0.5f, 0.f), (float)ph - 1.f);
            float ix = fminf(fmaxf(sx * ((float)ox + 0.5f) - 0.5f, 0.f), (float)pw - 1.f);
            int y1 = (int)iy, x1 = (int)ix;
            int y2 = y1 + 1 < ph - 1 ? y1 + 1 : ph - 1, x2 = x1 + 1 < pw - 1 ? x1 + 1 : pw - 1;
            float wy = iy - (float)y1, wx = ix - (float)x1;
            float top = mixf(grey_px(rgb, w, h, x1, y1), grey_px(rgb, w, h, x2, y1), wx);
            float bot = mixf(grey_px(rgb, w, h, x1, y2), grey_px(rgb, w, h, x2, y2), wx);
            y[(size_t)oy * ow + ox] = mixf(top, bot, wy);
        }
}

/* gpu.rs:563-593: the first mh x mw part of the model output m (row stride `stride`) resized
 * to the page (w x h) bilinearly, before the threshold. */
void orc_mask_up_prob(const float *m, int stride, int mw, int mh, int w, int h, float sx, float sy, float *prob) {
#pragma omp parallel for schedule(static)
    for (int oy = 0; oy < h; oy++) {
        float iy = fminf(fmaxf(sy * ((float)oy + 0.5f) - 0.5f, 0.f), (float)mh - 1.f);
        int y1 = (int)iy, y2 = y1 + 1 < mh - 1 ? y1 + 1 : mh - 1;
        float fy = iy - (float)y1;
        for (int ox = 0; ox < w; ox++) {
            float ix = fminf(fmaxf(sx * ((float)ox + 0.5f) - 0.5f, 0.f), (float)mw - 1.f);
            int x1 = (int)ix, x2 = x1 + 1 < mw - 1 ? x1 + 1 : mw - 1;
            float fx = ix - (float)x1;
            float top = mixf(m[(size_t)y1 * stride + x1], m[(size_t)y1 * stride + x2], fx);
            float bot = mixf(m[(size_t)y2 * stride + x1], m[(size_t)y2 * stride + x2], fx);
            prob[(size_t)oy * w + ox] = mixf(top, bot, fy);
        }
    }
}

/* gpu.rs:589-591: bit (x % 32) of word y * ceil(w / 32) + x / 32 is set when prob > thr. */
void orc_pack_bits(const float *prob, int w, int h, float thr, uint32_t *bits) {
    int words = (w + 31) / 32;
    memset(bits, 0, sizeof(uint32_t) * (size_t)words * h);
    for (int y = 0; y < h; y++)
        for (int x = 0; x < w; x++)
            if (prob[(size_t)y * w + x] > thr) bits[(size_t)y * words + x / 32] |= 1u << (x % 32);
}

/* Line image of the page pipeline (the role of ocrs' prepare_recognition_input, called at
 * src/bin/ocr-bench.rs:378, and the batch assembly of ocr-bench.rs:388-404): crop pixel
 * (cx, cy) is the ocrs grey value of page pixel (left + cx, top + cy) when cx lies in one of the
 * row's spans [x0, x1) and the pixel is on the page, else black (-0.5); the crop (bh x bw) is
 * resized bilinearly (half-pixel, clamped) to 64 x out_w and written into dst [64][wb], padded
 * with black. */
static float crop_px(const uint8_t *rgb, int pw, int ph, int left, int top, const int *row_off, const int *spans,
                     int cx, int cy) {
    for (int s = row_off[cy]; s < row_off[cy + 1]; s += 2)
        if (cx >= spans[s] && cx < spans[s + 1]) {
            int x = left + cx, y = top + cy;
            if (x < 0 || y < 0 || x >= pw || y >= ph) return -0.5f;
            return grey_px(rgb, pw, ph, x, y);
        }
    return -0.5f;
}

void orc_line_crop(const uint8_t *rgb, int pw, int ph, int left, int top, int bw, int bh, int out_w,
                   const int *row_off, const int *spans, int wb, float *dst) {
    const int H = 64;
    float sy = (float)bh / (float)H, sx = (float)bw / (float)out_w;
    for (int oy = 0; oy < H; oy++)
        for (int ox = 0; ox < wb; ox++) {
            float v = -0.5f;
            if (ox < out_w) {
                float iy = fminf(fmaxf(sy * ((float)oy + 0.5f) - 0.5f, 0.f), (float)bh - 1.f);
                float ix = fminf(fmaxf(sx * ((float)ox + 0.5f) - 0.5f, 0.f), (float)bw - 1.f);
                int y1 = (int)iy, x1 = (int)ix;
                int y2 = y1 + 1 < bh - 1 ? y1 + 1 : bh - 1, x2 = x1 + 1 < bw - 1 ? x1 + 1 : bw - 1;
                float fy = iy - (float)y1, fx = ix - (float)x1;
                float t0 = mixf(crop_px(rgb, pw, ph, left, top, row_off, spans, x1, y1),
                                crop_px(rgb, pw, ph, left, top, row_off, spans, x2, y1), fx);
                float b0 = mixf(crop_px(rgb, pw, ph, left, top, row_off, spans, x1, y2),
                                crop_px(rgb, pw, ph, left, top, row_off, spans, x2, y2), fx);
                v = mixf(t0, b0, fy);
            }
            dst[(size_t)oy * wb + ox] = v;
        }
}

/* PP-OCR detection input (src/nd.rs:172-204, NdGraph::det_input nd.rs:1353-1369): the page's RGB
 * bytes resized bilinearly (half-pixel, clamped, x then y with the reference's mix) to ow x oh,
 * channels in BGR order, each (v / 255 - mean) / dev with ImageNet's mean and deviation.
 * Output [3][oh][ow]. */
void orc_det_prep(const uint8_t *rgb, int w, int h, int ow, int oh, float *y) {
    const float mean[3] = {0.485f, 0.456f, 0.406f}, dev[3] = {0.229f, 0.224f, 0.225f};
    const float sx = (float)w / (float)ow, sy = (float)h / (float)oh;
    for (int oy = 0; oy < oh; oy++)
        for (int ox = 0; ox < ow; ox++) {
            float ix = fminf(fmaxf(sx * ((float)ox + 0.5f) - 0.5f, 0.f), (float)w - 1.f);
            float iy = fminf(fmaxf(sy * ((float)oy + 0.5f) - 0.5f, 0.f), (float)h - 1.f);
            int x1 = (int)ix, y1 = (int)iy;
            int x2 = x1 + 1 < w - 1 ? x1 + 1 : w - 1, y2 = y1 + 1 < h - 1 ? y1 + 1 : h - 1;
            float fx = ix - (float)x1, fy = iy - (float)y1;
            for (int c = 0; c < 3; c++) {
                int k = 2 - c;
                float a = mixf((float)rgb[((size_t)y1 * w + x1) * 3 + k], (float)rgb[((size_t)y1 * w + x2) * 3 + k], fx);
                float b = mixf((float)rgb[((size_t)y2 * w + x1) * 3 + k], (float)rgb[((size_t)y2 * w + x2) * 3 + k], fx);
                y[((size_t)c * oh + oy) * ow + ox] = (mixf(a, b, fy) / 255.f - mean[c]) / dev[c];
            }
        }
}

/* PP-OCR line image (ppocr::line_input, src/ppocr.rs:42-62, batched as ppocr::batch,
 * ppocr.rs:64-78): the page box [left, left + cw) x [top, top + ch) resized to 48 rows and out_w
 * columns bilinearly (half-pixel, clamped; pixels off the page read 0), rounded to bytes (half
 * away from zero) as an 8-bit resize gives them, then (v / 255 - 0.5) / 0.5 per RGB channel;
 * dst [3][48][wb], zero past out_w. The reference resizes with the image crate's Triangle filter,
 * which this does not restate (parity with it is unpinned). */
static float pp_px(const uint8_t *rgb, int pw, int ph, int x, int y, int c) {
    if (x < 0 || y < 0 || x >= pw || y >= ph) return 0.f;
    return (float)rgb[((size_t)y * pw + x) * 3 + c];
}

void orc_pp_line_input(const uint8_t *rgb, int pw, int ph, int left, int top, int cw, int ch, int out_w, int wb,
                       float *dst) {
    const int H = 48;
    float sy = (float)ch / (float)H, sx = (float)cw / (float)out_w;
    for (int oy = 0; oy < H; oy++)
        for (int ox = 0; ox < wb; ox++) {
            for (int c = 0; c < 3; c++) dst[((size_t)c * H + oy) * wb + ox] = 0.f;
            if (ox >= out_w) continue;
            float iy = fminf(fmaxf(sy * ((float)oy + 0.5f) - 0.5f, 0.f), (float)ch - 1.f);
            float ix = fminf(fmaxf(sx * ((float)ox + 0.5f) - 0.5f, 0.f), (float)cw - 1.f);
            int y1 = (int)iy, x1 = (int)ix;
            int y2 = y1 + 1 < ch - 1 ? y1 + 1 : ch - 1, x2 = x1 + 1 < cw - 1 ? x1 + 1 : cw - 1;
            float fy = iy - (float)y1, fx = ix - (float)x1;
            for (int c = 0; c < 3; c++) {
                float t0 = mixf(pp_px(rgb, pw, ph, left + x1, top + y1, c), pp_px(rgb, pw, ph, left + x2, top + y1, c), fx);
                float b0 = mixf(pp_px(rgb, pw, ph, left + x1, top + y2, c), pp_px(rgb, pw, ph, left + x2, top + y2, c), fx);
                float q = floorf(mixf(t0, b0, fy) + 0.5f);
                dst[((size_t)c * H + oy) * wb + ox] = (q / 255.f - 0.5f) / 0.5f;
            }
        }
}
