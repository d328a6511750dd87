// Memory-bound kernels of the path, NHWC float32 activations. Semantics follow the reference's
// WGSL programs in src/gpu.rs (line numbers at each kernel); the layouts are this library's own.
#include <hip/hip_runtime.h>

#include <cmath>

#include "../kernels.h"
#include "../runtime.h"

namespace ocr {

namespace {

__device__ inline float act_f(float v, int act) {
    if (act == ACT_RELU) return fmaxf(v, 0.f);
    if (act == ACT_SIGMOID) return 1.f / (1.f + expf(-v));
    if (act == ACT_GELU) return 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    if (act == ACT_SILU) return v / (1.f + expf(-v));
    return v;
}

inline unsigned blocks_for(size_t n, int per = 256) {
    size_t b = (n + per - 1) / per;
    if (b > 0x7fffffff) fail("grid too large");
    return unsigned(b ? b : 1);
}

// WGSL mix(a, b, t) = a * (1 - t) + b * t, unfused as the reference states it: contraction into
// fused multiply-adds is off in the front- and back-end kernels below.
__device__ inline float mixf(float a, float b, float t) {
#pragma clang fp contract(off)
    return a * (1.f - t) + b * t;
}

// ---- conv_generic: any group / stride, float32, one thread per output value -----------------
__global__ void conv_generic_kernel(const float *x, int n, int h, int w, int cin, int xcs, float *y, int oh, int ow,
                                    int cout, int ycs, const float *wt, const float *b, int kh, int kw, int sh,
                                    int sw, int pt, int pl, int group, int act) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    size_t total = size_t(n) * oh * ow * cout;
    if (i >= total) return;
    int co = int(i % cout);
    size_t pix = i / cout;
    int ox = int(pix % ow), oy = int((pix / ow) % oh), img = int(pix / (size_t(ow) * oh));
    int cin_g = cin / group, cout_g = cout / group, g0 = (co / cout_g) * cin_g;
    float acc = 0.f;
    for (int c = 0; c < cin_g; c++)
        for (int ky = 0; ky < kh; ky++) {
            int iy = oy * sh - pt + ky;
            if (iy < 0 || iy >= h) continue;
            for (int kx = 0; kx < kw; kx++) {
                int ix = ox * sw - pl + kx;
                if (ix < 0 || ix >= w) continue;
                acc += x[((size_t(img) * h + iy) * w + ix) * xcs + g0 + c] * wt[((size_t(co) * cin_g + c) * kh + ky) * kw + kx];
            }
        }
    y[pix * ycs + co] = act_f(acc + (b ? b[co] : 0.f), act);
}

// ---- conv_direct (gpu.rs:385-422): cin = 1, stride 1, act, MaxPool (ph, pw) fused ------------
// A workgroup owns a tile of DTY x DTX pooled outputs of one image and every output channel. The
// input window of the tile and all weights are staged in LDS; thread i takes channel i % cout
// of successive pixels, so the NHWC stores of a row of the tile are contiguous. Template
// arguments fix the kernel and pool sizes of the common cases (0: taken from the arguments).
constexpr int DTY = 8, DTX = 32, DMAXK = 7, DMAXP = 4, DMAXC = 64;
constexpr int DIN_ROWS = DTY * DMAXP + DMAXK - 1, DIN_COLS = DTX * DMAXP + DMAXK - 1;

template <int KS, int PS>
__global__ __launch_bounds__(256) void conv_direct_kernel(const float *__restrict__ x, int h, int w, int xcs,
                                                          float *__restrict__ y, int oh, int ow, int cout, int ycs,
                                                          const float *__restrict__ wt, const float *__restrict__ b,
                                                          int kh_, int kw_, int pad, int act, int ph_, int pw_,
                                                          int tiles_x) {
    const int kh = KS ? KS : kh_, kw = KS ? KS : kw_, ph = PS ? PS : ph_, pw = PS ? PS : pw_;
    __shared__ float s_in[DIN_ROWS * DIN_COLS];
    __shared__ float s_w[DMAXC * DMAXK * DMAXK];
    __shared__ float s_b[DMAXC];
    const int tid = threadIdx.x;
    const int tx = blockIdx.x % tiles_x, ty = blockIdx.x / tiles_x, img = blockIdx.y;
    const int oy0 = ty * DTY, ox0 = tx * DTX;
    const int rows = DTY * ph + kh - 1, cols = DTX * pw + kw - 1;
    const int iy0 = oy0 * ph - pad, ix0 = ox0 * pw - pad;
    const float *xi = x + size_t(img) * h * w * xcs;
    for (int i = tid; i < rows * cols; i += 256) {
        const int r = i / cols, c = i - r * cols;
        const int iy = iy0 + r, ix = ix0 + c;
        s_in[i] = (iy >= 0 && iy < h && ix >= 0 && ix < w) ? xi[(size_t(iy) * w + ix) * xcs] : 0.f;
    }
    for (int i = tid; i < cout * kh * kw; i += 256) s_w[i] = wt[i];
    for (int i = tid; i < cout; i += 256) s_b[i] = b[i];
    __syncthreads();
    for (int idx = tid; idx < DTY * DTX * cout; idx += 256) {
        const int co = idx % cout, p = idx / cout;
        const int py = p / DTX, px = p - py * DTX;
        const int oy = oy0 + py, ox = ox0 + px;
        if (oy >= oh || ox >= ow) continue;
        const float *wc = s_w + co * kh * kw;
        const float bias = s_b[co];
        float best = -INFINITY;
        for (int qy = 0; qy < ph; qy++)
            for (int qx = 0; qx < pw; qx++) {
                const float *src = s_in + (py * ph + qy) * cols + px * pw + qx;
                float acc = 0.f;
                for (int ky = 0; ky < kh; ky++)
                    for (int kx = 0; kx < kw; kx++) acc = __fmaf_rn(src[ky * cols + kx], wc[ky * kw + kx], acc);
                best = fmaxf(best, act_f(acc + bias, act));
            }
        y[((size_t(img) * oh + oy) * ow + ox) * ycs + co] = best;
    }
}

// ---- conv_transpose (gpu.rs:424-460): gather form, taps with ky = oy mod s ------------------
// Weights re-laid out as [ky][kx][cin][cout]; consecutive threads take consecutive channels.
__global__ void convt_kernel(const float *x, int n, int h, int w, int cin, int xcs, float *y, int oh, int ow,
                             int cout, int ycs, const float *wt, const float *b, int kh, int kw, int s, int act) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(n) * oh * ow * cout) return;
    int co = int(i % cout);
    size_t pix = i / cout;
    int ox = int(pix % ow), oy = int((pix / ow) % oh), img = int(pix / (size_t(ow) * oh));
    float acc = 0.f;
    for (int ky = oy % s; ky < kh && ky <= oy; ky += s) {
        int iy = (oy - ky) / s;
        if (iy >= h) continue;
        for (int kx = ox % s; kx < kw && kx <= ox; kx += s) {
            int ix = (ox - kx) / s;
            if (ix >= w) continue;
            const float *xp = x + ((size_t(img) * h + iy) * w + ix) * xcs;
            const float *wp = wt + (size_t(ky * kw + kx) * cin) * cout + co;
            for (int ci = 0; ci < cin; ci++) acc += xp[ci] * wp[size_t(ci) * cout];
        }
    }
    y[pix * ycs + co] = act_f(acc + b[co], act);
}

// ConvTranspose with kernel = stride = 2 (gpu.rs:424-460 for this case): output pixel (oy, ox)
// is input pixel (oy / 2, ox / 2) times the one tap (oy % 2, ox % 2), no overlapping taps. The
// weights [ky][kx][cin][cout] sit in LDS. A thread makes four output channels (c0 .. c0 + 3) of
// phase px in output row oy for four neighbouring input columns, so each weight read from LDS
// serves 16 FMAs; neighbouring lanes take the channel quads, then the two phases, so a store
// instruction writes whole neighbouring pixels. float32 FMAs over the input channels in order,
// the bias added last as in convt_kernel. Grid-stride, so each workgroup fills its LDS once.
constexpr int CT2_MAXW = 16384;  // weight floats in LDS (64 KB)

__global__ __launch_bounds__(256) void convt_k2s2_kernel(const float *x, int h, int w, int cin, long xcs, float *y,
                                                          long total, int oh, int ow, int cout, long ycs, int nxg,
                                                          const float *wt, const float *b, int act) {
    extern __shared__ float sw[];
    for (int i = threadIdx.x; i < 4 * cin * cout; i += 256) sw[i] = wt[i];
    __syncthreads();
    const int cq = cout >> 2;
    for (long g = long(blockIdx.x) * 256 + threadIdx.x; g < total; g += long(gridDim.x) * 256) {
        const int q = int(g % cq);
        long t = g / cq;
        const int px = int(t & 1);
        t >>= 1;
        const int xg = int(t % nxg);
        t /= nxg;
        const int oy = int(t % oh), img = int(t / oh);
        const float *xrow = x + (size_t(img) * h + (oy >> 1)) * w * xcs;
        const float *xp[4];
        bool live[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int ix = 4 * xg + k;
            live[k] = ix < w && 2 * ix + px < ow;
            xp[k] = xrow + size_t(live[k] ? ix : 0) * xcs;
        }
        const float4 *wp = reinterpret_cast<const float4 *>(sw + size_t(((oy & 1) * 2 + px) * cin) * cout) + q;
        float acc[4][4] = {};
        // The next block of 4 input channels is loaded before this block's FMAs.
        float4 nx[4];
#pragma unroll
        for (int k = 0; k < 4; k++) nx[k] = *reinterpret_cast<const float4 *>(xp[k]);
        for (int ci = 0; ci < cin; ci += 4) {
            float xs[4][4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float4 v = nx[k];
                xs[k][0] = v.x, xs[k][1] = v.y, xs[k][2] = v.z, xs[k][3] = v.w;
            }
            if (ci + 4 < cin)
#pragma unroll
                for (int k = 0; k < 4; k++) nx[k] = *reinterpret_cast<const float4 *>(xp[k] + ci + 4);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float4 wv = wp[size_t(ci + e) * cq];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    acc[k][0] = fmaf(xs[k][e], wv.x, acc[k][0]);
                    acc[k][1] = fmaf(xs[k][e], wv.y, acc[k][1]);
                    acc[k][2] = fmaf(xs[k][e], wv.z, acc[k][2]);
                    acc[k][3] = fmaf(xs[k][e], wv.w, acc[k][3]);
                }
            }
        }
        const int c0 = 4 * q;
        const float b0 = b[c0], b1 = b[c0 + 1], b2 = b[c0 + 2], b3 = b[c0 + 3];
        float *yrow = y + (size_t(img) * oh + oy) * ow * ycs + c0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (!live[k]) continue;
            float4 o;
            o.x = act_f(acc[k][0] + b0, act);
            o.y = act_f(acc[k][1] + b1, act);
            o.z = act_f(acc[k][2] + b2, act);
            o.w = act_f(acc[k][3] + b3, act);
            *reinterpret_cast<float4 *>(yrow + size_t(2 * (4 * xg + k) + px) * ycs) = o;
        }
    }
}

// ---- maxpool (gpu.rs:462-482): kernel = stride, no padding, floor ---------------------------
__global__ void maxpool_kernel(const float *x, int n, int h, int w, int c, int xcs, float *y, int oh, int ow, int ycs,
                               int kh, int kw) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(n) * oh * ow * c) return;
    int ch = int(i % c);
    size_t pix = i / c;
    int ox = int(pix % ow), oy = int((pix / ow) % oh), img = int(pix / (size_t(ow) * oh));
    float m = -3.4e38f;
    for (int ky = 0; ky < kh; ky++)
        for (int kx = 0; kx < kw; kx++)
            m = fmaxf(m, x[((size_t(img) * h + oy * kh + ky) * w + ox * kw + kx) * xcs + ch]);
    y[pix * ycs + ch] = m;
}

// ---- copy: out[n][y][x][c] = in[n][y + y0][x + x0][c] (gpu.rs:484-515, Slice and Concat) -----
__global__ void copy_kernel(const float *x, int xh, int xw, int xcs, float *y, int n, int h, int w, int c, int ycs,
                            int y0, int x0) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(n) * h * w * c) return;
    int ch = int(i % c);
    size_t pix = i / c;
    int ox = int(pix % w), oy = int((pix / w) % h), img = int(pix / (size_t(w) * h));
    y[pix * ycs + ch] = x[((size_t(img) * xh + oy + y0) * xw + ox + x0) * xcs + ch];
}

__global__ void activate_kernel(const float *x, int xcs, float *y, int ycs, size_t pixels, int c, int act) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= pixels * c) return;
    size_t pix = i / c;
    int ch = int(i % c);
    y[pix * ycs + ch] = act_f(x[pix * xcs + ch], act);
}

__global__ void fill_kernel(float *p, size_t count, float v) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) p[i] = v;
}

// ---- grey_resize (gpu.rs:530-561) -------------------------------------------------------------
__device__ inline float grey_at(const uint8_t *rgb, int w, int h, int x, int yy) {
#pragma clang fp contract(off)
    if (x >= w || yy >= h) return -0.5f;
    const uint8_t *q = rgb + (size_t(yy) * w + x) * 3;
    float g = -0.5f + float(q[0]) * (0.299f / 255.f);
    g = g + float(q[1]) * (0.587f / 255.f);
    return g + float(q[2]) * (0.114f / 255.f);
}

// Up to GPMAX pages a launch (blockIdx.y): one thread per output pixel.
constexpr int GPMAX = 16;
struct GreyParams {
    GreyPage pg[GPMAX];
    int ow, oh;
};
__global__ void grey_resize_kernel(const GreyParams p) {
#pragma clang fp contract(off)
    const GreyPage &g = p.pg[blockIdx.y];
    const int ow = p.ow, oh = p.oh;
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= ow * oh) return;
    int ox = i % ow, oy = i / ow;
    float iy = fminf(fmaxf(g.sy * (float(oy) + 0.5f) - 0.5f, 0.f), float(g.ph) - 1.f);
    float ix = fminf(fmaxf(g.sx * (float(ox) + 0.5f) - 0.5f, 0.f), float(g.pw) - 1.f);
    int y1 = int(iy), x1 = int(ix);
    int y2 = min(y1 + 1, g.ph - 1), x2 = min(x1 + 1, g.pw - 1);
    float wy = iy - float(y1), wx = ix - float(x1);
    float top = mixf(grey_at(g.rgb, g.w, g.h, x1, y1), grey_at(g.rgb, g.w, g.h, x2, y1), wx);
    float bot = mixf(grey_at(g.rgb, g.w, g.h, x1, y2), grey_at(g.rgb, g.w, g.h, x2, y2), wx);
    g.y[i] = mixf(top, bot, wy);
}

// ---- mask_up (gpu.rs:563-593): a wavefront per MJ blocks of 64 columns (2*MJ bit words, one
// 64-byte store a row) of MR rows; a lane takes column 64*j + lane of block j, and block j's
// ballot gives words 2j and 2j+1. The map rows the MR output rows read are interpolated across
// once per block and lane (two taps a map row instead of four an output row).
constexpr int MR = 8, MJ = 8;
struct MaskParams {
    MaskPage pg[GPMAX];
    int stride;
    float thr;
};
// Source coordinate of output index o (monotone in o, so a run of output rows reads a run of map
// rows).
__device__ inline float mask_src(float s, int o, int n) {
#pragma clang fp contract(off)
    return fminf(fmaxf(s * (float(o) + 0.5f) - 0.5f, 0.f), float(n) - 1.f);
}
// The bit word of one output row that lane 2j (low half) or 2j + 1 (high half) stores: block j's
// pixels thresholded after the vertical step of the bilinear interpolation.
__device__ __forceinline__ uint32_t mask_word(const float (&top)[MJ], const float (&bot)[MJ], const bool (&col)[MJ],
                                              float fy, float thr, int lane) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < MJ; j++) {
        const unsigned long long b = __ballot(col[j] && mixf(top[j], bot[j], fy) > thr);
        if (lane == 2 * j) word = uint32_t(b);
        if (lane == 2 * j + 1) word = uint32_t(b >> 32);
    }
    return word;
}
__global__ void mask_up_kernel(const MaskParams p) {
#pragma clang fp contract(off)
    const MaskPage &g = p.pg[blockIdx.y];
    const float *m = g.m;
    const int stride = p.stride, mw = g.mw, mh = g.mh, w = g.w, h = g.h, words = (g.w + 31) / 32;
    const float sx = g.sx, sy = g.sy, thr = p.thr;
    uint32_t *bits = g.bits;
    const int lane = threadIdx.x & 63;
    // The wavefront's index, uniform (read from lane 0) so that everything derived from it is too.
    // Blocks are renumbered so that each XCD takes a contiguous run (neighbouring row groups share
    // map rows, which that XCD's L2 then serves once).
    const int G = gridDim.x, q8 = G >> 3, r8 = G & 7, xb = blockIdx.x & 7;
    const int blk = xb * q8 + min(xb, r8) + (blockIdx.x >> 3);
    const long wv = long(blk) * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int chunks = (words + 2 * MJ - 1) / (2 * MJ), groups = (h + MR - 1) / MR;
    if (wv >= long(chunks) * groups) return;  // the whole wavefront
    const int rg = int(wv / chunks), wc = int(wv - long(rg) * chunks);
    int x1[MJ], x2[MJ];
    float fx[MJ];
    bool col[MJ];
#pragma unroll
    for (int j = 0; j < MJ; j++) {
        const int ox = (wc * MJ + j) * 64 + lane;
        col[j] = ox < w;
        const float ix = mask_src(sx, ox, mw);
        x1[j] = int(ix), x2[j] = min(x1[j] + 1, mw - 1);
        fx[j] = ix - float(x1[j]);
    }
    // Output row oy reads map rows y1 = int(iy) and min(y1 + 1, mh - 1), iy its source coordinate
    // (monotone in oy); ya and yl are the group's first and last y1 (uniform). When
    // yl - ya + 2 <= HR (a page larger than the map), the rows ya .. ya + HR - 1, clamped to the
    // map, are interpolated across once per block and lane, and the output rows are walked pair
    // by pair: pair q (rows ya + q and ya + q + 1, which the clamp makes the same row at the
    // map's last) takes the output rows whose y1 is ya + q in a uniform loop, so its registers
    // are fixed. Every tap address is inside the map, so the loads are unconditional and in
    // flight together; a lane past the page width only has its result dropped.
    constexpr int HR = 5;
    const int k1 = min(MR, h - rg * MR);  // output rows of the group
    const int ya = int(mask_src(sy, rg * MR, mh)), yl = int(mask_src(sy, rg * MR + k1 - 1, mh));
    const int wi = wc * 2 * MJ + lane;  // the word lane < 2*MJ stores
    if (yl - ya + 2 <= HR) {
        float hrow[HR][MJ];
#pragma unroll
        for (int q = 0; q < HR; q++) {
            const float *r = m + size_t(min(ya + q, mh - 1)) * stride;
#pragma unroll
            for (int j = 0; j < MJ; j++) hrow[q][j] = mixf(r[x1[j]], r[x2[j]], fx[j]);
        }
        int k = 0;
#pragma unroll
        for (int q = 0; q + 1 < HR; q++)
            for (; k < k1; k++) {
                const int oy = rg * MR + k;
                const float iy = mask_src(sy, oy, mh);
                const int y1 = int(iy);
                if (y1 != ya + q) break;
                const uint32_t word = mask_word(hrow[q], hrow[q + 1], col, iy - float(y1), thr, lane);
                if (lane < 2 * MJ && wi < words) bits[size_t(oy) * words + wi] = word;
            }
    } else {
        for (int k = 0; k < k1; k++) {
            const int oy = rg * MR + k;
            const float iy = mask_src(sy, oy, mh);
            const int y1 = int(iy), y2 = min(y1 + 1, mh - 1);
            const float *r1 = m + size_t(y1) * stride, *r2 = m + size_t(y2) * stride;
            float top[MJ], bot[MJ];
#pragma unroll
            for (int j = 0; j < MJ; j++) {
                top[j] = mixf(r1[x1[j]], r1[x2[j]], fx[j]);
                bot[j] = mixf(r2[x1[j]], r2[x2[j]], fx[j]);
            }
            const uint32_t word = mask_word(top, bot, col, iy - float(y1), thr, lane);
            if (lane < 2 * MJ && wi < words) bits[size_t(oy) * words + wi] = word;
        }
    }
}

// ---- 1 x 1 convolution to CO <= 4 channels (gpu.rs:37-350 for this shape): one thread a pixel,
// the input channels in float4 loads, float32 products summed in channel order.
template <int CO>
__global__ void conv1x1_narrow_kernel(const float *__restrict__ x, long pixels, int cin, int xcs, float *__restrict__ y,
                                      int ycs, const float *__restrict__ w, const float *__restrict__ b, int act) {
    const long p = long(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= pixels) return;
    const float4 *xp = reinterpret_cast<const float4 *>(x + size_t(p) * xcs);
    float acc[CO];
#pragma unroll
    for (int c = 0; c < CO; c++) acc[c] = 0.f;
    for (int k = 0; k < cin / 4; k++) {
        const float4 v = xp[k];
#pragma unroll
        for (int c = 0; c < CO; c++) {
            const float *wc = w + c * cin + 4 * k;
            acc[c] = fmaf(v.x, wc[0], acc[c]);
            acc[c] = fmaf(v.y, wc[1], acc[c]);
            acc[c] = fmaf(v.z, wc[2], acc[c]);
            acc[c] = fmaf(v.w, wc[3], acc[c]);
        }
    }
#pragma unroll
    for (int c = 0; c < CO; c++) y[size_t(p) * ycs + c] = act_f(acc[c] + (b ? b[c] : 0.f), act);
}

// ---- avgpool_t (gpu.rs:595-614): [n][kh][T][c] -> X[t][ntot][c] at line offset noff ----------
// Up to APMAXSEG inputs a launch; segment s owns the blocks from blk0 (its elements padded to
// whole blocks, so a block lies in one segment).
struct ApSeg {
    const float *x;
    int n, h, T, xcs, noff, blk0;
};
constexpr int APMAXSEG = 32;
struct ApParams {
    int nseg, kh, c, ntot;
    float *X;
    ApSeg seg[APMAXSEG];
};

__global__ __launch_bounds__(256) void avgpool_t_kernel(const ApParams p) {
    int sg = 0;
    while (sg + 1 < p.nseg && int(blockIdx.x) >= p.seg[sg + 1].blk0) sg++;
    const ApSeg &S = p.seg[sg];
    const size_t i = size_t(int(blockIdx.x) - S.blk0) * 256 + threadIdx.x;
    const int c = p.c;
    if (i >= size_t(S.n) * S.T * c) return;
    const int ch = int(i % c);
    const int t = int((i / c) % S.T), img = int(i / (size_t(c) * S.T));
    float s = 0.f;
    for (int r = 0; r < p.kh; r++) s += S.x[((size_t(img) * S.h + r) * S.T + t) * S.xcs + ch];
    p.X[(size_t(t) * p.ntot + S.noff + img) * c + ch] = s / float(p.kh);
}

// ---- argmax: 16 lanes a row (four rows a wavefront), the last index on ties -----------------
// A row of the recogniser's 97 classes is 388 bytes: 16 lanes read it in seven coalesced steps,
// all issued before the first compare, and reduce it in four exchanges. A wavefront a row left
// 48 lanes idle in its second step and ran 70 000 short wavefronts a launch, bound by their
// launch and lifetime (1.4 TB/s); 4, 8 and 32 lanes a row measured slower than 16.
constexpr int AMAX_LANES = 16, AMAX_BATCH = 8;
__global__ void argmax_kernel(const float *x, int rows, int classes, uint32_t *best, const int *map) {
    const int sub = threadIdx.x & (AMAX_LANES - 1);
    int row = int((size_t(blockIdx.x) * blockDim.x + threadIdx.x) / AMAX_LANES);
    if (row >= rows) return;  // the whole group of 16 lanes leaves together
    if (map) row = map[row];
    const float *r = x + size_t(row) * classes;
    float bv = -INFINITY;
    int bi = -1;
    for (int j0 = sub; j0 < classes; j0 += AMAX_LANES * AMAX_BATCH) {
        float v[AMAX_BATCH];
#pragma unroll
        for (int k = 0; k < AMAX_BATCH; k++) {
            const int j = j0 + k * AMAX_LANES;
            v[k] = j < classes ? r[j] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < AMAX_BATCH; k++) {
            const int j = j0 + k * AMAX_LANES;
            if (j < classes && (bi < 0 || v[k] >= bv)) { bv = v[k]; bi = j; }
        }
    }
    for (int off = AMAX_LANES / 2; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, AMAX_LANES);
        const int oi = __shfl_xor(bi, off, AMAX_LANES);
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) { bv = ov; bi = oi; }
    }
    if (sub == 0) best[row] = uint32_t(bi < 0 ? 0 : bi);
}

}  // namespace

void conv_generic(const Act &x, const Act &y, const float *w, const float *b, int kh, int kw, int sh, int sw, int pt,
                  int pl, int group, int act, hipStream_t s) {
    size_t total = y.count();
    ProbeScope probe("conv_generic", s, 2.0 * double(total) * (x.c / group) * kh * kw,
                     4.0 * double(x.count() + y.count()));
    hipLaunchKernelGGL(conv_generic_kernel, dim3(blocks_for(total)), dim3(256), 0, s, x.p, x.n, x.h, x.w, x.c, x.cs,
                       y.p, y.h, y.w, y.c, y.cs, w, b, kh, kw, sh, sw, pt, pl, group, act);
    OCR_HIP(hipGetLastError());
}

void conv_direct(const Act &x, const Act &y, const float *w, const float *b, int kh, int kw, int pad, int act, int ph,
                 int pw, hipStream_t s, const uint16_t *frag) {
    if (frag && kh == 3 && kw == 3 && pad == 1 && conv1_mfma(x, y, frag, b, act, ph, pw, s)) return;
    if (kh > DMAXK || kw > DMAXK || ph > DMAXP || pw > DMAXP || y.c > DMAXC)
        fail("conv_direct: kernel above 7 x 7, pool above 4 x 4 or more than 64 channels");
    if (x.c != 1) fail("conv_direct: one input channel");
    ProbeScope probe("conv_direct", s, 2.0 * double(y.pixels()) * ph * pw * y.c * kh * kw,
                     4.0 * double(x.pixels() + y.count()));
    const int tiles_x = (y.w + DTX - 1) / DTX, tiles_y = (y.h + DTY - 1) / DTY;
    if (size_t(tiles_x) * tiles_y > 0x7fffffff || y.n > 65535) fail("conv_direct: grid too large");
    dim3 grid(unsigned(tiles_x * tiles_y), unsigned(y.n));
    if (kh == 3 && kw == 3 && ph == 2 && pw == 2)
        hipLaunchKernelGGL((conv_direct_kernel<3, 2>), grid, dim3(256), 0, s, x.p, x.h, x.w, x.cs, y.p, y.h, y.w, y.c,
                           y.cs, w, b, kh, kw, pad, act, ph, pw, tiles_x);
    else if (kh == 3 && kw == 3 && ph == 1 && pw == 1)
        hipLaunchKernelGGL((conv_direct_kernel<3, 1>), grid, dim3(256), 0, s, x.p, x.h, x.w, x.cs, y.p, y.h, y.w, y.c,
                           y.cs, w, b, kh, kw, pad, act, ph, pw, tiles_x);
    else
        hipLaunchKernelGGL((conv_direct_kernel<0, 0>), grid, dim3(256), 0, s, x.p, x.h, x.w, x.cs, y.p, y.h, y.w, y.c,
                           y.cs, w, b, kh, kw, pad, act, ph, pw, tiles_x);
    OCR_HIP(hipGetLastError());
}

void conv_transpose(const Act &x, const Act &y, const float *w, const float *b, int kh, int kw, int stride, int act,
                    hipStream_t s) {
    ProbeScope probe("conv_transpose", s, 2.0 * double(x.pixels()) * x.c * y.c * kh * kw,
                     4.0 * double(x.count() + y.count()));
    hipLaunchKernelGGL(convt_kernel, dim3(blocks_for(y.count())), dim3(256), 0, s, x.p, x.n, x.h, x.w, x.c, x.cs, y.p,
                       y.h, y.w, y.c, y.cs, w, b, kh, kw, stride, act);
    OCR_HIP(hipGetLastError());
}

bool convt_k2s2(const Act &x, const Act &y, const float *w, const float *b, int kh, int kw, int stride, int act,
                hipStream_t s) {
    if (kh != 2 || kw != 2 || stride != 2 || !b) return false;
    if (x.c % 4 || y.c % 4 || x.cs % 4 || y.cs % 4 || 4 * x.c * y.c > CT2_MAXW) return false;
    if ((reinterpret_cast<uintptr_t>(x.p) & 15) || (reinterpret_cast<uintptr_t>(y.p) & 15)) return false;
    if (x.n != y.n || y.h > 2 * x.h || y.w > 2 * x.w || y.h < 1 || y.w < 1) return false;
    // Threads: channel quads x 2 phases x groups of 4 input columns (of the ceil(ow / 2) the row
    // reads) x output rows x images.
    const int nxg = ((y.w + 1) / 2 + 3) / 4;
    const long total = long(y.n) * y.h * nxg * 2 * (y.c / 4);
    ProbeScope probe("conv_transpose", s, 2.0 * double(y.pixels()) * x.c * y.c,
                     4.0 * double(x.count() + y.count()));
    // Four workgroups a CU: each fills its LDS once and walks several blocks of outputs.
    const unsigned grid = unsigned(std::min<long>((total + 255) / 256, 1024));
    hipLaunchKernelGGL(convt_k2s2_kernel, dim3(grid), dim3(256), size_t(4) * 4 * x.c * y.c, s, x.p, x.h, x.w, x.c,
                       long(x.cs), y.p, total, y.h, y.w, y.c, long(y.cs), nxg, w, b, act);
    OCR_HIP(hipGetLastError());
    return true;
}

void maxpool(const Act &x, const Act &y, int kh, int kw, hipStream_t s) {
    ProbeScope probe("maxpool", s, double(x.count()), 4.0 * double(x.count() + y.count()));
    hipLaunchKernelGGL(maxpool_kernel, dim3(blocks_for(y.count())), dim3(256), 0, s, x.p, x.n, x.h, x.w, x.c, x.cs,
                       y.p, y.h, y.w, y.cs, kh, kw);
    OCR_HIP(hipGetLastError());
}

void copy_act(const Act &x, const Act &y, int y0, int x0, hipStream_t s) {
    ProbeScope probe("copy", s, 0, 8.0 * double(y.count()));
    hipLaunchKernelGGL(copy_kernel, dim3(blocks_for(y.count())), dim3(256), 0, s, x.p, x.h, x.w, x.cs, y.p, y.n, y.h,
                       y.w, y.c, y.cs, y0, x0);
    OCR_HIP(hipGetLastError());
}

void activate(const Act &x, const Act &y, int act, hipStream_t s) {
    hipLaunchKernelGGL(activate_kernel, dim3(blocks_for(y.count())), dim3(256), 0, s, x.p, x.cs, y.p, y.cs, y.pixels(),
                       y.c, act);
    OCR_HIP(hipGetLastError());
}

void fill(float *p, size_t count, float v, hipStream_t s) {
    if (!count) return;
    hipLaunchKernelGGL(fill_kernel, dim3(blocks_for(count)), dim3(256), 0, s, p, count, v);
    OCR_HIP(hipGetLastError());
}

void grey_resize(const GreyPage *pages, int count, int ow, int oh, hipStream_t s) {
    ProbeScope probe("grey_resize", s, 0, 16.0 * double(ow) * oh * count);
    for (int k0 = 0; k0 < count; k0 += GPMAX) {
        GreyParams p{};
        const int cnt = std::min(GPMAX, count - k0);
        for (int k = 0; k < cnt; k++) p.pg[k] = pages[k0 + k];
        p.ow = ow;
        p.oh = oh;
        hipLaunchKernelGGL(grey_resize_kernel, dim3(blocks_for(size_t(ow) * oh), unsigned(cnt)), dim3(256), 0, s, p);
        OCR_HIP(hipGetLastError());
    }
}

void mask_up(const MaskPage *pages, int count, int stride, float thr, hipStream_t s) {
    double bytes = 0;
    size_t waves = 0;
    for (int k = 0; k < count; k++) {
        const int words = (pages[k].w + 31) / 32;
        bytes += 4.0 * double(pages[k].mw) * pages[k].mh + 4.0 * double(words) * pages[k].h;
        waves = std::max(waves, size_t((words + 2 * MJ - 1) / (2 * MJ)) * ((pages[k].h + MR - 1) / MR));
    }
    ProbeScope probe("mask_up", s, 0, bytes);
    for (int k0 = 0; k0 < count; k0 += GPMAX) {
        MaskParams p{};
        const int cnt = std::min(GPMAX, count - k0);
        for (int k = 0; k < cnt; k++) p.pg[k] = pages[k0 + k];
        p.stride = stride;
        p.thr = thr;
        hipLaunchKernelGGL(mask_up_kernel, dim3(blocks_for(waves * 64), unsigned(cnt)), dim3(256), 0, s, p);
        OCR_HIP(hipGetLastError());
    }
}

void conv1x1_narrow(const Act &x, const Act &y, const float *w, const float *b, int act, hipStream_t s) {
    if (y.c < 1 || y.c > 4 || x.c % 4 || x.cs % 4 || (reinterpret_cast<uintptr_t>(x.p) & 15) || x.n != y.n ||
        x.h != y.h || x.w != y.w)
        fail("conv1x1_narrow: shape");
    const long pixels = long(x.n) * x.h * x.w;
    ProbeScope probe("conv_narrow", s, 2.0 * double(pixels) * x.c * y.c, 4.0 * double(pixels) * (x.c + y.c));
    const dim3 grid(blocks_for(size_t(pixels))), blk(256);
    if (y.c == 1) hipLaunchKernelGGL((conv1x1_narrow_kernel<1>), grid, blk, 0, s, x.p, pixels, x.c, x.cs, y.p, y.cs, w, b, act);
    else if (y.c == 2) hipLaunchKernelGGL((conv1x1_narrow_kernel<2>), grid, blk, 0, s, x.p, pixels, x.c, x.cs, y.p, y.cs, w, b, act);
    else if (y.c == 3) hipLaunchKernelGGL((conv1x1_narrow_kernel<3>), grid, blk, 0, s, x.p, pixels, x.c, x.cs, y.p, y.cs, w, b, act);
    else hipLaunchKernelGGL((conv1x1_narrow_kernel<4>), grid, blk, 0, s, x.p, pixels, x.c, x.cs, y.p, y.cs, w, b, act);
    OCR_HIP(hipGetLastError());
}

void avgpool_t(const Act *xs, int count, int kh, float *X, int ntot, hipStream_t s) {
    if (count < 1) return;
    const int c = xs[0].c;
    double bytes = 0;
    int noff = 0;
    for (int k0 = 0; k0 < count; k0 += APMAXSEG) {
        const int cnt = std::min(APMAXSEG, count - k0);
        ApParams p{};
        p.nseg = cnt;
        p.kh = kh;
        p.c = c;
        p.ntot = ntot;
        p.X = X;
        long long blocks = 0;
        for (int k = 0; k < cnt; k++) {
            const Act &x = xs[k0 + k];
            if (kh < 1 || kh > x.h) fail("avgpool_t: pool height");
            if (x.c != c) fail("avgpool_t: channel counts differ");
            p.seg[k] = ApSeg{x.p, x.n, x.h, x.w, x.cs, noff, int(blocks)};
            blocks += (long long)((size_t(x.n) * x.w * c + 255) / 256);
            if (blocks > 2147483647LL) fail("avgpool_t: grid too large");
            noff += x.n;
            bytes += 4.0 * double(x.n) * x.w * c * (kh + 1);
        }
        if (noff > ntot) fail("avgpool_t: more lines than the output holds");
        if (blocks == 0) continue;
        ProbeScope probe("avgpool_t", s, 0, bytes);
        bytes = 0;
        hipLaunchKernelGGL(avgpool_t_kernel, dim3(unsigned(blocks)), dim3(256), 0, s, p);
        OCR_HIP(hipGetLastError());
    }
}

void argmax_rows(const float *x, int rows, int classes, uint32_t *best, hipStream_t s, const int *map) {
    if (rows <= 0) return;
    ProbeScope probe("argmax", s, 0, 4.0 * double(rows) * (classes + 1));
    hipLaunchKernelGGL(argmax_kernel, dim3(blocks_for(size_t(rows), 256 / AMAX_LANES)), dim3(256), 0, s, x, rows,
                       classes, best, map);
    OCR_HIP(hipGetLastError());
}

}  // namespace ocr
