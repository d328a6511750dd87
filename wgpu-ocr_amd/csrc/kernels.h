// Host-side launchers of the HIP kernels (each defined next to its kernel in kernels/*.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace ocr {

// ---- MFMA implicit-GEMM convolution (kernels/conv.hip) ----------------------------------
// Weights are packed once per layer by pack_conv_weights: float16 hi (exact when the model's
// weights are float16 values) and, if not exact, the float16 remainder lo.
struct ConvPack {
    int cin = 0, cout = 0, kh = 0, kw = 0;
    int bn = 0;       // output channels per workgroup: 16, 32 or 64
    int chunks = 0;   // input channels in slices of 32
    int nblocks = 0;  // ceil(cout / bn)
    bool exact = true;
    size_t halves() const { return size_t(nblocks) * chunks * kh * kw * bn * 32; }
    // Weight slices of the fragment layout (pack_conv_frags): the float16 values, then, for
    // weights that are not all float16 values, their float16 remainders as further slices.
    int frag_chunks() const { return exact ? chunks : 2 * chunks; }
    size_t frag_halves() const { return halves() * (exact ? 1 : 2); }
};

// Layout of a packed weight set: [nblock][chunk][tap][bn][32 input channels], float16.
// w is ONNX's [cout][cin][kh][kw]. Returns the pack description; hi/lo (host) are filled.
ConvPack plan_conv_pack(int cin, int cout, int kh, int kw);
void pack_conv_weights(const ConvPack &pk, const float *w, uint16_t *hi, uint16_t *lo, bool *exact);
// The same weights as MFMA fragments for the DMA-fed kernels: [16-channel tile][slice][tap]
// [lane][8], lane 16 g + r holding inputs 8g..8g+7 of channel 16 * tile + r. Slices 0 .. chunks-1
// hold hi; when the pack is not exact, slices chunks .. 2 chunks-1 hold lo (the kernels run the
// input's slices twice, so sum x (hi + lo) gives float32-class products). pk.frag_halves() halves.
void pack_conv_frags(const ConvPack &pk, const uint16_t *hi, const uint16_t *lo, uint16_t *frag);

struct ConvArgs {
    Act x, y;                       // input and output views (NHWC, or NCHW with nchw set)
    const uint16_t *wt_hi = nullptr, *wt_lo = nullptr;
    const uint16_t *wt_frag = nullptr;  // pack_conv_frags of wt_hi (conv_igemm), or null
    const float *bias = nullptr;    // [cout] or null
    const float *res = nullptr;     // residual added after the activation (gpu.rs:65), or null
    int res_cs = 0;
    int pt = 0, pl = 0;             // leading pads (stride 1)
    int act = ACT_NONE;
    bool nchw = false;              // x and y (and res) are NCHW tensors (the N-D executor)
    const float *affine = nullptr;  // BatchNormalization folded: scale[cout] then shift[cout]
    const float *in_scale = nullptr;  // [n][cin] input scale (the SE gate), or null
    // When set, no output is written: for every output pixel (GEMM row) and block of BN
    // channels, (max value, index as float bits) of acc + bias, first index on ties, at
    // amax_part[pixel * nblocks + block] (float2 pairs).
    float *amax_part = nullptr;
    // MaxPool (ph, pw) fused (kernel = stride, floor; NHWC, 3 x 3 only): the pooled output goes
    // to ypool; the full-size output to y as well when keep_full (its other readers need it).
    Act ypool;
    int ph = 1, pw = 1;
    bool keep_full = true;
    // NHWC output pixel strides (0: dense): column, row and image steps in pixels, so a conv can
    // write one phase of a strided output (ConvTranspose's sub-pixel phases).
    long y_px = 0, y_row = 0, y_img = 0;
    // 1 x 1 GEMM over x = [1][1][M] pixels: GEMM row i reads x's row rows[i] and writes y's row
    // rows[i] (M = x.w entries), so only the listed rows are computed; or null (dense).
    const int *rows = nullptr;
    // ConvTranspose with kernel = stride s as one 1 x 1 GEMM over the input pixels: output
    // channel k * ph_cout + c of input pixel (i, j) is channel c of y's pixel
    // (s i + k / s, s j + k % s) (conv_igemm only; 0: off).
    int ph_cout = 0, ph_s = 0;
    // conv3x3_dma only: with a 2 x 1 MaxPool of a 4-row output, the two pooled rows averaged into
    // one (AveragePool (2, 1)) and written time-major: column t of image i to
    // tm[(t * tm_ntot + tm_noff + i) * cout + c]; nothing else is written (0: off).
    float *tm = nullptr;
    int tm_ntot = 0, tm_noff = 0;
    ConvPack pk;
};
// True when the MFMA path takes this shape (stride 1, kernel at most 3 x 3).
bool conv_mfma_supported(int kh, int kw, int sh, int sw);
// Runs the convolution on the matrix cores: conv_igemm when it takes the shape, else the general
// kernel (NCHW, SE input scale, BatchNormalization affine, residual, arg-max partials, any pool).
void conv_mfma(const ConvArgs &a, hipStream_t s);
// The NHWC hot path (kernels/igemm.hip): kernel up to 3 x 3, float16-exact weights, bias +
// activation, optional 2 x 2 / 2 x 1 MaxPool, output pixel strides or a GEMM row map. Returns
// false (and launches nothing) for anything else.
bool conv_igemm(const ConvArgs &a, hipStream_t s);
// 1 x 1 convolution / GEMM (kernels/gemm.hip): NHWC pixels or GEMM rows with a row map, at
// least four 32-wide input chunks, float16-exact weights with wt_frag, bias + ReLU / Sigmoid.
// Returns false (and launches nothing) for anything else.
bool gemm_dma(const ConvArgs &a, hipStream_t s);
// 3 x 3, pad 1, NHWC, float16-exact weights with wt_frag, bias +
// ReLU / Sigmoid, optional 2 x 2 / 2 x 1 MaxPool (kernels/conv3.hip): operands fed by LDS DMA.
// Returns false (and launches nothing) for anything else.
bool conv3x3_dma(const ConvArgs &a, hipStream_t s);
// The same conv over several tensors in one launch (the width batches of a recogniser pass): same
// weights, bias, activation, pool, height and channel layout, any widths and image counts.
// Returns false (and launches nothing) unless every one is taken and they are alike.
bool conv3x3_dma_multi(const ConvArgs *args, int count, hipStream_t s);
// 1 x 1 convolution to at most 4 output channels (a detector head) in float32 on the vector ALU:
// bandwidth-bound, one thread a pixel (kernels/ops.hip). w [cout][cin] float32.
void conv1x1_narrow(const Act &x, const Act &y, const float *w, const float *b, int act, hipStream_t s);

// ---- Everything else (kernels/ops.hip) ----------------------------------------------------
// Any conv (grouped, strided) in float32, one thread per output: the fallback path.
void conv_generic(const Act &x, const Act &y, const float *w, const float *b, int kh, int kw, int sh, int sw,
                  int pt, int pl, int group, int act, hipStream_t s);
// One input channel, stride 1, act, and a fused MaxPool (ph, pw) (gpu.rs:385-422).
void conv_direct(const Act &x, const Act &y, const float *w, const float *b, int kh, int kw, int pad, int act,
                 int ph, int pw, hipStream_t s,
                 const uint16_t *frag = nullptr);
// The matrix-core path of conv_direct (kernels/conv1.hip): 3 x 3, pad 1, 16 to 64 output channels
// (a multiple of 16), float16-exact weights packed by pack_conv1_frags ([cout][9] float32 in,
// cout / 16 KiB of fragments out), no pool or a 2 x 2 one. Returns false for anything else.
void pack_conv1_frags(const float *w, int cout, uint16_t *frag);
// With ypool (2 x 2 pool, full-size y) both outputs are written.
bool conv1_mfma(const Act &x, const Act &y, const uint16_t *frag, const float *b, int act, int ph, int pw,
                hipStream_t s, const Act *ypool = nullptr);
// The same over count inputs of one height (any widths and image counts), one launch for up to
// 32 of them; ypool is null or an array of count pooled outputs.
bool conv1_mfma_multi(const Act *x, const Act *y, const Act *ypool, int count, const uint16_t *frag, const float *b,
                      int act, int ph, int pw, hipStream_t s);
// ConvTranspose gather form (gpu.rs:424-460); w re-laid out as [ky][kx][cin][cout].
void conv_transpose(const Act &x, const Act &y, const float *w, const float *b, int kh, int kw, int stride,
                    int act, hipStream_t s);
// The same for kernel = stride = 2 with channel counts multiples of 4 and 4 cin cout <= 16384
// (the weights in LDS): one float32 pass at HBM speed. False (nothing launched) otherwise.
bool convt_k2s2(const Act &x, const Act &y, const float *w, const float *b, int kh, int kw, int stride, int act,
                hipStream_t s);
// ConvTranspose (stride s <= 4, kernel at least the stride) as one matrix-core GEMM over the
// output's s x s blocks (kernels/convt_rows.hip): pk packs the cin -> s s cout weights as a
// pk.kh x pk.kw conv over the input (tap (a, b) reads x[i - (kh - 1 - a)][j - (kw - 1 - b)];
// output column k cout + c is channel c of phase k = py s + px; 1 x 1 when kernel = stride), b
// the cout biases, act none / ReLU / Sigmoid. False (nothing launched) for anything else.
bool convt_rows(const Act &x, const Act &y, const uint16_t *whi, const uint16_t *wlo, const ConvPack &pk,
                const float *b, int stride, int act, hipStream_t st);
void maxpool(const Act &x, const Act &y, int kh, int kw, hipStream_t s);
void copy_act(const Act &x, const Act &y, int y0, int x0, hipStream_t s);  // Slice / Concat copies
void activate(const Act &x, const Act &y, int act, hipStream_t s);
void fill(float *p, size_t count, float v, hipStream_t s);
// RGB bytes -> ocrs grey, padded with black (to pw x ph), bilinear to ow x oh (gpu.rs:530-561):
// every page of a detection pass in one launch.
struct GreyPage {
    const uint8_t *rgb;
    int w, h, pw, ph;
    float *y;
    float sx, sy;
};
void grey_resize(const GreyPage *pages, int count, int ow, int oh, hipStream_t s);
// Model output (row stride `stride`, valid mw x mh) -> page size bits (gpu.rs:563-593): every
// page of a detection pass in one launch.
struct MaskPage {
    const float *m;
    int mw, mh;
    uint32_t *bits;
    int w, h;
    float sx, sy;
};
void mask_up(const MaskPage *pages, int count, int stride, float thr, hipStream_t s);
// Run-length labelling of detection masks (kernels/ccl.hip): for every page, its runs row by
// row (row y's are [row_off[y], row_off[y + 1]), pixels x0[i] .. x1[i]) and root[i], the first
// run of run i's 8-connected component. row_off has h + 1 entries; when the page has more than
// cap runs only row_off and *total (the run count) are written. Widths and heights up to 65536.
struct CclPage {
    const uint32_t *bits;
    int w, h;
    uint16_t *x0, *x1;
    int32_t *root, *row_off;
    int cap;
    int32_t *total;  // [0] runs, [1] components, [2] row slots (the rest of 4 ints unused)
    uint16_t *ry;    // scratch: each run's row (cap entries)
    int32_t *cbot;   // scratch (cap): a root's bottom row, then its first row slot
    // Every component as {first run, top row, rows, first slot} (unordered, ccap entries), and
    // per row slot the component's leftmost and rightmost pixel in that row (scap entries each).
    // Past either capacity (or cap runs) the totals say so and these hold nothing usable.
    int32_t *comps;
    uint32_t *xmin, *xmax;
    int ccap, scap;
};
void ccl_runs(const CclPage *pages, int count, hipStream_t s);
// AvgPool (kh, 1) over the first kh rows to one row, written time-major into X[t][ntot][c]
// (gpu.rs:595-614): the count inputs (same channel count) at line offsets 0, n0, n0 + n1, ...
void avgpool_t(const Act *xs, int count, int kh, float *X, int ntot, hipStream_t s);
// Per row of [rows][classes]: the arg-max, the last index on ties (ocr-bench.rs:67). With a row
// map, row i is physical row map[i] of x and of best.
void argmax_rows(const float *x, int rows, int classes, uint32_t *best, hipStream_t s, const int *map = nullptr);

// ---- GRU recurrence (kernels/gru.hip) -------------------------------------------------------
// One layer, both directions, every line with its own length (gpu.rs:680-819). G [t][n][1536]
// holds W x + Wb; R [2][768][256] float16 (exact values); Rb [2][768]; Y [t][n][512].
// steps: the sum of lens (for the probe's work count only).
void gru_recurrence(const float *G, const uint16_t *R, const float *Rb, float *Y, const uint32_t *lens, int ntot,
                    int tmax, long long steps, hipStream_t s);
// The same with float32 recurrent weights, given transposed: Rt [2][256 k][768 rows] (for R
// that is not float16-valued when rounding it is not allowed; R streams from L2 every step).
void gru_recurrence_f32(const float *G, const float *Rt, const float *Rb, float *Y, const uint32_t *lens, int ntot,
                        long long steps, hipStream_t s);

}  // namespace ocr
