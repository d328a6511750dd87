// Launchers of the N-D executor's kernels (kernels/nd.hip, kernels/bgemm.hip). Row-major
// (ONNX) float32 tensors.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "common.h"
#include "kernels.h"

namespace ocr {

constexpr int ND_RANK = 6;

// An index space of up to ND_RANK dimensions with two stride sets (in elements): for the copy,
// input and output strides; for a broadcast binary op, the strides of a and b (0 on a
// broadcast dimension).
struct NdIndex {
    size_t total = 0;
    int rank = 0;
    size_t dims[ND_RANK] = {};
    size_t s0[ND_RANK] = {}, s1[ND_RANK] = {};
};

enum UnaryOp : int { UN_RELU = 1, UN_SIGMOID = 2, UN_HARDSIGMOID = 3, UN_ERF = 4, UN_SQRT = 5 };
enum BinaryOp : int { BIN_ADD = 0, BIN_SUB = 1, BIN_MUL = 2, BIN_DIV = 3, BIN_POW = 4 };

void nd_unary(const float *x, float *y, size_t n, int op, float alpha, float beta, hipStream_t s);
void nd_binary(const float *a, const float *b, float *y, const NdIndex &ix, int op, hipStream_t s);
void nd_copy(const float *x, float *y, const NdIndex &ix, size_t ibase, size_t obase, hipStream_t s);
// y = x * st[c] + st[C + c], c = (i / inner) % C (BatchNormalization folded, nd.rs:788-800).
void nd_affine(const float *x, const float *st, float *y, size_t total, int c, size_t inner, hipStream_t s);
void nd_reduce_mean(const float *x, float *y, size_t rows, int len, hipStream_t s);
// gb: gamma[len] then beta[len].
void nd_layer_norm(const float *x, const float *gb, float *y, size_t rows, int len, float eps, hipStream_t s);
void nd_softmax(const float *x, float *y, size_t rows, int len, hipStream_t s);
// Arg-max per row, the first index on ties (src/nd.rs:383).
void nd_argmax(const float *x, uint32_t *best, size_t rows, int len, hipStream_t s);
// Reduces [rows][parts] (value, index-as-bits) pairs to the row's arg-max (first index on ties).
void nd_argmax_partials(const float *part, int parts, size_t rows, uint32_t *best, hipStream_t s);
void nd_pool(const float *x, float *y, size_t nc, int h, int w, int oh, int ow, int kh, int kw, int sh, int sw,
             int pt, int pl, bool avg, hipStream_t s);
void nd_resize_nearest(const float *x, float *y, size_t nc, int h, int w, int oh, int ow, float sy, float sx,
                       hipStream_t s);

// A Conv in NCHW on the general kernel (strided, grouped, depthwise). Epilogue:
// act(affine(acc + b)) + res, with in_scale[n][cin] applied to the input first (the SE gate).
struct NdConvArgs {
    const float *x = nullptr;
    int n = 0, cin = 0, h = 0, w = 0;
    const float *wt = nullptr;  // [cout][cin / group][kh][kw]
    const float *b = nullptr;
    const float *affine = nullptr;    // scale[cout] then shift[cout], or null
    const float *res = nullptr;       // [n][cout][oh][ow], or null
    const float *in_scale = nullptr;  // [n][cin], or null
    float *y = nullptr;
    int cout = 0, oh = 0, ow = 0, kh = 0, kw = 0, sh = 1, sw = 1, pt = 0, pl = 0, group = 1, act = 0;
};
void nd_conv_generic(const NdConvArgs &a, hipStream_t s);
// Depthwise (group = cin = cout, 3 x 3 or 5 x 5, strides 1 or 2 per axis; no residual or input
// scale), the taps summed as nd_conv_generic sums them. False (nothing launched) otherwise.
bool nd_conv_dw(const NdConvArgs &a, hipStream_t s);
// Group 1, 3 x 3, one or three input channels, at most 64 output channels, any stride (the
// stems): one thread an output pixel. False (nothing launched) otherwise.
bool nd_conv_small(const NdConvArgs &a, hipStream_t s);

// A group-1, stride-1 conv up to 3 x 3 in NCHW on the matrix cores (kernels/ndconv.hip), with
// the weights packed by pack_conv_weights: act(affine(acc + b)) + res, in_scale[n][cin] applied to
// the input first. False (nothing launched) for shapes it does not take.
struct NdMfmaConvArgs {
    const float *x = nullptr;
    int n = 0, cin = 0, h = 0, w = 0;
    float *y = nullptr;
    int cout = 0, oh = 0, ow = 0;
    const uint16_t *wt_hi = nullptr, *wt_lo = nullptr;
    ConvPack pk;
    const float *bias = nullptr, *affine = nullptr, *res = nullptr, *in_scale = nullptr;
    int pt = 0, pl = 0, act = ACT_NONE;
};
bool nd_conv_nchw_mfma(const NdMfmaConvArgs &a, hipStream_t s);

// y [m][n] = act(x [m][k] W + b) (+ res [m][n]) with W packed as n rows of k (pack_conv_weights,
// 1 x 1), on the matrix cores. False (nothing launched) for packs it does not take.
struct NdRowsArgs {
    const float *x = nullptr;
    int m = 0, k = 0, n = 0;
    const uint16_t *wt_hi = nullptr, *wt_lo = nullptr;
    ConvPack pk;
    const float *bias = nullptr, *res = nullptr;
    float *y = nullptr;
    int act = ACT_NONE;
};
bool nd_gemm_rows(const NdRowsArgs &a, hipStream_t s);
// The CTC head without its logits: per row of x, nd_head_parts partial (max, index bits) pairs of
// x W + b (first index on ties) at part[row * parts + j], for nd_argmax_partials. Needs 64-column
// blocks and k <= 256. False (nothing launched) otherwise.
int nd_head_parts(int m, const ConvPack &pk);
bool nd_head_argmax(const NdRowsArgs &a, float *part, int parts, hipStream_t s);

// ConvTranspose, group 1, no pads; wt is ONNX's [cin][cout][kh][kw].
void nd_conv_transpose(const float *x, int n, int cin, int h, int w, const float *wt, const float *b, float *y,
                       int cout, int kh, int kw, int stride, int act, hipStream_t s);
// The PP-OCR detection input: RGB bytes (h x w x 3) -> [1][3][oh][ow], bilinear half-pixel,
// BGR, ImageNet mean / deviation (src/nd.rs:172-204).
void nd_det_prep(const uint8_t *rgb, int w, int h, float *y, int ow, int oh, hipStream_t s);
// prob > thr as bit rows: h rows of ceil(w / 32) words, bit x % 32 of word x / 32.
void nd_threshold_bits(const float *prob, int w, int h, float thr, uint32_t *bits, hipStream_t s);

// Multi-head self-attention from a fused QKV projection: x [n][t][3 heads d] (q, k, v blocks of
// heads x d), y[i][j][h d + c] = sum_k softmax_k(scale q_j . k_k) v_k[c] (kernels/attn.hip).
void nd_attention(const float *x, int n, int t, int heads, int d, float scale, float *y, hipStream_t s);

// Batched C[b] = A[b] (M x K) * B[b] (K x N) on the matrix cores, both operands float32 split
// into float16 hi + lo (three passes: hi*hi, hi*lo, lo*hi), float32 accumulation. Element
// (m, k) of batch b of A is at a[b * sab + m * sam + k * sak]; likewise B and C.
struct BgemmArgs {
    const float *a = nullptr, *b = nullptr;
    float *c = nullptr;
    int batch = 0, m = 0, n = 0, k = 0;
    size_t sab = 0, sam = 0, sak = 0, sbb = 0, sbk = 0, sbn = 0, scb = 0, scm = 0, scn = 0;
};
void nd_bgemm(const BgemmArgs &g, hipStream_t s);

}  // namespace ocr
