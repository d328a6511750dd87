// Kernels of the N-D executor (the reference's src/nd.rs WGSL programs, nd.rs:32-408, restated
// for gfx950). Tensors are row-major float32 (ONNX's own layout). Elementwise and copy kernels
// walk flat indices with 64-bit arithmetic; reductions over a row give each row one wavefront
// (rows up to a few thousand long) or one workgroup (the 18 708-class rows), with DPP/shuffle
// reductions instead of the reference's thread-per-row loops.
#include <hip/hip_runtime.h>

#include <cmath>

#include "../nd_kernels.h"
#include "../runtime.h"

namespace ocr {

namespace {

inline unsigned grid_for(size_t n, int per = 256) {
    size_t b = (n + per - 1) / per;
    if (b > 0x7fffffff) fail("nd: grid too large");
    return unsigned(b ? b : 1);
}

__device__ inline float act_nd(float v, int act) {
    if (act == ACT_RELU) return fmaxf(v, 0.f);
    if (act == ACT_SIGMOID) return 1.f / (1.f + expf(-v));
    if (act == ACT_GELU) return 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    if (act == ACT_SILU) return v / (1.f + expf(-v));
    return v;
}

__device__ inline float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ inline float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// ---- unary (nd.rs nd_unary): 1 Relu, 2 Sigmoid, 3 HardSigmoid clamp(a v + b, 0, 1), 4 Erf, 5 Sqrt
__global__ void unary_kernel(const float *x, float *y, size_t n, int op, float alpha, float beta) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = x[i];
    switch (op) {
    case UN_RELU: v = fmaxf(v, 0.f); break;
    case UN_SIGMOID: v = 1.f / (1.f + expf(-v)); break;
    case UN_HARDSIGMOID: v = fminf(fmaxf(alpha * v + beta, 0.f), 1.f); break;
    case UN_ERF: v = erff(v); break;
    case UN_SQRT: v = sqrtf(v); break;
    default: break;
    }
    y[i] = v;
}

// ---- broadcast binary (nd.rs nd_binary): Add, Sub, Mul, Div, Pow (x^2 exactly when b == 2) --
__global__ void binary_kernel(const float *a, const float *b, float *y, NdIndex ix, int op) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= ix.total) return;
    size_t rem = i, ai = 0, bi = 0;
    for (int d = ix.rank - 1; d >= 0; d--) {
        const size_t c = rem % ix.dims[d];
        rem /= ix.dims[d];
        ai += c * ix.s0[d];
        bi += c * ix.s1[d];
    }
    const float u = a[ai], v = b[bi];
    float r;
    switch (op) {
    case BIN_ADD: r = u + v; break;
    case BIN_SUB: r = u - v; break;
    case BIN_MUL: r = u * v; break;
    case BIN_DIV: r = u / v; break;
    default: r = (v == 2.f) ? u * u : powf(u, v); break;
    }
    y[i] = r;
}

// ---- strided copy (nd.rs nd_copy): Transpose, Slice and Concat --------------------------------
__global__ void copy_nd_kernel(const float *x, float *y, NdIndex ix, size_t ibase, size_t obase) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= ix.total) return;
    size_t rem = i, xi = ibase, yi = obase;
    for (int d = ix.rank - 1; d >= 0; d--) {
        const size_t c = rem % ix.dims[d];
        rem /= ix.dims[d];
        xi += c * ix.s0[d];
        yi += c * ix.s1[d];
    }
    y[yi] = x[xi];
}

// ---- channel affine (BatchNormalization folded, nd.rs nd_affine) ----------------------------
__global__ void affine_kernel(const float *x, const float *st, float *y, size_t total, int c, size_t inner) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int ch = int((i / inner) % size_t(c));
    y[i] = __fmaf_rn(x[i], st[ch], st[c + ch]);
}

// ---- mean over a row (ReduceMean over trailing axes, GlobalAveragePool) -----------------------
__global__ void reduce_mean_kernel(const float *x, float *y, size_t rows, int len) {
    const size_t row = size_t(blockIdx.x) * (blockDim.x / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *r = x + row * size_t(len);
    float s = 0.f;
    for (int j = lane; j < len; j += 64) s += r[j];
    s = wave_sum(s);
    if (lane == 0) y[row] = s / float(len);
}

// ---- LayerNorm over the last axis (the exporter's 9-node chain, fused as nd.rs:583-611) -------
// (x - mean) / sqrt(var + eps) * gamma + beta, var the mean of squared deviations.
__global__ void layer_norm_kernel(const float *x, const float *gb, float *y, size_t rows, int len, float eps) {
    const size_t row = size_t(blockIdx.x) * (blockDim.x / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *r = x + row * size_t(len);
    float *o = y + row * size_t(len);
    float s = 0.f;
    for (int j = lane; j < len; j += 64) s += r[j];
    const float mean = wave_sum(s) / float(len);
    float v = 0.f;
    for (int j = lane; j < len; j += 64) {
        const float d = r[j] - mean;
        v += d * d;
    }
    const float den = sqrtf(wave_sum(v) / float(len) + eps);
    for (int j = lane; j < len; j += 64) o[j] = (r[j] - mean) / den * gb[j] + gb[len + j];
}

// ---- softmax over the last axis (nd.rs nd_softmax): one wavefront per row ---------------------
__global__ void softmax_wave_kernel(const float *x, float *y, size_t rows, int len) {
    const size_t row = size_t(blockIdx.x) * (blockDim.x / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float *r = x + row * size_t(len);
    float *o = y + row * size_t(len);
    float m = -INFINITY;
    for (int j = lane; j < len; j += 64) m = fmaxf(m, r[j]);
    m = wave_max(m);
    float s = 0.f;
    for (int j = lane; j < len; j += 64) s += expf(r[j] - m);
    s = wave_sum(s);
    for (int j = lane; j < len; j += 64) o[j] = expf(r[j] - m) / s;
}

// Long rows (the CTC head's 18 708 classes): one workgroup of 256 per row.
__global__ __launch_bounds__(256) void softmax_block_kernel(const float *x, float *y, int len) {
    __shared__ float part[4];
    const size_t row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *r = x + row * size_t(len);
    float *o = y + row * size_t(len);
    float m = -INFINITY;
    for (int j = tid; j < len; j += 256) m = fmaxf(m, r[j]);
    m = wave_max(m);
    if (lane == 0) part[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    __syncthreads();
    float s = 0.f;
    for (int j = tid; j < len; j += 256) s += expf(r[j] - m);
    s = wave_sum(s);
    if (lane == 0) part[wave] = s;
    __syncthreads();
    s = part[0] + part[1] + part[2] + part[3];
    for (int j = tid; j < len; j += 256) o[j] = expf(r[j] - m) / s;
}

// ---- arg-max over the last axis (nd.rs nd_argmax): the first index on ties (nd.rs:383) --------
__global__ __launch_bounds__(256) void argmax_first_kernel(const float *x, uint32_t *best, int len) {
    __shared__ float pv[4];
    __shared__ int pi[4];
    const size_t row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *r = x + row * size_t(len);
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int j = tid; j < len; j += 256) {
        const float v = r[j];
        if (v > bv) { bv = v; bi = j; }  // j increases: the first index wins ties
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { pv[wave] = bv; pi[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int k = 1; k < 4; k++)
            if (pv[k] > bv || (pv[k] == bv && pi[k] < bi)) { bv = pv[k]; bi = pi[k]; }
        best[row] = uint32_t(bi == 0x7fffffff ? 0 : bi);
    }
}

// Partial arg-max results (value, index) of the fused head GEMM, reduced per row: a wavefront
// per row, its lanes reading neighbouring partials (coalesced), then a butterfly over the lanes.
__global__ __launch_bounds__(256) void argmax_partials_kernel(const float2 *part, int parts, size_t rows,
                                                              uint32_t *best) {
    const size_t row = size_t(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int k = lane; k < parts; k += 64) {
        const float2 p = part[row * parts + k];
        const int idx = __float_as_int(p.y);
        if (p.x > bv || (p.x == bv && idx < bi)) { bv = p.x; bi = idx; }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) best[row] = uint32_t(bi == 0x7fffffff ? 0 : bi);
}

// ---- pooling (nd.rs nd_pool): stride, leading padding; the average never counts padding -------
__global__ void pool_nd_kernel(const float *x, float *y, size_t nc, int h, int w, int oh, int ow, int kh, int kw,
                               int sh, int sw, int pt, int pl, int avg) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= nc * oh * ow) return;
    const int ox = int(i % ow), oy = int((i / ow) % oh);
    const size_t c = i / (size_t(ow) * oh);
    const float *xc = x + c * h * w;
    float m = -INFINITY, s = 0.f;
    int n = 0;
    for (int ky = 0; ky < kh; ky++) {
        const int iy = oy * sh + ky - pt;
        if (iy < 0 || iy >= h) continue;
        for (int kx = 0; kx < kw; kx++) {
            const int ix = ox * sw + kx - pl;
            if (ix < 0 || ix >= w) continue;
            const float v = xc[size_t(iy) * w + ix];
            m = fmaxf(m, v);
            s += v;
            n++;
        }
    }
    y[i] = avg ? s / float(n > 0 ? n : 1) : m;
}

// ---- nearest Resize, asymmetric, floor (nd.rs nd_resize) --------------------------------------
__global__ void resize_nearest_kernel(const float *x, float *y, size_t nc, int h, int w, int oh, int ow, float sy,
                                      float sx) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= nc * oh * ow) return;
    const int ox = int(i % ow), oy = int((i / ow) % oh);
    const size_t c = i / (size_t(ow) * oh);
    const int iy = min(int(floorf(float(oy) / sy)), h - 1), ix = min(int(floorf(float(ox) / sx)), w - 1);
    y[i] = x[(c * h + iy) * w + ix];
}

// ---- any Conv in NCHW, one thread per output (strided, grouped / depthwise) -------------------
// Epilogue in the executor's order: act(affine(acc + bias)) + residual.
__global__ void conv_nchw_generic_kernel(NdConvArgs a) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t total = size_t(a.n) * a.cout * a.oh * a.ow;
    if (i >= total) return;
    const int ox = int(i % a.ow), oy = int((i / a.ow) % a.oh);
    const int co = int((i / (size_t(a.ow) * a.oh)) % a.cout);
    const int img = int(i / (size_t(a.ow) * a.oh * a.cout));
    const int cin_g = a.cin / a.group, cout_g = a.cout / a.group, g0 = (co / cout_g) * cin_g;
    float acc = 0.f;
    for (int c = 0; c < cin_g; c++) {
        const float *xc = a.x + (size_t(img) * a.cin + g0 + c) * a.h * a.w;
        const float sc = a.in_scale ? a.in_scale[size_t(img) * a.cin + g0 + c] : 1.f;
        const float *wc = a.wt + (size_t(co) * cin_g + c) * a.kh * a.kw;
        for (int ky = 0; ky < a.kh; ky++) {
            const int iy = oy * a.sh - a.pt + ky;
            if (iy < 0 || iy >= a.h) continue;
            for (int kx = 0; kx < a.kw; kx++) {
                const int ix = ox * a.sw - a.pl + kx;
                if (ix < 0 || ix >= a.w) continue;
                float xv = xc[size_t(iy) * a.w + ix];
                if (a.in_scale) xv *= sc;
                acc = __fmaf_rn(xv, wc[ky * a.kw + kx], acc);
            }
        }
    }
    float v = acc + (a.b ? a.b[co] : 0.f);
    if (a.affine) v = v * a.affine[co] + a.affine[a.cout + co];
    v = act_nd(v, a.act);
    if (a.res) v += a.res[i];
    a.y[i] = v;
}

// ---- ConvTranspose in NCHW (group 1, no pads), gather over the taps with k = o mod s ----------
__global__ void convt_nchw_kernel(const float *x, int n, int cin, int h, int w, const float *wt, const float *b,
                                  float *y, int cout, int oh, int ow, int kh, int kw, int s, int act) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(n) * cout * oh * ow) return;
    const int ox = int(i % ow), oy = int((i / ow) % oh);
    const int co = int((i / (size_t(ow) * oh)) % cout);
    const int img = int(i / (size_t(ow) * oh * cout));
    float acc = 0.f;
    for (int ky = oy % s; ky < kh && ky <= oy; ky += s) {
        const int iy = (oy - ky) / s;
        if (iy >= h) continue;
        for (int kx = ox % s; kx < kw && kx <= ox; kx += s) {
            const int ix = (ox - kx) / s;
            if (ix >= w) continue;
            const float *xp = x + (size_t(img) * cin * h + iy) * w + ix;
            const float *wp = wt + (size_t(co) * kh + ky) * kw + kx;  // [cin][cout][kh][kw]
            for (int ci = 0; ci < cin; ci++)
                acc = __fmaf_rn(xp[size_t(ci) * h * w], wp[size_t(ci) * cout * kh * kw], acc);
        }
    }
    y[i] = act_nd(acc + (b ? b[co] : 0.f), act);
}

// ConvTranspose with kernel = stride S (no overlap: input pixel (iy, ix) alone makes the S x S
// outputs (S iy + a, S ix + b)): a thread per input pixel and output channel, the channel sum in
// the order convt_nchw_kernel takes it, the S x S results stored as S rows of S neighbours.
template <int S>
__global__ void convt_ks_nchw_kernel(const float *x, int n, int cin, int h, int w, const float *wt, const float *b,
                                     float *y, int cout, int act) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(n) * cout * h * w) return;
    const int ix = int(i % w), iy = int((i / w) % h);
    const int co = int((i / (size_t(w) * h)) % cout);
    const int img = int(i / (size_t(w) * h * cout));
    float acc[S][S];
#pragma unroll
    for (int a = 0; a < S; a++)
#pragma unroll
        for (int c = 0; c < S; c++) acc[a][c] = 0.f;
    const float *xp = x + (size_t(img) * cin * h + iy) * w + ix;
    const float *wp = wt + size_t(co) * S * S;  // [cin][cout][S][S]
    for (int ci = 0; ci < cin; ci++) {
        const float xv = xp[size_t(ci) * h * w];
        const float *wc = wp + size_t(ci) * cout * S * S;
#pragma unroll
        for (int a = 0; a < S; a++)
#pragma unroll
            for (int c = 0; c < S; c++) acc[a][c] = __fmaf_rn(xv, wc[a * S + c], acc[a][c]);
    }
    const float bv = b ? b[co] : 0.f;
    const int ow = w * S;
    float *yp = y + ((size_t(img) * cout + co) * h * S + size_t(iy) * S) * ow + size_t(ix) * S;
#pragma unroll
    for (int a = 0; a < S; a++)
#pragma unroll
        for (int c = 0; c < S; c++) yp[size_t(a) * ow + c] = act_nd(acc[a][c] + bv, act);
}

// ---- PP-OCR detection input (nd.rs nd_det_prep, src/nd.rs:1353-1369) -------------------------
// WGSL mix(a, b, t) = a (1 - t) + b t, each operation rounded on its own: contraction into
// fused multiply-adds is off in the front-end kernels so they follow the stated arithmetic.
__device__ inline float mix_ref(float a, float b, float t) {
#pragma clang fp contract(off)
    return a * (1.f - t) + b * t;
}

__global__ void det_prep_kernel(const uint8_t *rgb, int w, int h, float *y, int ow, int oh, float sx, float sy) {
#pragma clang fp contract(off)
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= ow * oh) return;
    const int ox = i % ow, oy = i / ow;
    const float ix = fminf(fmaxf(sx * (float(ox) + 0.5f) - 0.5f, 0.f), float(w) - 1.f);
    const float iy = fminf(fmaxf(sy * (float(oy) + 0.5f) - 0.5f, 0.f), float(h) - 1.f);
    const int x1 = int(ix), y1 = int(iy), x2 = min(x1 + 1, w - 1), y2 = min(y1 + 1, h - 1);
    const float fx = ix - float(x1), fy = iy - float(y1);
    const float mean[3] = {0.485f, 0.456f, 0.406f}, dev[3] = {0.229f, 0.224f, 0.225f};
    for (int c = 0; c < 3; c++) {
        const int k = 2 - c;  // BGR: output channel 0 is the blue byte
        const float a = mix_ref(float(rgb[(size_t(y1) * w + x1) * 3 + k]), float(rgb[(size_t(y1) * w + x2) * 3 + k]), fx);
        const float bb = mix_ref(float(rgb[(size_t(y2) * w + x1) * 3 + k]), float(rgb[(size_t(y2) * w + x2) * 3 + k]), fx);
        y[size_t(c) * ow * oh + i] = (mix_ref(a, bb, fy) / 255.f - mean[c]) / dev[c];
    }
}

// ---- DB threshold (the host step of ppdet.rs:88 moved to the GPU): prob > thr as bit rows ------
__global__ void threshold_bits_kernel(const float *prob, int w, int h, float thr, uint32_t *bits) {
    const int words = (w + 31) / 32;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= words * h) return;
    const int wx = i % words, y = i / words;
    uint32_t out = 0;
    for (int b = 0; b < 32; b++) {
        const int x = wx * 32 + b;
        if (x >= w) break;
        if (prob[size_t(y) * w + x] > thr) out |= 1u << b;
    }
    bits[i] = out;
}

}  // namespace

void nd_unary(const float *x, float *y, size_t n, int op, float alpha, float beta, hipStream_t s) {
    if (!n) return;
    ProbeScope probe("nd_elementwise", s, 0, 8.0 * double(n));
    hipLaunchKernelGGL(unary_kernel, dim3(grid_for(n)), dim3(256), 0, s, x, y, n, op, alpha, beta);
    OCR_HIP(hipGetLastError());
}

void nd_binary(const float *a, const float *b, float *y, const NdIndex &ix, int op, hipStream_t s) {
    if (!ix.total) return;
    ProbeScope probe("nd_elementwise", s, 0, 12.0 * double(ix.total));
    hipLaunchKernelGGL(binary_kernel, dim3(grid_for(ix.total)), dim3(256), 0, s, a, b, y, ix, op);
    OCR_HIP(hipGetLastError());
}

void nd_copy(const float *x, float *y, const NdIndex &ix, size_t ibase, size_t obase, hipStream_t s) {
    if (!ix.total) return;
    ProbeScope probe("nd_copy", s, 0, 8.0 * double(ix.total));
    hipLaunchKernelGGL(copy_nd_kernel, dim3(grid_for(ix.total)), dim3(256), 0, s, x, y, ix, ibase, obase);
    OCR_HIP(hipGetLastError());
}

void nd_affine(const float *x, const float *st, float *y, size_t total, int c, size_t inner, hipStream_t s) {
    if (!total) return;
    ProbeScope probe("nd_elementwise", s, 0, 8.0 * double(total));
    hipLaunchKernelGGL(affine_kernel, dim3(grid_for(total)), dim3(256), 0, s, x, st, y, total, c, inner);
    OCR_HIP(hipGetLastError());
}

void nd_reduce_mean(const float *x, float *y, size_t rows, int len, hipStream_t s) {
    if (!rows) return;
    ProbeScope probe("nd_reduce", s, 0, 4.0 * double(rows) * (len + 1));
    hipLaunchKernelGGL(reduce_mean_kernel, dim3(grid_for(rows, 4)), dim3(256), 0, s, x, y, rows, len);
    OCR_HIP(hipGetLastError());
}

void nd_layer_norm(const float *x, const float *gb, float *y, size_t rows, int len, float eps, hipStream_t s) {
    if (!rows) return;
    ProbeScope probe("nd_layer_norm", s, 0, 8.0 * double(rows) * len);
    hipLaunchKernelGGL(layer_norm_kernel, dim3(grid_for(rows, 4)), dim3(256), 0, s, x, gb, y, rows, len, eps);
    OCR_HIP(hipGetLastError());
}

void nd_softmax(const float *x, float *y, size_t rows, int len, hipStream_t s) {
    if (!rows) return;
    ProbeScope probe("nd_softmax", s, 0, 8.0 * double(rows) * len);
    if (len > 2048) {
        if (rows > 0x7fffffff) fail("nd_softmax: too many rows");
        hipLaunchKernelGGL(softmax_block_kernel, dim3(unsigned(rows)), dim3(256), 0, s, x, y, len);
    } else {
        hipLaunchKernelGGL(softmax_wave_kernel, dim3(grid_for(rows, 4)), dim3(256), 0, s, x, y, rows, len);
    }
    OCR_HIP(hipGetLastError());
}

void nd_argmax(const float *x, uint32_t *best, size_t rows, int len, hipStream_t s) {
    if (!rows) return;
    if (rows > 0x7fffffff) fail("nd_argmax: too many rows");
    ProbeScope probe("nd_argmax", s, 0, 4.0 * double(rows) * len);
    hipLaunchKernelGGL(argmax_first_kernel, dim3(unsigned(rows)), dim3(256), 0, s, x, best, len);
    OCR_HIP(hipGetLastError());
}

void nd_argmax_partials(const float *part, int parts, size_t rows, uint32_t *best, hipStream_t s) {
    if (!rows) return;
    ProbeScope probe("nd_argmax", s, 0, 8.0 * double(rows) * parts + 4.0 * double(rows));
    hipLaunchKernelGGL(argmax_partials_kernel, dim3(grid_for(rows, 4)), dim3(256), 0, s,
                       reinterpret_cast<const float2 *>(part), parts, rows, best);
    OCR_HIP(hipGetLastError());
}

void nd_pool(const float *x, float *y, size_t nc, int h, int w, int oh, int ow, int kh, int kw, int sh, int sw,
             int pt, int pl, bool avg, hipStream_t s) {
    const size_t total = nc * oh * ow;
    if (!total) return;
    ProbeScope probe("nd_pool", s, 0, 4.0 * double(nc) * (double(h) * w + double(oh) * ow));
    hipLaunchKernelGGL(pool_nd_kernel, dim3(grid_for(total)), dim3(256), 0, s, x, y, nc, h, w, oh, ow, kh, kw, sh, sw,
                       pt, pl, avg ? 1 : 0);
    OCR_HIP(hipGetLastError());
}

void nd_resize_nearest(const float *x, float *y, size_t nc, int h, int w, int oh, int ow, float sy, float sx,
                       hipStream_t s) {
    const size_t total = nc * oh * ow;
    if (!total) return;
    ProbeScope probe("nd_resize", s, 0, 4.0 * double(nc) * (double(h) * w + double(oh) * ow));
    hipLaunchKernelGGL(resize_nearest_kernel, dim3(grid_for(total)), dim3(256), 0, s, x, y, nc, h, w, oh, ow, sy, sx);
    OCR_HIP(hipGetLastError());
}

void nd_conv_generic(const NdConvArgs &a, hipStream_t s) {
    const size_t total = size_t(a.n) * a.cout * a.oh * a.ow;
    if (!total) return;
    ProbeScope probe("nd_conv_generic", s, 2.0 * double(total) * (a.cin / a.group) * a.kh * a.kw,
                     4.0 * (double(a.n) * a.cin * a.h * a.w + double(total)));
    hipLaunchKernelGGL(conv_nchw_generic_kernel, dim3(grid_for(total)), dim3(256), 0, s, a);
    OCR_HIP(hipGetLastError());
}

void nd_conv_transpose(const float *x, int n, int cin, int h, int w, const float *wt, const float *b, float *y,
                       int cout, int kh, int kw, int stride, int act, hipStream_t s) {
    const int oh = (h - 1) * stride + kh, ow = (w - 1) * stride + kw;
    const size_t total = size_t(n) * cout * oh * ow;
    if (!total) return;
    ProbeScope probe("nd_conv_transpose", s, 2.0 * double(n) * h * w * cin * cout * kh * kw,
                     4.0 * (double(n) * cin * h * w + double(total)));
    const size_t inputs = size_t(n) * cout * h * w;
    if (kh == stride && kw == stride && stride >= 1 && stride <= 4) {
        if (stride == 2)
            hipLaunchKernelGGL(convt_ks_nchw_kernel<2>, dim3(grid_for(inputs)), dim3(256), 0, s, x, n, cin, h, w, wt, b, y,
                               cout, act);
        else if (stride == 1)
            hipLaunchKernelGGL(convt_ks_nchw_kernel<1>, dim3(grid_for(inputs)), dim3(256), 0, s, x, n, cin, h, w, wt, b, y,
                               cout, act);
        else if (stride == 3)
            hipLaunchKernelGGL(convt_ks_nchw_kernel<3>, dim3(grid_for(inputs)), dim3(256), 0, s, x, n, cin, h, w, wt, b, y,
                               cout, act);
        else
            hipLaunchKernelGGL(convt_ks_nchw_kernel<4>, dim3(grid_for(inputs)), dim3(256), 0, s, x, n, cin, h, w, wt, b, y,
                               cout, act);
    } else {
        hipLaunchKernelGGL(convt_nchw_kernel, dim3(grid_for(total)), dim3(256), 0, s, x, n, cin, h, w, wt, b, y, cout, oh,
                           ow, kh, kw, stride, act);
    }
    OCR_HIP(hipGetLastError());
}

void nd_det_prep(const uint8_t *rgb, int w, int h, float *y, int ow, int oh, hipStream_t s) {
    ProbeScope probe("nd_det_prep", s, 0, 12.0 * double(ow) * oh + 12.0 * double(ow) * oh);
    hipLaunchKernelGGL(det_prep_kernel, dim3(grid_for(size_t(ow) * oh)), dim3(256), 0, s, rgb, w, h, y, ow, oh,
                       float(w) / float(ow), float(h) / float(oh));
    OCR_HIP(hipGetLastError());
}

void nd_threshold_bits(const float *prob, int w, int h, float thr, uint32_t *bits, hipStream_t s) {
    const size_t words = size_t((w + 31) / 32) * h;
    ProbeScope probe("nd_threshold", s, 0, 4.0 * double(w) * h + 4.0 * double(words));
    hipLaunchKernelGGL(threshold_bits_kernel, dim3(grid_for(words)), dim3(256), 0, s, prob, w, h, thr, bits);
    OCR_HIP(hipGetLastError());
}

}  // namespace ocr
