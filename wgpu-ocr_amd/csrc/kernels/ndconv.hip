// The N-D executor's convolutions and row GEMMs (the reference's nd_conv / nd_matmul programs,
// src/nd.rs:222-358, run by NdGraph::run, nd.rs:834-1195) for row-major (ONNX NCHW) float32
// tensors on gfx950.
//
// conv_nchw: group-1, stride-1 convolutions up to 3 x 3 on the matrix cores
// (v_mfma_f32_16x16x32_f16). No LDS staging: every wavefront loads its own operands. The A
// operand is 16 neighbouring output pixels of one row x 32 input channels, eight reads a lane of
// one channel plane each (16 lanes read 64 neighbouring bytes); the B operand is 32 input channels
// x 16 output channels of the packed float16 weights, one 16-byte read a lane. The float32
// inputs are split into float16 hi + lo (x = hi + lo to about 2^-22) and both go through the
// matrix core, accumulating in float32: float32-class results. A lane's four accumulators are
// four neighbouring pixels of one output channel, stored with one 16-byte write. A wavefront owns 16 MT pixels of one output row (of the flattened plane for a
// 1 x 1 conv) and 16 NT output channels; when there are too few such tiles to fill the GPU, up
// to four wavefronts of a workgroup share one tile's K steps and add their accumulators through
// LDS in a fixed order. Kernel rows that fall wholly into the padding are skipped (a 3 x 3 conv
// over a one-row tensor does one row of work).
//
// conv_dw: depthwise convolution, one thread an output, the taps summed in the order the general
// kernel sums them (the same float32 results).
// conv_small: group-1 convolutions with at most 27 taps in all (the 3-channel stems), one thread
// an output pixel for every output channel, the weights in LDS.
// gemm_rows: x [m][k] by packed weights to y [m][n] (MatMul + bias + activation), a wavefront a
// 16 RT x 16 NT tile with its operands read straight from memory; with `amax` the logits are
// never written: each wavefront walks a range of 64-column blocks keeping every row's best
// (value, index), first index on ties, and writes one partial a row (the CTC head).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "../kernels.h"
#include "../nd_kernels.h"
#include "../runtime.h"

namespace ocr {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

__device__ inline float act_dev(float v, int act) {
    if (act == ACT_RELU) return fmaxf(v, 0.f);
    if (act == ACT_SIGMOID) return 1.f / (1.f + expf(-v));
    if (act == ACT_GELU) return 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    if (act == ACT_SILU) return v / (1.f + expf(-v));
    return v;
}

__device__ inline void split8(const float (&v)[8], half8 &hi, half8 &lo) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const _Float16 h = (_Float16)v[j];
        hi[j] = h;
        lo[j] = (_Float16)(v[j] - (float)h);
    }
}

// ---- conv_nchw -------------------------------------------------------------------------------
struct NchwParams {
    const float *x;
    float *y;
    const half8 *wt, *wt_lo;  // [nblock][chunk][tap][bn][32] float16 (hi; lo when not exact)
    const float *bias, *affine, *res, *in_scale;
    int n, cin, h, w, cout, oh, ow;
    int bn, chunks, kh, kw, pt, pl, act;
    int flat;        // 1 x 1: pixels run over the flattened plane (h * w of them)
    int tiles_line;  // wavefront tiles along an output row (flat: along a plane)
    int tiles;       // all tiles of one channel block: lines x tiles_line
    int ksplit;      // wavefronts sharing one tile's K steps (1, 2 or 4 of 4; 8 or 16 of 16)
};

// WPB wavefronts a workgroup: 4, or 16 for launches of few tiles and long K (up to 16 wavefronts
// share one tile's K steps).
template <int MT, int NT, bool LO, int WPB>
__global__ __launch_bounds__(64 * WPB) void conv_nchw_kernel(NchwParams p) {
    extern __shared__ float s_red[];  // ksplit > 1: [wave][MT * NT * 4][64 lanes]
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = blockIdx.x * (WPB / p.ksplit) + wave / p.ksplit;
    const int kpart = wave % p.ksplit;
    const int nb = blockIdx.y;
    const int r = lane & 15, g = lane >> 4;
    const bool live = tile < p.tiles;
    const int lim = p.flat ? p.h * p.w : p.w;  // input pixels along a tile's line
    const size_t plane = size_t(p.h) * p.w;
    const unsigned planeu = unsigned(plane);

    floatx4 acc[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; m++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[m][t] = floatx4{0.f, 0.f, 0.f, 0.f};

    int img = 0, oy = 0, x0 = 0;
    if (live) {
        const int line = tile / p.tiles_line;
        x0 = (tile - line * p.tiles_line) * (16 * MT);
        if (p.flat) {
            img = line;
        } else {
            img = line / p.oh;
            oy = line - img * p.oh;
        }
        const int taps = p.kh * p.kw, steps = p.chunks * taps;
        const float *xim = p.x + size_t(img) * p.cin * plane;
        // K step s is (chunk, tap); steps whose kernel row reads only padding are skipped (the
        // same for the whole wavefront).
        auto valid_from = [&](int s) {
            for (; s < steps; s += p.ksplit) {
                if (p.flat) return s;
                const int tap = s % taps, iy = oy + tap / p.kw - p.pt;
                if (iy >= 0 && iy < p.h) return s;
            }
            return steps;
        };
        // Operands of one K step: the weight fragments and the float32 inputs (split at use).
        half8 a[NT], al[NT];
        float v[MT][8];
        auto load = [&](int s, half8 (&wa)[NT], half8 (&wl)[NT], float (&xv)[MT][8]) {
            const int chunk = s / taps, tap = s - chunk * taps;
            const int ky = tap / p.kw, kx = tap - ky * p.kw;
            const size_t wo = (size_t(nb * p.chunks + chunk) * taps + tap) * (p.bn * 4) + size_t(r) * 4 + g;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                wa[t] = p.wt[wo + t * 64];
                if constexpr (LO) wl[t] = p.wt_lo[wo + t * 64];
            }
            const int c0 = chunk * 32 + 8 * g;
            // The row base is the same for the whole wavefront; a lane's inputs are 32-bit byte
            // offsets from it (an image holds fewer than 2^30 values, checked by the host). The
            // reads are unconditional, from a position inside the image (channel clamped to the
            // last, pixel to the row's first), and the values outside are zeroed after.
            const float *xrow = xim + (p.flat ? 0 : size_t(oy + ky - p.pt) * p.w);
            const bool full = c0 + 8 <= p.cin;
#pragma unroll
            for (int m = 0; m < MT; m++) {
                const int px = x0 + 16 * m + r + (p.flat ? 0 : kx - p.pl);
                const bool in = px >= 0 && px < lim;
                const unsigned pxc = in ? unsigned(px) : 0u;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int ci = full ? c0 + j : min(c0 + j, p.cin - 1);
                    const unsigned boff = (unsigned(ci) * planeu + pxc) * 4u;
                    float t = *reinterpret_cast<const float *>(reinterpret_cast<const char *>(xrow) + boff);
                    if (p.in_scale) t *= p.in_scale[size_t(img) * p.cin + ci];
                    xv[m][j] = (in && (full || c0 + j < p.cin)) ? t : 0.f;
                }
            }
        };
        int s = valid_from(kpart);
        if (s < steps) load(s, a, al, v);
        while (s < steps) {
            // The next step's loads go out before this step's matrix work.
            const int sn = valid_from(s + p.ksplit);
            half8 na[NT], nal[NT];
            float nv[MT][8];
            if (sn < steps) load(sn, na, nal, nv);
#pragma unroll
            for (int m = 0; m < MT; m++) {
                half8 hi, lo;
                split8(v[m], hi, lo);
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi, a[t], acc[m][t], 0, 0, 0);
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(lo, a[t], acc[m][t], 0, 0, 0);
                    if constexpr (LO) acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi, al[t], acc[m][t], 0, 0, 0);
                }
            }
            if (sn >= steps) break;
            s = sn;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                a[t] = na[t];
                if constexpr (LO) al[t] = nal[t];
            }
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
                for (int j = 0; j < 8; j++) v[m][j] = nv[m][j];
        }
    }
    if (p.ksplit > 1) {
        // Every wavefront reaches this barrier (also those without a tile).
        constexpr int NV = MT * NT * 4;
        if (kpart != 0) {
            float *mine = s_red + size_t(wave) * NV * 64 + lane;
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
                for (int t = 0; t < NT; t++)
#pragma unroll
                    for (int k = 0; k < 4; k++) mine[((m * NT + t) * 4 + k) * 64] = acc[m][t][k];
        }
        __syncthreads();
        if (kpart != 0) return;
        for (int q = 1; q < p.ksplit; q++) {
            const float *o = s_red + size_t(wave + q) * NV * 64 + lane;
#pragma unroll
            for (int m = 0; m < MT; m++)
#pragma unroll
                for (int t = 0; t < NT; t++)
#pragma unroll
                    for (int k = 0; k < 4; k++) acc[m][t][k] += o[((m * NT + t) * 4 + k) * 64];
        }
    }
    if (!live) return;
    // Lane (r, g) holds pixels 16m + 4g .. 16m + 4g + 3 of its tile for output channel 16t + r:
    // one 16-byte store where the four are whole and aligned.
    const int olim = p.flat ? p.oh * p.ow : p.ow;
    const size_t oplane = size_t(p.oh) * p.ow;
    const bool vec = (p.flat ? (oplane & 3) == 0 : (p.ow & 3) == 0) && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0 &&
                     (!p.res || (reinterpret_cast<uintptr_t>(p.res) & 15) == 0);
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int co = nb * p.bn + 16 * t + r;
        if (co >= p.cout) continue;
        const float b = p.bias ? p.bias[co] : 0.f;
        const float as = p.affine ? p.affine[co] : 1.f, at = p.affine ? p.affine[p.cout + co] : 0.f;
        const size_t o0 = (size_t(img) * p.cout + co) * oplane + (p.flat ? 0 : size_t(oy) * p.ow);
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const int px = x0 + 16 * m + 4 * g;
            if (px >= olim) continue;
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float u = acc[m][t][k] + b;
                if (p.affine) u = u * as + at;
                v[k] = act_dev(u, p.act);
            }
            float *dst = p.y + o0 + px;
            if (vec && px + 4 <= olim) {
                if (p.res) {
                    const float4 q = *reinterpret_cast<const float4 *>(p.res + o0 + px);
                    v[0] += q.x, v[1] += q.y, v[2] += q.z, v[3] += q.w;
                }
                *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (px + k < olim) dst[k] = v[k] + (p.res ? p.res[o0 + px + k] : 0.f);
            }
        }
    }
}

template <int MT, int NT, int WPB>
void launch_nchw(const NchwParams &p, bool lo, dim3 grid, size_t lds, hipStream_t s) {
    if (lo) hipLaunchKernelGGL((conv_nchw_kernel<MT, NT, true, WPB>), grid, dim3(64 * WPB), lds, s, p);
    else hipLaunchKernelGGL((conv_nchw_kernel<MT, NT, false, WPB>), grid, dim3(64 * WPB), lds, s, p);
}

template <int MT, int WPB = 4>
void launch_nchw_nt(const NchwParams &p, int nt, bool lo, dim3 grid, size_t lds, hipStream_t s) {
    if (nt == 1) launch_nchw<MT, 1, WPB>(p, lo, grid, lds, s);
    else if (nt == 2) launch_nchw<MT, 2, WPB>(p, lo, grid, lds, s);
    else launch_nchw<MT, 4, WPB>(p, lo, grid, lds, s);
}

// ---- conv_dw ---------------------------------------------------------------------------------
struct DwParams {
    const float *x;
    float *y;
    const float *wt, *bias, *affine;  // wt [c][1][k][k]
    int c, h, w, oh, ow, pt, pl, act, quads, tiles_plane;
    int vec;  // ow % 4 == 0 and y 16-byte aligned: 16-byte stores
};

// A thread makes four neighbouring outputs of one row: each input row segment is read once for
// the four (the taps of one output still summed in the general kernel's order).
template <int K, int SH, int SW>
__global__ __launch_bounds__(256) void conv_dw_kernel(DwParams p) {
    constexpr int SEG = 3 * SW + K;  // input columns under four outputs
    const int plane = blockIdx.x / p.tiles_plane;
    const int item = (blockIdx.x - plane * p.tiles_plane) * 256 + threadIdx.x;
    if (item >= p.oh * p.quads) return;
    const int ch = plane % p.c;
    const int oy = item / p.quads, ox0 = (item - oy * p.quads) * 4;
    const float *xp = p.x + size_t(plane) * p.h * p.w;
    const float *wp = p.wt + size_t(ch) * K * K;
    float wk[K * K];
#pragma unroll
    for (int k = 0; k < K * K; k++) wk[k] = wp[k];
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    const int ix0 = ox0 * SW - p.pl;
#pragma unroll
    for (int ky = 0; ky < K; ky++) {
        const int iy = oy * SH - p.pt + ky;
        if (iy < 0 || iy >= p.h) continue;
        const float *row = xp + size_t(iy) * p.w;
        float seg[SEG];
#pragma unroll
        for (int j = 0; j < SEG; j++) {
            const int ix = ix0 + j;
            seg[j] = (ix >= 0 && ix < p.w) ? row[ix] : 0.f;
        }
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int kx = 0; kx < K; kx++) {
                const int ix = ix0 + q * SW + kx;
                if (ix >= 0 && ix < p.w) acc[q] = __fmaf_rn(seg[q * SW + kx], wk[ky * K + kx], acc[q]);
            }
    }
    const float b = p.bias ? p.bias[ch] : 0.f;
    float *yr = p.y + size_t(plane) * p.oh * p.ow + size_t(oy) * p.ow;
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        v[q] = acc[q] + b;
        if (p.affine) v[q] = v[q] * p.affine[ch] + p.affine[p.c + ch];
        v[q] = act_dev(v[q], p.act);
    }
    if (p.vec && ox0 + 4 <= p.ow) {
        *reinterpret_cast<float4 *>(yr + ox0) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (ox0 + q < p.ow) yr[ox0 + q] = v[q];
    }
}

template <int K>
bool launch_dw(const DwParams &p, int sh, int sw, dim3 grid, hipStream_t s) {
    if (sh == 1 && sw == 1) hipLaunchKernelGGL((conv_dw_kernel<K, 1, 1>), grid, dim3(256), 0, s, p);
    else if (sh == 2 && sw == 2) hipLaunchKernelGGL((conv_dw_kernel<K, 2, 2>), grid, dim3(256), 0, s, p);
    else if (sh == 2 && sw == 1) hipLaunchKernelGGL((conv_dw_kernel<K, 2, 1>), grid, dim3(256), 0, s, p);
    else if (sh == 1 && sw == 2) hipLaunchKernelGGL((conv_dw_kernel<K, 1, 2>), grid, dim3(256), 0, s, p);
    else return false;
    return true;
}

// ---- conv_small ------------------------------------------------------------------------------
struct SmallParams {
    const float *x;
    float *y;
    const float *wt, *bias, *affine, *res, *in_scale;  // wt [cout][cin][kh][kw]
    int n, h, w, cout, oh, ow, sh, sw, pt, pl, act;
};

// blockIdx.y picks 16 output channels; a thread keeps 8 accumulators at a time (8 independent
// chains, the weights of 8 channels read from LDS as two 16-byte reads a tap).
template <int CIN, int KH, int KW>
__global__ __launch_bounds__(256) void conv_small_kernel(SmallParams p) {
    constexpr int T = CIN * KH * KW;
    __shared__ __align__(16) float s_w[T][16];  // this block's channels, [tap][channel]
    const int cb = blockIdx.y * 16;
    for (int i = threadIdx.x; i < T * 16; i += 256) {
        const int t = i / 16, c = i % 16;
        s_w[t][c] = cb + c < p.cout ? p.wt[size_t(cb + c) * T + t] : 0.f;
    }
    __syncthreads();
    const size_t opl = size_t(p.oh) * p.ow;
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= size_t(p.n) * opl) return;
    const int img = int(i / opl);
    const int rem = int(i - size_t(img) * opl);
    const int oy = rem / p.ow, ox = rem - oy * p.ow;
    float xv[T];
    bool ok[T];
#pragma unroll
    for (int c = 0; c < CIN; c++) {
        const float *xc = p.x + (size_t(img) * CIN + c) * p.h * p.w;
        const float sc = p.in_scale ? p.in_scale[size_t(img) * CIN + c] : 1.f;
#pragma unroll
        for (int ky = 0; ky < KH; ky++) {
            const int iy = oy * p.sh - p.pt + ky;
#pragma unroll
            for (int kx = 0; kx < KW; kx++) {
                const int ix = ox * p.sw - p.pl + kx;
                const int t = (c * KH + ky) * KW + kx;
                ok[t] = iy >= 0 && iy < p.h && ix >= 0 && ix < p.w;
                float v = ok[t] ? xc[size_t(iy) * p.w + ix] : 0.f;
                if (p.in_scale) v *= sc;
                xv[t] = v;
            }
        }
    }
#pragma unroll
    for (int half = 0; half < 2; half++) {
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < T; t++) {
            const float4 w0 = *reinterpret_cast<const float4 *>(&s_w[t][8 * half]);
            const float4 w1 = *reinterpret_cast<const float4 *>(&s_w[t][8 * half + 4]);
            const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
            if (ok[t]) {
#pragma unroll
                for (int j = 0; j < 8; j++) acc[j] = __fmaf_rn(xv[t], wv[j], acc[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int co = cb + 8 * half + j;
            if (co >= p.cout) break;
            float v = acc[j] + (p.bias ? p.bias[co] : 0.f);
            if (p.affine) v = v * p.affine[co] + p.affine[p.cout + co];
            v = act_dev(v, p.act);
            const size_t o = (size_t(img) * p.cout + co) * opl + rem;
            if (p.res) v += p.res[o];
            p.y[o] = v;
        }
    }
}

// ---- gemm_rows -------------------------------------------------------------------------------
struct RowsParams {
    const float *x;  // [m][k]
    const half8 *wt, *wt_lo;  // [nblock][chunk][1][bn][32]
    float *y;        // [m][n]
    const float *bias, *res;
    float2 *amax;    // [m][parts] (value, index bits), or null
    int m, k, n, bn, chunks, nblocks, act;
    int rtiles;      // ceil(m / (16 RT))
    int parts, nb_per_wave;
    int tsplit;      // wavefronts a 64-column block is split between (1, 2 or 4)
    int vec;         // k % 4 == 0 and x 16-byte aligned: 16-byte loads
};

// The B operand of one 16-row tile: rows r0 + r, inputs c0 + 8g .. c0 + 8g + 7, split hi / lo.
__device__ inline void rows_frag(const RowsParams &p, int row, int c0, half8 &hi, half8 &lo) {
    float v[8];
    if (row < p.m && p.vec && c0 + 8 <= p.k) {
        const float4 *src = reinterpret_cast<const float4 *>(p.x + size_t(row) * p.k + c0);
        const float4 q0 = src[0], q1 = src[1];
        v[0] = q0.x, v[1] = q0.y, v[2] = q0.z, v[3] = q0.w, v[4] = q1.x, v[5] = q1.y, v[6] = q1.z, v[7] = q1.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = (row < p.m && c0 + j < p.k) ? p.x[size_t(row) * p.k + c0 + j] : 0.f;
    }
    split8(v, hi, lo);
}

// A wavefront: RT 16-row tiles by NT 16-column tiles (part `tpart` of its 64-column block). The
// operands of KC input chunks are read at once, then the matrix work of those chunks.
template <int RT, int NT, int KC, bool LO>
__global__ __launch_bounds__(256) void gemm_rows_kernel(RowsParams p) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wid = blockIdx.x * 4 + wave, nb = blockIdx.y;
    const int rt = wid / p.tsplit, tpart = wid - rt * p.tsplit;
    if (rt >= p.rtiles) return;
    const int r = lane & 15, g = lane >> 4;
    const int r0 = rt * 16 * RT, t0 = tpart * NT;
    floatx4 acc[RT][NT];
#pragma unroll
    for (int m = 0; m < RT; m++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[m][t] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int cg = 0; cg < p.chunks; cg += KC) {
        half8 bh[RT][KC], bl[RT][KC], a[KC][NT], al[KC][NT];
#pragma unroll
        for (int c = 0; c < KC; c++) {
            if (cg + c >= p.chunks) break;
            const size_t wo = size_t(nb * p.chunks + cg + c) * (p.bn * 4) + size_t(r) * 4 + g;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                a[c][t] = p.wt[wo + (t0 + t) * 64];
                if constexpr (LO) al[c][t] = p.wt_lo[wo + (t0 + t) * 64];
            }
#pragma unroll
            for (int m = 0; m < RT; m++) rows_frag(p, r0 + 16 * m + r, (cg + c) * 32 + 8 * g, bh[m][c], bl[m][c]);
        }
#pragma unroll
        for (int c = 0; c < KC; c++) {
            if (cg + c >= p.chunks) break;
#pragma unroll
            for (int m = 0; m < RT; m++)
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c][t], bh[m][c], acc[m][t], 0, 0, 0);
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c][t], bl[m][c], acc[m][t], 0, 0, 0);
                    if constexpr (LO)
                        acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[c][t], bh[m][c], acc[m][t], 0, 0, 0);
                }
        }
    }
    // Lane (r, g) holds columns 4g..4g+3 of n-tile t for row 16m + r.
#pragma unroll
    for (int m = 0; m < RT; m++) {
        const int row = r0 + 16 * m + r;
        if (row >= p.m) continue;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int c = nb * p.bn + 16 * (t0 + t) + 4 * g;
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int co = c + k;
                float u = acc[m][t][k] + ((p.bias && co < p.n) ? p.bias[co] : 0.f);
                v[k] = act_dev(u, p.act);
            }
            float *dst = p.y + size_t(row) * p.n + c;
            if ((p.n & 3) == 0 && c + 4 <= p.n) {
                if (p.res) {
                    const float4 q = *reinterpret_cast<const float4 *>(p.res + size_t(row) * p.n + c);
                    v[0] += q.x, v[1] += q.y, v[2] += q.z, v[3] += q.w;
                }
                *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (c + k < p.n) dst[k] = v[k] + (p.res ? p.res[size_t(row) * p.n + c + k] : 0.f);
            }
        }
    }
}

// The head: a wavefront's rows' operands stay in registers (KC chunks at most) while it walks
// its range of column blocks.
template <int RT, int KC, bool LO>
__global__ __launch_bounds__(256) void gemm_rows_amax_kernel(RowsParams p) {
    constexpr int NT = 4;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wid = blockIdx.x * 4 + wave;
    const int rt = wid / p.parts, part = wid - rt * p.parts;
    if (rt >= p.rtiles) return;
    const int r = lane & 15, g = lane >> 4;
    const int r0 = rt * 16 * RT;
    half8 bh[RT][KC], bl[RT][KC];
#pragma unroll
    for (int m = 0; m < RT; m++)
#pragma unroll
        for (int c = 0; c < KC; c++) {
            if (c < p.chunks) {
                rows_frag(p, r0 + 16 * m + r, c * 32 + 8 * g, bh[m][c], bl[m][c]);
            } else {
                bh[m][c] = half8{};
                bl[m][c] = half8{};
            }
        }
    float bv[RT];
    int bi[RT];
#pragma unroll
    for (int m = 0; m < RT; m++) bv[m] = -INFINITY, bi[m] = 0x7fffffff;
    const int nb0 = part * p.nb_per_wave, nb1 = min(p.nblocks, nb0 + p.nb_per_wave);
    for (int nb = nb0; nb < nb1; nb++) {
        floatx4 acc[RT][NT];
#pragma unroll
        for (int m = 0; m < RT; m++)
#pragma unroll
            for (int t = 0; t < NT; t++) acc[m][t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < KC; c++) {
            if (c >= p.chunks) break;
            const size_t wo = size_t(nb * p.chunks + c) * (p.bn * 4) + size_t(r) * 4 + g;
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const half8 a = p.wt[wo + t * 64];
#pragma unroll
                for (int m = 0; m < RT; m++) {
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bh[m][c], acc[m][t], 0, 0, 0);
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl[m][c], acc[m][t], 0, 0, 0);
                }
                if constexpr (LO) {
                    const half8 al = p.wt_lo[wo + t * 64];
#pragma unroll
                    for (int m = 0; m < RT; m++)
                        acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bh[m][c], acc[m][t], 0, 0, 0);
                }
            }
        }
        // This lane's columns rise with t and k: a strict > keeps the first index on ties.
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int co = nb * 64 + 16 * t + 4 * g + k;
                if (co >= p.n) continue;
                const float b = p.bias ? p.bias[co] : 0.f;
#pragma unroll
                for (int m = 0; m < RT; m++) {
                    const float v = acc[m][t][k] + b;
                    if (v > bv[m]) bv[m] = v, bi[m] = co;
                }
            }
    }
#pragma unroll
    for (int m = 0; m < RT; m++) {
        float v = bv[m];
        int i = bi[m];
        for (int off = 16; off < 64; off <<= 1) {
            const float ov = __shfl_xor(v, off);
            const int oi = __shfl_xor(i, off);
            if (ov > v || (ov == v && oi < i)) v = ov, i = oi;
        }
        const int row = r0 + 16 * m + r;
        if (g == 0 && row < p.m) p.amax[size_t(row) * p.parts + part] = make_float2(v, __int_as_float(i));
    }
}

}  // namespace

bool nd_conv_nchw_mfma(const NdMfmaConvArgs &a, hipStream_t s) {
    const ConvPack &pk = a.pk;
    if (pk.kh > 3 || pk.kw > 3 || pk.cin != a.cin || pk.cout != a.cout || !a.wt_hi) return false;
    if (!pk.exact && !a.wt_lo) return false;
    if (pk.bn != 16 && pk.bn != 32 && pk.bn != 64) return false;
    NchwParams p{};
    p.x = a.x;
    p.y = a.y;
    p.wt = reinterpret_cast<const half8 *>(a.wt_hi);
    p.wt_lo = reinterpret_cast<const half8 *>(a.wt_lo);
    p.bias = a.bias;
    p.affine = a.affine;
    p.res = a.res;
    p.in_scale = a.in_scale;
    p.n = a.n;
    p.cin = a.cin;
    p.h = a.h;
    p.w = a.w;
    p.cout = a.cout;
    p.oh = a.oh;
    p.ow = a.ow;
    p.bn = pk.bn;
    p.chunks = pk.chunks;
    p.kh = pk.kh;
    p.kw = pk.kw;
    p.pt = a.pt;
    p.pl = a.pl;
    p.act = a.act;
    // Stride 1: the output is the input size plus the pads less the kernel, checked by the caller.
    p.flat = (pk.kh == 1 && pk.kw == 1 && a.pt == 0 && a.pl == 0 && a.oh == a.h && a.ow == a.w) ? 1 : 0;
    if (double(a.cin) * a.h * a.w >= 1073741824.0) return false;  // 32-bit byte offsets within an image
    const double lim = p.flat ? double(a.h) * a.w : double(a.ow);
    const double lines = p.flat ? double(a.n) : double(a.n) * a.oh;
    if (lim > 0x7fffffff || lines > 0x7fffffff) return false;
    // Pixels a wavefront: the widest of 64 / 32 / 16 that wastes at most a quarter of its tiles
    // and still gives 8192 wavefronts (32 a CU, so that other wavefronts' loads cover each one's
    // load latency: the PP-OCR recogniser's convs take 1.12 ms a batch at this target, 1.18 at
    // 2048, 1.12 at 32768); else 16.
    const int nt = pk.bn / 16;
    auto tiles_of = [&](int m) { return lines * std::ceil(lim / (16.0 * m)); };
    int mt = 1;
    for (int cand : {4, 2}) {
        const double tl = std::ceil(lim / (16.0 * cand));
        if ((tl * 16 * cand - lim) * 4 <= lim && tiles_of(cand) * pk.nblocks >= 8192) { mt = cand; break; }
    }
    const int steps = pk.chunks * (p.flat ? 1 : std::min(pk.kh, a.h) * pk.kw);
    const double waves = tiles_of(mt) * pk.nblocks;
    // K split across a workgroup's wavefronts when the launch has few tiles: each wavefront walks
    // every ks-th K step, and the partial sums meet in LDS in a fixed order. A launch of under
    // 1024 wavefronts with 16 or more K steps (the SVTR neck's 3 x 3 convs over one-row tensors,
    // 90 steps, and its 1 x 1 convs) takes 16-wavefront workgroups and 8 or 16 parts (not for four
    // n-tiles of inexact weights, whose operands do not fit 128 VGPRs): the PP-OCR recogniser's
    // batch 1.12 -> 1.08 ms; with at most 4 parts the neck's 3 x 3 convs took 14-23 us each on a
    // few hundred wavefronts, each walking 22 dependent steps. 8 steps as the bar measured 1.10 ms.
    int ks = 1, wpb = 4;
    if (waves < 1024 && steps >= 16 && (nt <= 2 || pk.exact)) ks = waves < 512 ? 16 : 8, wpb = 16, mt = 1;
    else if (waves < 1024 && steps >= 8) ks = 4;
    else if (waves < 2048 && steps >= 4) ks = 2;
    if (ks > 1 && mt * nt > 8) mt = std::max(1, 8 / nt);
    p.tiles_line = int(std::ceil(lim / (16.0 * mt)));
    if (tiles_of(mt) > 0x3fffffff) return false;
    p.tiles = int(tiles_of(mt));
    p.ksplit = ks;
    const size_t lds = ks > 1 ? size_t(wpb) * mt * nt * 4 * 64 * sizeof(float) : 0;
    const int per_block = wpb / ks;
    dim3 grid(unsigned((p.tiles + per_block - 1) / per_block), unsigned(pk.nblocks));
    if (pk.nblocks > 65535) return false;
    const double flops = 2.0 * a.n * a.oh * a.ow * a.cout * a.cin * pk.kh * pk.kw;
    const double bytes = 4.0 * (double(a.n) * a.h * a.w * a.cin + double(a.n) * a.oh * a.ow * a.cout) +
                         2.0 * double(pk.halves()) * (pk.exact ? 1 : 2);
    ProbeScope probe("nd_conv_nchw", s, flops, bytes);
    const bool lo = !pk.exact;
    if (wpb == 16) launch_nchw_nt<1, 16>(p, nt, lo, grid, lds, s);
    else if (mt == 4) launch_nchw_nt<4>(p, nt, lo, grid, lds, s);
    else if (mt == 2) launch_nchw_nt<2>(p, nt, lo, grid, lds, s);
    else launch_nchw_nt<1>(p, nt, lo, grid, lds, s);
    OCR_HIP(hipGetLastError());
    return true;
}

bool nd_conv_dw(const NdConvArgs &a, hipStream_t s) {
    if (a.group != a.cin || a.cout != a.cin || a.kh != a.kw || (a.kh != 3 && a.kh != 5)) return false;
    if (a.res || a.in_scale) return false;
    const size_t opl = size_t(a.oh) * a.ow, planes = size_t(a.n) * a.cin;
    if (opl == 0 || planes == 0) return true;
    if (opl > 0x7fffffff) return false;
    DwParams p{};
    p.x = a.x;
    p.y = a.y;
    p.wt = a.wt;
    p.bias = a.b;
    p.affine = a.affine;
    p.c = a.cin;
    p.h = a.h;
    p.w = a.w;
    p.oh = a.oh;
    p.ow = a.ow;
    p.pt = a.pt;
    p.pl = a.pl;
    p.act = a.act;
    p.quads = (a.ow + 3) / 4;
    p.vec = (a.ow % 4 == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0) ? 1 : 0;
    p.tiles_plane = int((size_t(a.oh) * p.quads + 255) / 256);
    const double blocks = double(p.tiles_plane) * planes;
    if (blocks > 0x7fffffff) return false;
    const dim3 grid{unsigned(blocks)};
    ProbeScope probe("nd_conv_dw", s, 2.0 * double(planes) * opl * a.kh * a.kw,
                     4.0 * (double(planes) * a.h * a.w + double(planes) * opl));
    const bool ok = a.kh == 3 ? launch_dw<3>(p, a.sh, a.sw, grid, s) : launch_dw<5>(p, a.sh, a.sw, grid, s);
    if (ok) OCR_HIP(hipGetLastError());
    return ok;
}

bool nd_conv_small(const NdConvArgs &a, hipStream_t s) {
    if (a.group != 1 || a.cout > 64 || a.cout < 1) return false;
    const bool k3 = a.kh == 3 && a.kw == 3;
    if (!k3 || (a.cin != 1 && a.cin != 3)) return false;
    const size_t total = size_t(a.n) * a.oh * a.ow;
    if (total == 0) return true;
    if (total / 256 + 1 > 0x7fffffff) return false;
    SmallParams p{};
    p.x = a.x;
    p.y = a.y;
    p.wt = a.wt;
    p.bias = a.b;
    p.affine = a.affine;
    p.res = a.res;
    p.in_scale = a.in_scale;
    p.n = a.n;
    p.h = a.h;
    p.w = a.w;
    p.cout = a.cout;
    p.oh = a.oh;
    p.ow = a.ow;
    p.sh = a.sh;
    p.sw = a.sw;
    p.pt = a.pt;
    p.pl = a.pl;
    p.act = a.act;
    const dim3 grid{unsigned((total + 255) / 256), unsigned((a.cout + 15) / 16)};
    ProbeScope probe("nd_conv_small", s, 2.0 * double(total) * a.cout * a.cin * 9,
                     4.0 * (double(a.n) * a.cin * a.h * a.w + double(total) * a.cout));
    if (a.cin == 3) hipLaunchKernelGGL((conv_small_kernel<3, 3, 3>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((conv_small_kernel<1, 3, 3>), grid, dim3(256), 0, s, p);
    OCR_HIP(hipGetLastError());
    return true;
}

namespace {

RowsParams rows_params(const NdRowsArgs &a) {
    RowsParams p{};
    p.x = a.x;
    p.wt = reinterpret_cast<const half8 *>(a.wt_hi);
    p.wt_lo = reinterpret_cast<const half8 *>(a.wt_lo);
    p.y = a.y;
    p.bias = a.bias;
    p.res = a.res;
    p.m = a.m;
    p.k = a.k;
    p.n = a.n;
    p.bn = a.pk.bn;
    p.chunks = a.pk.chunks;
    p.nblocks = a.pk.nblocks;
    p.act = a.act;
    p.vec = (a.k % 4 == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0) ? 1 : 0;
    return p;
}

}  // namespace

bool nd_gemm_rows(const NdRowsArgs &a, hipStream_t s) {
    const ConvPack &pk = a.pk;
    if (pk.kh != 1 || pk.kw != 1 || pk.cin != a.k || pk.cout != a.n || !a.wt_hi) return false;
    if (!pk.exact && !a.wt_lo) return false;
    if (pk.bn != 16 && pk.bn != 32 && pk.bn != 64) return false;
    if (a.m <= 0) return true;
    if (pk.nblocks > 65535) return false;
    RowsParams p = rows_params(a);
    // 32 rows a wavefront, then 16, then a part of the column block, until there are 2048
    // wavefronts (8 a CU) or no smaller split.
    const int ntf = pk.bn / 16;
    auto waves = [&](int rt, int ts) { return double((a.m + 16 * rt - 1) / (16 * rt)) * ts * pk.nblocks; };
    int rt = 2, ts = 1;
    if (waves(rt, ts) < 2048) rt = 1;
    while (waves(rt, ts) < 2048 && ts < ntf) ts *= 2;
    const int nt = ntf / ts;
    p.rtiles = (a.m + 16 * rt - 1) / (16 * rt);
    p.tsplit = ts;
    const double blocks = std::ceil(double(p.rtiles) * ts / 4);
    if (blocks > 0x7fffffff) return false;
    const dim3 grid{unsigned(blocks), unsigned(pk.nblocks)};
    ProbeScope probe("nd_gemm_rows", s, 2.0 * a.m * double(a.k) * a.n,
                     4.0 * (double(a.m) * a.k + double(a.m) * a.n) + 2.0 * double(pk.halves()) * (pk.exact ? 1 : 2));
    const bool lo = !pk.exact, k8 = pk.chunks > 4;
#define ROWS_LAUNCH(RT, NT)                                                                          \
    do {                                                                                             \
        if (lo && k8) hipLaunchKernelGGL((gemm_rows_kernel<RT, NT, 8, true>), grid, dim3(256), 0, s, p);   \
        else if (lo) hipLaunchKernelGGL((gemm_rows_kernel<RT, NT, 4, true>), grid, dim3(256), 0, s, p);    \
        else if (k8) hipLaunchKernelGGL((gemm_rows_kernel<RT, NT, 8, false>), grid, dim3(256), 0, s, p);   \
        else hipLaunchKernelGGL((gemm_rows_kernel<RT, NT, 4, false>), grid, dim3(256), 0, s, p);           \
    } while (0)
    if (rt == 2) {
        if (nt == 1) ROWS_LAUNCH(2, 1);
        else if (nt == 2) ROWS_LAUNCH(2, 2);
        else ROWS_LAUNCH(2, 4);
    } else {
        if (nt == 1) ROWS_LAUNCH(1, 1);
        else if (nt == 2) ROWS_LAUNCH(1, 2);
        else ROWS_LAUNCH(1, 4);
    }
#undef ROWS_LAUNCH
    OCR_HIP(hipGetLastError());
    return true;
}

int nd_head_parts(int m, const ConvPack &pk) {
    const int rtiles = (m + 31) / 32;
    int per = std::max(1, (pk.nblocks * rtiles + 3071) / 3072);
    return (pk.nblocks + per - 1) / per;
}

bool nd_head_argmax(const NdRowsArgs &a, float *part, int parts, hipStream_t s) {
    const ConvPack &pk = a.pk;
    if (pk.kh != 1 || pk.kw != 1 || pk.cin != a.k || pk.cout != a.n || pk.bn != 64 || !a.wt_hi) return false;
    if (!pk.exact && !a.wt_lo) return false;
    if (pk.chunks > 8 || a.res || a.act != ACT_NONE) return false;
    if (a.m <= 0) return true;
    RowsParams p = rows_params(a);
    p.amax = reinterpret_cast<float2 *>(part);
    p.rtiles = (a.m + 31) / 32;
    p.nb_per_wave = (pk.nblocks + parts - 1) / parts;
    p.parts = parts;
    if (nd_head_parts(a.m, pk) != parts) fail("nd_head_argmax: partial count differs from nd_head_parts");
    const double waves = double(p.rtiles) * parts;
    if (waves / 4 + 1 > 0x7fffffff) return false;
    const dim3 grid{unsigned((waves + 3) / 4)};
    ProbeScope probe("nd_head", s, 2.0 * a.m * double(a.k) * a.n,
                     4.0 * double(a.m) * a.k + 2.0 * double(pk.halves()) * (pk.exact ? 1 : 2) + 8.0 * double(a.m) * parts);
    const bool lo = !pk.exact;
    if (pk.chunks <= 4) {
        if (lo) hipLaunchKernelGGL((gemm_rows_amax_kernel<2, 4, true>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((gemm_rows_amax_kernel<2, 4, false>), grid, dim3(256), 0, s, p);
    } else {
        if (lo) hipLaunchKernelGGL((gemm_rows_amax_kernel<2, 8, true>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((gemm_rows_amax_kernel<2, 8, false>), grid, dim3(256), 0, s, p);
    }
    OCR_HIP(hipGetLastError());
    return true;
}

}  // namespace ocr
