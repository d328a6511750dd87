// Multi-head self-attention of the N-D executor in one launch: the exporter's chain from the
// fused QKV projection (reshape, transpose, slice q / k / v, scale q, q k^T, softmax over the last
// axis, times v, transpose, reshape; src/nd.rs:291-391 runs it as separate programs) on gfx950.
//
// x is [n][T][3 H d] (q, then k, then v, each H heads of d values), y is [n][T][H d]. A workgroup
// takes 32 queries of one head of one image; eight lanes share a query, each walking every eighth
// key. Keys and values come through LDS in tiles of KT keys (each row padded with zeros to D
// values). The softmax runs in float32 over each tile twice: the tile's maximum first, then
// exp(s - max) and the value sums, the running sums rescaled when a later tile raises the
// maximum (so any T works; for T <= KT it is the plain max-subtracted softmax). The eight lanes
// combine their sums at the end and divide once.
#include <hip/hip_runtime.h>

#include <cmath>

#include "../nd_kernels.h"
#include "../runtime.h"

namespace ocr {

namespace {

struct AttnParams {
    const float *x;
    float *y;
    int n, t, heads, d;
    float scale;
};

template <int D, int KT>
__global__ __launch_bounds__(256) void attention_kernel(AttnParams p) {
    __shared__ __align__(16) float s_k[KT][D];
    __shared__ __align__(16) float s_v[KT][D];
    const int img = blockIdx.z, h = blockIdx.y;
    const int q = blockIdx.x * 32 + (threadIdx.x >> 3), j8 = threadIdx.x & 7;
    const int hd = p.heads * p.d;
    const size_t row = size_t(3) * hd;
    const float *base = p.x + size_t(img) * p.t * row;
    // Lanes of queries past T compute with zeros and store nothing (the eight lanes of a query
    // stay together for the exchanges).
    float qv[D];
#pragma unroll
    for (int k = 0; k < D; k++)
        qv[k] = (q < p.t && k < p.d) ? base[size_t(q) * row + size_t(h) * p.d + k] * p.scale : 0.f;
    float m = -INFINITY, l = 0.f, o[D];
#pragma unroll
    for (int k = 0; k < D; k++) o[k] = 0.f;
    for (int k0 = 0; k0 < p.t; k0 += KT) {
        const int kt = min(KT, p.t - k0);
        __syncthreads();
        for (int i = threadIdx.x; i < kt * D; i += 256) {
            const int j = i / D, k = i - j * D;
            const float *src = base + size_t(k0 + j) * row + size_t(h) * p.d + k;
            s_k[j][k] = k < p.d ? src[hd] : 0.f;
            s_v[j][k] = k < p.d ? src[2 * hd] : 0.f;
        }
        __syncthreads();
        auto score = [&](int j) {
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < D; k += 4) {
                const float4 kk = *reinterpret_cast<const float4 *>(&s_k[j][k]);
                s = __fmaf_rn(qv[k], kk.x, s);
                s = __fmaf_rn(qv[k + 1], kk.y, s);
                s = __fmaf_rn(qv[k + 2], kk.z, s);
                s = __fmaf_rn(qv[k + 3], kk.w, s);
            }
            return s;
        };
        float mt = -INFINITY;
        for (int j = j8; j < kt; j += 8) mt = fmaxf(mt, score(j));
        for (int off = 1; off < 8; off <<= 1) mt = fmaxf(mt, __shfl_xor(mt, off));
        const float mn = fmaxf(m, mt);
        const float f = m == -INFINITY ? 0.f : expf(m - mn);
        l *= f;
#pragma unroll
        for (int k = 0; k < D; k++) o[k] *= f;
        m = mn;
        for (int j = j8; j < kt; j += 8) {
            const float e = expf(score(j) - m);
            l += e;
#pragma unroll
            for (int k = 0; k < D; k += 4) {
                const float4 vv = *reinterpret_cast<const float4 *>(&s_v[j][k]);
                o[k] = __fmaf_rn(e, vv.x, o[k]);
                o[k + 1] = __fmaf_rn(e, vv.y, o[k + 1]);
                o[k + 2] = __fmaf_rn(e, vv.z, o[k + 2]);
                o[k + 3] = __fmaf_rn(e, vv.w, o[k + 3]);
            }
        }
    }
    for (int off = 1; off < 8; off <<= 1) {
        l += __shfl_xor(l, off);
#pragma unroll
        for (int k = 0; k < D; k++) o[k] += __shfl_xor(o[k], off);
    }
    if (q >= p.t) return;
    float *dst = p.y + (size_t(img) * p.t + q) * hd + size_t(h) * p.d;
#pragma unroll
    for (int k = 0; k < D; k++)
        if (k % 8 == j8 && k < p.d) dst[k] = o[k] / l;
}

}  // namespace

void nd_attention(const float *x, int n, int t, int heads, int d, float scale, float *y, hipStream_t s) {
    if (n <= 0 || t <= 0) return;
    if (d <= 0 || d > 64) fail("nd_attention: " + std::to_string(d) + " values a head (at most 64)");
    AttnParams p{x, y, n, t, heads, d, scale};
    const dim3 grid{unsigned((t + 31) / 32), unsigned(heads), unsigned(n)};
    const double tt = double(t);
    ProbeScope probe("nd_attention", s, 4.0 * n * heads * tt * tt * d, 4.0 * n * tt * (3.0 * heads * d + heads * d));
    if (d <= 16) hipLaunchKernelGGL((attention_kernel<16, 256>), grid, dim3(256), 0, s, p);
    else if (d <= 32) hipLaunchKernelGGL((attention_kernel<32, 256>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((attention_kernel<64, 128>), grid, dim3(256), 0, s, p);
    OCR_HIP(hipGetLastError());
}

}  // namespace ocr
