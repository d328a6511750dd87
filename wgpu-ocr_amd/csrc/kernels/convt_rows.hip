// ConvTranspose (the U-Net's upsamplers, src/gpu.rs:424-460) in NHWC as one GEMM on the gfx950
// matrix cores (v_mfma_f32_16x16x32_f16) over the positions (i, j) of the output's s x s blocks:
// output column k cout + c of position (i, j) is channel c of y's pixel (s i + k / s, s j + k % s),
// written when that pixel lies inside y. The K dimension walks input channels x taps: tap (a, b)
// of the ty x tx window reads input pixel (i - (ty - 1 - a), j - (tx - 1 - b)), zero outside the
// input, against the weight of ky = k / s + s (ty - 1 - a), kx = k % s + s (tx - 1 - b) (packed
// by the caller, zero past the kernel). A kernel equal to the stride has one tap and the
// positions are the input pixels; the detector's 2 x 3 upsampler at stride 2 has a 1 x 2 window.
// No LDS: a wavefront loads its own operands, the packed float16 weights as the A operand (one
// 16-byte read a lane) and 16 positions' input channels as the B operand (two 16-byte reads a
// lane), split into float16 hi + lo (x = hi + lo to about 2^-22) and both multiplied,
// accumulating in float32 (float32-class results). A lane's four accumulators are four
// neighbouring channels of one output pixel: one 16-byte store. A wavefront owns 16 RT positions
// x 16 NT output columns and walks the input channels one 32-channel chunk (and tap) at a time:
// the kernel is one pass over its operands, bound by loads in flight across wavefronts, so
// registers go to occupancy (5 wavefronts a SIMD at RT = 2, NT = 4; 2 with four chunks' operands
// held at once, 28 % slower over the detector's upsamplers).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "../kernels.h"
#include "../runtime.h"

namespace ocr {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

struct CtParams {
    const float *x;
    long xcs;
    int npx, ghw, gw, h, w, cin;  // positions (n gh gw), gh gw, gw; input h, w, channels
    int ty, tx, taps;             // tap window (ty x tx)
    const half8 *wt, *wt_lo;      // [nblock][chunk][tap][bn][32]: cin -> s s cout
    int bn, chunks;
    float *y;
    long ycs;
    int oh, ow, cout, s, ncol;  // ncol = s s cout
    const float *bias;
    int act;
    int rtiles, tsplit, vecx, vecy;
};

__device__ inline float ct_act(float v, int act) {
    if (act == ACT_RELU) return fmaxf(v, 0.f);
    if (act == ACT_SIGMOID) return 1.f / (1.f + expf(-v));
    return v;
}

template <int RT, int NT, bool LO>
__global__ __launch_bounds__(256) void convt_rows_kernel(CtParams p) {
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
    // This lane's position in each row tile: image, block row and column (-1: past the end).
    int pimg[RT], pi[RT], pj[RT];
#pragma unroll
    for (int m = 0; m < RT; m++) {
        const int q = r0 + 16 * m + r;
        pimg[m] = q < p.npx ? q / p.ghw : -1;
        const int rem = q - (q < p.npx ? pimg[m] : 0) * p.ghw;
        pi[m] = rem / p.gw;
        pj[m] = rem - pi[m] * p.gw;
    }
    for (int k = 0; k < p.chunks * p.taps; k++) {
        const int c = k / p.taps, tap = k - c * p.taps;
        const int da = p.ty - 1 - tap / p.tx, db = p.tx - 1 - (tap - (tap / p.tx) * p.tx);
        half8 bh[RT], bl[RT], a[NT], al[NT];
        const size_t wo = (size_t(nb * p.chunks + c) * p.taps + tap) * (p.bn * 4) + size_t(r) * 4 + g;
#pragma unroll
        for (int t = 0; t < NT; t++) {
            a[t] = p.wt[wo + (t0 + t) * 64];
            if constexpr (LO) al[t] = p.wt_lo[wo + (t0 + t) * 64];
        }
        const int c0 = c * 32 + 8 * g;
#pragma unroll
        for (int m = 0; m < RT; m++) {
            const int iy = pi[m] - da, ix = pj[m] - db;
            const bool in = pimg[m] >= 0 && unsigned(iy) < unsigned(p.h) && unsigned(ix) < unsigned(p.w);
            const size_t px = in ? (size_t(pimg[m]) * p.h + iy) * p.w + ix : 0;
            float v[8];
            if (in && p.vecx && c0 + 8 <= p.cin) {
                const float4 *src = reinterpret_cast<const float4 *>(p.x + px * p.xcs + c0);
                const float4 q0 = src[0], q1 = src[1];
                v[0] = q0.x, v[1] = q0.y, v[2] = q0.z, v[3] = q0.w, v[4] = q1.x, v[5] = q1.y, v[6] = q1.z, v[7] = q1.w;
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = (in && c0 + j < p.cin) ? p.x[px * p.xcs + c0 + j] : 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const _Float16 hv = (_Float16)v[j];
                bh[m][j] = hv;
                bl[m][j] = (_Float16)(v[j] - (float)hv);
            }
        }
#pragma unroll
        for (int m = 0; m < RT; m++)
#pragma unroll
            for (int t = 0; t < NT; t++) {
                acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], bh[m], acc[m][t], 0, 0, 0);
                acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], bl[m], acc[m][t], 0, 0, 0);
                if constexpr (LO) acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[t], bh[m], acc[m][t], 0, 0, 0);
            }
    }
    // Lane (r, g) holds columns 4g..4g+3 of n-tile t for position 16m + r.
#pragma unroll
    for (int m = 0; m < RT; m++) {
        if (pimg[m] < 0) continue;
        const int img = pimg[m], iy = pi[m], ix = pj[m];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int col0 = nb * p.bn + 16 * (t0 + t) + 4 * g;
            if (col0 >= p.ncol) continue;
            if (p.vecy) {
                // cout % 4 == 0: the four columns are neighbouring channels of one phase.
                const int ph = col0 / p.cout, c = col0 - ph * p.cout;
                const int oy = p.s * iy + ph / p.s, ox = p.s * ix + ph % p.s;
                if (oy >= p.oh || ox >= p.ow) continue;
                float4 o;
                o.x = ct_act(acc[m][t][0] + p.bias[c], p.act);
                o.y = ct_act(acc[m][t][1] + p.bias[c + 1], p.act);
                o.z = ct_act(acc[m][t][2] + p.bias[c + 2], p.act);
                o.w = ct_act(acc[m][t][3] + p.bias[c + 3], p.act);
                *reinterpret_cast<float4 *>(p.y + ((size_t(img) * p.oh + oy) * p.ow + ox) * p.ycs + c) = o;
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int col = col0 + k;
                    if (col >= p.ncol) break;
                    const int ph = col / p.cout, c = col - ph * p.cout;
                    const int oy = p.s * iy + ph / p.s, ox = p.s * ix + ph % p.s;
                    if (oy < p.oh && ox < p.ow)
                        p.y[((size_t(img) * p.oh + oy) * p.ow + ox) * p.ycs + c] = ct_act(acc[m][t][k] + p.bias[c], p.act);
                }
            }
        }
    }
}

}  // namespace

bool convt_rows(const Act &x, const Act &y, const uint16_t *whi, const uint16_t *wlo, const ConvPack &pk,
                const float *b, int stride, int act, hipStream_t st) {
    if (stride < 1 || stride > 4 || !whi || !b || (!pk.exact && !wlo)) return false;
    // The tap window: ceil(kernel / stride) a side, at most 3 (packed by the caller).
    if (pk.kh < 1 || pk.kw < 1 || pk.kh > 3 || pk.kw > 3) return false;
    if (pk.cin != x.c || pk.cout != stride * stride * y.c) return false;
    if (pk.bn != 16 && pk.bn != 32 && pk.bn != 64) return false;
    if (act != ACT_NONE && act != ACT_RELU && act != ACT_SIGMOID) return false;
    const int gh = (y.h + stride - 1) / stride, gw = (y.w + stride - 1) / stride;
    if (x.n != y.n || y.h < 1 || y.w < 1 || x.h < 1 || x.w < 1) return false;
    // Every position reads inside or just past the input (the window's leading pads).
    if (gh > x.h + pk.kh - 1 || gw > x.w + pk.kw - 1) return false;
    const double npx = double(x.n) * gh * gw;
    if (npx >= 2147483647.0 - 64 || pk.nblocks > 65535 || double(y.n) * y.h * y.w * y.cs >= 9.0e18) return false;
    CtParams p{};
    p.x = x.p;
    p.xcs = x.cs;
    p.npx = int(npx);
    p.ghw = gh * gw;
    p.gw = gw;
    p.h = x.h;
    p.w = x.w;
    p.cin = x.c;
    p.ty = pk.kh;
    p.tx = pk.kw;
    p.taps = pk.kh * pk.kw;
    p.wt = reinterpret_cast<const half8 *>(whi);
    p.wt_lo = reinterpret_cast<const half8 *>(wlo);
    p.bn = pk.bn;
    p.chunks = pk.chunks;
    p.y = y.p;
    p.ycs = y.cs;
    p.oh = y.h;
    p.ow = y.w;
    p.cout = y.c;
    p.s = stride;
    p.ncol = pk.cout;
    p.bias = b;
    p.act = act;
    p.vecx = (x.c % 4 == 0 && x.cs % 4 == 0 && (reinterpret_cast<uintptr_t>(x.p) & 15) == 0) ? 1 : 0;
    p.vecy = (y.c % 4 == 0 && y.cs % 4 == 0 && (reinterpret_cast<uintptr_t>(y.p) & 15) == 0) ? 1 : 0;
    if (p.npx == 0) return true;
    // 32 positions a wavefront, then 16, then a part of the column block, until there are 2048
    // wavefronts (8 a CU) or no smaller split.
    const int ntf = pk.bn / 16;
    auto waves = [&](int rt, int ts) { return std::ceil(npx / (16.0 * rt)) * ts * pk.nblocks; };
    int rt = 2, ts = 1;
    if (waves(rt, ts) < 2048) rt = 1;
    while (waves(rt, ts) < 2048 && ts < ntf) ts *= 2;
    const int nt = ntf / ts;
    p.rtiles = int((npx + 16 * rt - 1) / (16 * rt));
    p.tsplit = ts;
    const double blocks = std::ceil(double(p.rtiles) * ts / 4);
    if (blocks > 2147483647.0) return false;
    const dim3 grid{unsigned(blocks), unsigned(pk.nblocks)};
    ProbeScope probe("conv_transpose", st, 2.0 * npx * p.taps * double(x.c) * pk.cout,
                     4.0 * (double(x.n) * x.h * x.w * x.c + double(y.n) * y.h * y.w * y.c) +
                         2.0 * double(pk.halves()) * (pk.exact ? 1 : 2));
    const bool lo = !pk.exact;
#define CT_LAUNCH(RT, NT)                                                                        \
    do {                                                                                         \
        if (lo) hipLaunchKernelGGL((convt_rows_kernel<RT, NT, true>), grid, dim3(256), 0, st, p); \
        else hipLaunchKernelGGL((convt_rows_kernel<RT, NT, false>), grid, dim3(256), 0, st, p);   \
    } while (0)
    if (rt == 2) {
        if (nt == 1) CT_LAUNCH(2, 1);
        else if (nt == 2) CT_LAUNCH(2, 2);
        else CT_LAUNCH(2, 4);
    } else {
        if (nt == 1) CT_LAUNCH(1, 1);
        else if (nt == 2) CT_LAUNCH(1, 2);
        else CT_LAUNCH(1, 4);
    }
#undef CT_LAUNCH
    OCR_HIP(hipGetLastError());
    return true;
}

}  // namespace ocr
