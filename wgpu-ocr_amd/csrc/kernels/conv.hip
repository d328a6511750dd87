// Dense convolution as an LDS-staged implicit GEMM on the gfx950 matrix cores
// (v_mfma_f32_16x16x32_f16). Semantics of the reference's conv / conv_fast / conv128 programs
// (src/gpu.rs:37-350): M = output pixels, N = output channels, K = taps x input channels,
// epilogue y = act(acc + b[c]) (+ res when given).
//
// Precision: the float32 activations are split on the fly into a float16 "hi" part and the
// float16 remainder "lo" (x = hi + lo to about 2^-22 relative), and both are multiplied with the
// float16 weights, accumulating in float32. When the model's weights are float16 values (exact)
// that is two MFMA passes per product and float32-class accuracy; otherwise the weights' own
// remainder adds a third pass (x_hi * w_lo).
//
// Work split: a workgroup of 4 wavefronts owns a 2-D tile of 128 output pixels (TH x TW) of one
// image and BN output channels. For each slice of 32 input channels it stages the tile's input
// halo ((TH + KS - 1) x (TW + KS - 1) pixels, already split into hi/lo float16) and the slice's
// weights for all taps in LDS, then every tap is one shifted read of the halo: each input value
// is fetched from HBM once per workgroup instead of once per tap. Each wavefront computes 32
// pixels x BN channels with 2 x (BN / 16) accumulator tiles.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "../kernels.h"
#include "../runtime.h"

namespace ocr {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int KSTRIDE = 40;  // halves per LDS row: 32 channels + 8 padding (bank spread)

struct ConvParams {
    const float *x;
    int n, h, w, cin, xcs;
    float *y;
    int oh, ow, cout, ycs;
    const half8 *wt_hi, *wt_lo;
    const float *bias, *res, *affine, *in_scale;
    float2 *amax;  // arg-max partials [pixels][nblocks] instead of y, or null
    const int *rows;  // 1 x 1 GEMM: row i of x and of y is physical row rows[i] (gather/scatter), or null
    float *yp;     // MaxPool (ph, pw) of the activated output (NHWC), or null
    size_t yn, yy, yx;  // NHWC output pixel strides: image, row, column
    int poh, pow_, ypcs, ph, pw;
    int rcs;
    int kh, kw, pt, pl, act, chunks, tiles_x, tiles_y, vec, nchw;
};

__device__ inline float activate_dev(float v, int act) {
    if (act == ACT_RELU) return fmaxf(v, 0.f);
    if (act == ACT_SIGMOID) return 1.f / (1.f + expf(-v));
    if (act == ACT_GELU) return 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    if (act == ACT_SILU) return v / (1.f + expf(-v));
    return v;
}

template <int TW, int KS, int BN, bool LO>
__global__ __launch_bounds__(256) void conv_mfma_kernel(ConvParams p) {
    constexpr int TH = 128 / TW;
    constexpr int HH = TH + KS - 1, HWD = TW + KS - 1, HALO = HH * HWD;
    constexpr int NT = BN / 16;
    __shared__ __align__(16) _Float16 s_hi[HALO][KSTRIDE];
    __shared__ __align__(16) _Float16 s_lo[HALO][KSTRIDE];
    __shared__ __align__(16) _Float16 s_w[KS * KS][BN][KSTRIDE];
    __shared__ __align__(16) _Float16 s_wl[LO ? KS * KS : 1][LO ? BN : 1][KSTRIDE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int bx = blockIdx.x;
    const int tx = bx % p.tiles_x;
    bx /= p.tiles_x;
    const int ty = bx % p.tiles_y;
    const int img = bx / p.tiles_y;
    const int oy0 = ty * TH, ox0 = tx * TW;
    const int iy0 = oy0 - p.pt, ix0 = ox0 - p.pl;
    const int nb = blockIdx.y, co0 = nb * BN;
    const int taps = p.kh * p.kw;
    const float *xim = p.x + size_t(img) * p.h * p.w * p.xcs;

    floatx4 acc[2][NT];
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[m][t] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int g = lane >> 4, r = lane & 15;
    for (int chunk = 0; chunk < p.chunks; chunk++) {
        const int ci0 = chunk * 32;
        // Stage the halo as hi/lo float16, zero outside the image and past cin; the SE gate
        // (in_scale) multiplies the input first.
        if (p.nchw) {
            // NCHW: consecutive threads take consecutive pixels of one channel.
            for (int i = tid; i < HALO * 32; i += 256) {
                const int cl = i / HALO, hp = i - cl * HALO;
                const int hy = hp / HWD, hx = hp - hy * HWD;
                const int iy = iy0 + hy, ix = ix0 + hx, ci = ci0 + cl;
                float v = 0.f;
                if (iy >= 0 && iy < p.h && ix >= 0 && ix < p.w && ci < p.cin) {
                    v = p.x[((size_t(img) * p.cin + ci) * p.h + iy) * p.w + ix];
                    if (p.in_scale) v *= p.in_scale[size_t(img) * p.cin + ci];
                }
                const _Float16 hi = (_Float16)v;
                s_hi[hp][cl] = hi;
                s_lo[hp][cl] = (_Float16)(v - (float)hi);
            }
        } else {
            for (int i = tid; i < HALO * 8; i += 256) {
                const int hp = i >> 3, q = i & 7;
                const int hy = hp / HWD, hx = hp - hy * HWD;
                const int iy = iy0 + hy, ix = ix0 + hx, ci = ci0 + 4 * q;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (iy >= 0 && iy < p.h && ix >= 0 && ix < p.w && ci < p.cin) {
                    size_t px = size_t(iy) * p.w + ix;
                    if constexpr (KS == 1) if (p.rows) px = size_t(p.rows[ix]);
                    const float *src = xim + px * p.xcs + ci;
                    if (p.vec) {
                        v = *reinterpret_cast<const float4 *>(src);
                    } else {
                        v.x = src[0];
                        if (ci + 1 < p.cin) v.y = src[1];
                        if (ci + 2 < p.cin) v.z = src[2];
                        if (ci + 3 < p.cin) v.w = src[3];
                    }
                    if (p.in_scale) {
                        const float *sc = p.in_scale + size_t(img) * p.cin + ci;
                        v.x *= sc[0];
                        if (ci + 1 < p.cin) v.y *= sc[1];
                        if (ci + 2 < p.cin) v.z *= sc[2];
                        if (ci + 3 < p.cin) v.w *= sc[3];
                    }
                }
                half4 hi = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
                half4 lo = {(_Float16)(v.x - (float)hi[0]), (_Float16)(v.y - (float)hi[1]),
                            (_Float16)(v.z - (float)hi[2]), (_Float16)(v.w - (float)hi[3])};
                *reinterpret_cast<half4 *>(&s_hi[hp][4 * q]) = hi;
                *reinterpret_cast<half4 *>(&s_lo[hp][4 * q]) = lo;
            }
        }
        // Stage this slice's weights for every tap: [tap][BN][32] halves, contiguous in HBM.
        {
            const size_t base = (size_t(nb) * p.chunks + chunk) * taps * BN * 4;  // in half8 units
            for (int i = tid; i < taps * BN * 4; i += 256) {
                const int tap = i / (BN * 4), rem = i - tap * BN * 4, co = rem >> 2, q = rem & 3;
                *reinterpret_cast<half8 *>(&s_w[tap][co][8 * q]) = p.wt_hi[base + i];
                if constexpr (LO) *reinterpret_cast<half8 *>(&s_wl[tap][co][8 * q]) = p.wt_lo[base + i];
            }
        }
        __syncthreads();
        for (int tap = 0; tap < taps; tap++) {
            const int ky = tap / p.kw, kx = tap - ky * p.kw;
            half8 ahi[2], alo[2];
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const int pix = wave * 32 + m * 16 + r;
                const int py = pix / TW, px = pix - py * TW;
                const int hp = (py + ky) * HWD + px + kx;
                ahi[m] = *reinterpret_cast<const half8 *>(&s_hi[hp][8 * g]);
                alo[m] = *reinterpret_cast<const half8 *>(&s_lo[hp][8 * g]);
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const half8 b = *reinterpret_cast<const half8 *>(&s_w[tap][t * 16 + r][8 * g]);
#pragma unroll
                for (int m = 0; m < 2; m++) {
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[m], b, acc[m][t], 0, 0, 0);
                    acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[m], b, acc[m][t], 0, 0, 0);
                }
                if constexpr (LO) {
                    const half8 bl = *reinterpret_cast<const half8 *>(&s_wl[tap][t * 16 + r][8 * g]);
#pragma unroll
                    for (int m = 0; m < 2; m++)
                        acc[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[m], bl, acc[m][t], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }
    // Epilogue: lane holds rows 4g..4g+3 (pixels) of column r (channel) of each 16 x 16 tile.
    // y = act(affine(acc + b)) + res, in the order the fused nodes run.
    if (p.amax) {
        // Arg-max partials of a GEMM row (1 x 1, NHWC): the best of this block's channels, the
        // first index on ties, reduced over the 16 lanes that share the rows.
#pragma unroll
        for (int m = 0; m < 2; m++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float bv = -INFINITY;
                int bi = 0x7fffffff;
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const int co = co0 + t * 16 + r;
                    if (co >= p.cout) continue;
                    const float v = acc[m][t][i] + (p.bias ? p.bias[co] : 0.f);
                    if (v > bv) { bv = v; bi = co; }
                }
                for (int off = 8; off > 0; off >>= 1) {
                    const float ov = __shfl_xor(bv, off);
                    const int oi = __shfl_xor(bi, off);
                    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
                }
                const int pix = wave * 32 + m * 16 + 4 * g + i;
                const int oy = oy0 + pix / TW, ox = ox0 + pix % TW;
                if (r == 0 && oy < p.oh && ox < p.ow) {
                    const size_t o = (size_t(img) * p.oh + oy) * p.ow + ox;
                    p.amax[o * gridDim.y + nb] = make_float2(bv, __int_as_float(bi));
                }
            }
        return;
    }
    if constexpr (KS == 3) if (p.yp) {
        // MaxPool fused: the activated tile goes to LDS (the weight buffer, free after the last
        // barrier), then each thread takes one channel of successive pooled pixels, so pooled
        // (and full-size) NHWC stores are contiguous along the channels. The tile's TH x TW
        // pixels hold whole pooling windows (the host picks TH, TW divisible by ph, pw).
        constexpr int SROW = BN + 1;
        float *s_out = reinterpret_cast<float *>(&s_w[0][0][0]);
        static_assert(128 * SROW * 4 <= int(sizeof(s_w)), "pooled tile does not fit the weight buffer");
#pragma unroll
        for (int m = 0; m < 2; m++)
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const int co = co0 + t * 16 + r;
                const float bv = (co < p.cout && p.bias) ? p.bias[co] : 0.f;
#pragma unroll
                for (int i = 0; i < 4; i++)
                    s_out[(wave * 32 + m * 16 + 4 * g + i) * SROW + t * 16 + r] = activate_dev(acc[m][t][i] + bv, p.act);
            }
        __syncthreads();
        if (p.y) {
            for (int idx = tid; idx < 128 * BN; idx += 256) {
                const int c = idx % BN, pix = idx / BN;
                const int oy = oy0 + pix / TW, ox = ox0 + pix % TW;
                if (oy < p.oh && ox < p.ow && co0 + c < p.cout)
                    p.y[((size_t(img) * p.oh + oy) * p.ow + ox) * p.ycs + co0 + c] = s_out[pix * SROW + c];
            }
        }
        const int pth = TH / p.ph, ptw = TW / p.pw;
        for (int idx = tid; idx < pth * ptw * BN; idx += 256) {
            const int c = idx % BN, pp = idx / BN;
            const int py = pp / ptw, px = pp - py * ptw;
            const int poy = oy0 / p.ph + py, pox = ox0 / p.pw + px;
            if (poy >= p.poh || pox >= p.pow_ || co0 + c >= p.cout) continue;
            float v = -INFINITY;
            for (int qy = 0; qy < p.ph; qy++)
                for (int qx = 0; qx < p.pw; qx++)
                    v = fmaxf(v, s_out[((py * p.ph + qy) * TW + px * p.pw + qx) * SROW + c]);
            p.yp[((size_t(img) * p.poh + poy) * p.pow_ + pox) * p.ypcs + co0 + c] = v;
        }
        return;
    }
#pragma unroll
    for (int m = 0; m < 2; m++) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const int co = co0 + t * 16 + r;
            if (co >= p.cout) continue;
            const float bv = p.bias ? p.bias[co] : 0.f;
            const float as = p.affine ? p.affine[co] : 1.f, at = p.affine ? p.affine[p.cout + co] : 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int pix = wave * 32 + m * 16 + 4 * g + i;
                const int oy = oy0 + pix / TW, ox = ox0 + pix % TW;
                if (oy >= p.oh || ox >= p.ow) continue;
                float v = acc[m][t][i] + bv;
                if (p.affine) v = v * as + at;
                v = activate_dev(v, p.act);
                if (p.nchw) {
                    const size_t o = ((size_t(img) * p.cout + co) * p.oh + oy) * p.ow + ox;
                    if (p.res) v += p.res[o];
                    p.y[o] = v;
                } else {
                    size_t o = size_t(img) * p.yn + size_t(oy) * p.yy + size_t(ox) * p.yx;
                    if constexpr (KS == 1) if (p.rows) o = size_t(p.rows[ox]);
                    if (p.res) v += p.res[o * p.rcs + co];
                    p.y[o * p.ycs + co] = v;
                }
            }
        }
    }
}

template <int TW, int KS, int BN>
void launch3(const ConvParams &p, bool lo, dim3 grid, hipStream_t s) {
    if (lo)
        hipLaunchKernelGGL((conv_mfma_kernel<TW, KS, BN, true>), grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((conv_mfma_kernel<TW, KS, BN, false>), grid, dim3(256), 0, s, p);
}

template <int TW, int KS>
void launch2(const ConvParams &p, int bn, bool lo, dim3 grid, hipStream_t s) {
    if (bn == 16) launch3<TW, KS, 16>(p, lo, grid, s);
    else if (bn == 32) launch3<TW, KS, 32>(p, lo, grid, s);
    else launch3<TW, KS, 64>(p, lo, grid, s);
}

}  // namespace

ConvPack plan_conv_pack(int cin, int cout, int kh, int kw) {
    ConvPack pk;
    pk.cin = cin;
    pk.cout = cout;
    pk.kh = kh;
    pk.kw = kw;
    pk.bn = cout >= 64 ? 64 : (cout > 16 ? 32 : 16);
    pk.chunks = (cin + 31) / 32;
    pk.nblocks = (cout + pk.bn - 1) / pk.bn;
    return pk;
}

void pack_conv_weights(const ConvPack &pk, const float *w, uint16_t *hi, uint16_t *lo, bool *exact) {
    bool ex = true;
    const int taps = pk.kh * pk.kw;
    size_t i = 0;
    for (int nb = 0; nb < pk.nblocks; nb++)
        for (int ch = 0; ch < pk.chunks; ch++)
            for (int tap = 0; tap < taps; tap++)
                for (int c = 0; c < pk.bn; c++)
                    for (int k = 0; k < 32; k++, i++) {
                        const int co = nb * pk.bn + c, ci = ch * 32 + k;
                        float v = 0.f;
                        if (co < pk.cout && ci < pk.cin)
                            v = w[((size_t(co) * pk.cin + ci) * pk.kh + tap / pk.kw) * pk.kw + tap % pk.kw];
                        _Float16 h = (_Float16)v;
                        _Float16 l = (_Float16)(v - (float)h);
                        if ((float)h != v) ex = false;
                        __builtin_memcpy(&hi[i], &h, 2);
                        __builtin_memcpy(&lo[i], &l, 2);
                    }
    *exact = ex;
}

bool conv_mfma_supported(int kh, int kw, int sh, int sw) { return sh == 1 && sw == 1 && kh <= 3 && kw <= 3; }

void conv_mfma(const ConvArgs &a, hipStream_t s) {
    static const bool no_igemm = std::getenv("NOIGEMM") != nullptr, no_dma = std::getenv("NOCONVDMA") != nullptr;
    if (!no_igemm && !no_dma && conv3x3_dma(a, s)) return;
    if (!no_igemm && !no_dma && gemm_dma(a, s)) return;
    if (!no_igemm && conv_igemm(a, s)) return;
    const ConvPack &pk = a.pk;
    ConvParams p{};
    p.x = a.x.p;
    p.n = a.x.n;
    p.h = a.x.h;
    p.w = a.x.w;
    p.cin = a.x.c;
    p.xcs = a.x.cs;
    p.y = a.y.p;
    p.oh = a.y.h;
    p.ow = a.y.w;
    p.cout = a.y.c;
    p.ycs = a.y.cs;
    p.wt_hi = reinterpret_cast<const half8 *>(a.wt_hi);
    p.wt_lo = reinterpret_cast<const half8 *>(a.wt_lo);
    p.bias = a.bias;
    p.res = a.res;
    p.affine = a.affine;
    p.in_scale = a.in_scale;
    p.amax = reinterpret_cast<float2 *>(a.amax_part);
    p.rows = a.rows;
    if (a.rows && (pk.kh != 1 || pk.kw != 1 || a.nchw || a.x.n != 1 || a.x.h != 1 || a.amax_part || a.res ||
                   a.y_px || a.y_row || a.y_img))
        fail("conv_mfma: a row map needs a plain 1 x 1 NHWC GEMM over one row of pixels");
    p.nchw = a.nchw ? 1 : 0;
    p.rcs = a.res_cs;
    p.kh = pk.kh;
    p.kw = pk.kw;
    p.pt = a.pt;
    p.pl = a.pl;
    p.act = a.act;
    p.chunks = pk.chunks;
    p.vec = (p.cin % 4 == 0 && p.xcs % 4 == 0 && (reinterpret_cast<uintptr_t>(p.x) & 15) == 0) ? 1 : 0;
    if (a.amax_part && (a.nchw || pk.kh != 1 || pk.kw != 1)) fail("conv_mfma: arg-max partials need a 1 x 1 NHWC GEMM");
    if (pk.cin != a.x.c || pk.cout != a.y.c) fail("conv_mfma: channel counts differ from the packed weights");
    if (a.y.n != a.x.n) fail("conv_mfma: batch mismatch");
    const bool lo = !pk.exact;
    const int ks = (pk.kh == 1 && pk.kw == 1) ? 1 : 3;
    const bool pooled = a.ypool.p != nullptr;
    if (pooled) {
        if (ks != 3 || a.nchw || a.res || a.affine || a.amax_part) fail("conv_mfma: MaxPool fused only into a 3 x 3 NHWC conv");
        if (a.ph < 1 || a.pw < 1 || a.ph > 8 || a.pw > 16) fail("conv_mfma: pool size");
        if (a.ypool.h != a.y.h / a.ph || a.ypool.w != a.y.w / a.pw || a.ypool.c != a.y.c || a.ypool.n != a.y.n)
            fail("conv_mfma: pooled output shape");
    }
    p.y = pooled && !a.keep_full ? nullptr : a.y.p;
    p.yx = a.y_px ? size_t(a.y_px) : 1;
    p.yy = a.y_row ? size_t(a.y_row) : size_t(p.ow) * p.yx;
    p.yn = a.y_img ? size_t(a.y_img) : size_t(p.oh) * p.yy;
    if ((a.y_px || a.y_row || a.y_img) && (a.nchw || pooled || a.amax_part)) fail("conv_mfma: output strides only for plain NHWC");
    p.yp = a.ypool.p;
    p.poh = a.ypool.h;
    p.pow_ = a.ypool.w;
    p.ypcs = a.ypool.cs;
    p.ph = pooled ? a.ph : 1;
    p.pw = pooled ? a.pw : 1;
    int tw = 128;
    if (ks == 3) {
        // The tile shape that wastes the fewest pixels (padding and halo) for this output size
        // (whole pooling windows per tile when a MaxPool is fused).
        double best = 1e300;
        for (int cand : {16, 32, 64}) {
            const int th = 128 / cand;
            if (pooled && (th % a.ph != 0 || cand % a.pw != 0)) continue;
            const double cost = double((p.oh + th - 1) / th * th) * ((p.ow + cand - 1) / cand * cand) *
                                double((th + 2) * (cand + 2)) / (th * cand);
            if (cost < best) { best = cost; tw = cand; }
        }
        if (best == 1e300) fail("conv_mfma: no tile holds whole pooling windows");
    }
    const int th = 128 / tw;
    p.tiles_x = (p.ow + tw - 1) / tw;
    p.tiles_y = (p.oh + th - 1) / th;
    const size_t blocks = size_t(p.tiles_x) * p.tiles_y * p.n;
    if (blocks > 0x7fffffff) fail("conv_mfma: grid too large");
    dim3 grid(unsigned(blocks), unsigned(pk.nblocks));
    const double flops = 2.0 * p.n * p.oh * p.ow * p.cout * p.cin * pk.kh * pk.kw;
    const double bytes = 4.0 * (double(p.n) * p.h * p.w * p.cin + double(p.n) * p.oh * p.ow * p.cout) +
                         2.0 * double(pk.halves()) * (lo ? 2 : 1);
    ProbeScope probe("conv_mfma", s, flops, bytes);
    if (ks == 1) launch2<128, 1>(p, pk.bn, lo, grid, s);
    else if (tw == 16) launch2<16, 3>(p, pk.bn, lo, grid, s);
    else if (tw == 32) launch2<32, 3>(p, pk.bn, lo, grid, s);
    else launch2<64, 3>(p, pk.bn, lo, grid, s);
    OCR_HIP(hipGetLastError());
}

}  // namespace ocr
