// Stride-1 convolution (kernel up to 3 x 3) and 1 x 1 GEMM on the gfx950 matrix cores, for NHWC
// float32 activations and float32 weights: the hot path of the ocrs detector, recogniser
// trunk and GRU projections. Semantics of the reference's conv / conv_fast / conv128 and gemm
// programs (src/gpu.rs:37-350, 616-678): y = act(sum_k x * w + b[c]), then an optional MaxPool
// (gpu.rs:462-482) of the activated output.
//
// Precision: each float32 activation is split into float16 hi and the float16 remainder lo
// (x = hi + lo to about 2^-22) and both go through v_mfma_f32_16x16x32_f16 against the exact
// float16 weights with float32 accumulation: float32-class results at twice the f16 work.
//
// Work split (one output tile per workgroup of 4 wavefronts):
// - The workgroup owns TH x TW output pixels and BN = 16 * NT * WN output channels; wavefront
//   (wm, wn) of the WM x WN grid computes 64 pixels (4 MFMA row tiles) x 16 * NT channels, so
//   every A fragment read from LDS feeds 2 * NT MFMAs.
// - K runs over slices of 32 input channels; for each slice the tile's input halo
//   ((TH + kh - 1) x (TW + kw - 1) pixels) is staged in LDS once, split into hi / lo, and every
//   tap is a shifted read of it.
// - The weights never touch LDS: each B fragment (16 channels x 32 inputs of one tap, 1 KiB
//   contiguous in the packed layout) is loaded from L2 straight into registers one tap ahead.
// - Row tile geometry: an MFMA row tile is 16 pixels, either 16 of one row (GEMM rows) or a
//   2 x 8 block laid out as four 2 x 2 squares, one per group of 4 rows. The MFMA gives lane
//   (g, r) rows 4g..4g+3 of column r, i.e. one 2 x 2 square of one channel, so a fused 2 x 2 or
//   2 x 1 MaxPool is a max over the lane's own accumulators.
// - Blocks are renumbered so that the 8 XCDs each take a contiguous run of tiles (neighbouring
//   tiles share halo rows in that XCD's L2).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>
#include <cstring>

#include "../kernels.h"
#include "../runtime.h"

namespace ocr {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int PXS = 72;  // halves per LDS halo pixel: 32 hi, 32 lo, 8 padding (36 dwords)
constexpr int MT = 4;    // MFMA row tiles (of 16 pixels) per wavefront

struct IgParams {
    const float *x;
    int n, h, w, cin, xcs;
    float *y;  // full-size output, or null (pooled only)
    int oh, ow, ycs;
    long yn, yy, yx;  // output pixel strides: image, row, column
    float *yp;        // pooled output, or null
    int poh, pow_, ypcs, pool;  // pool: 0 none, 1 = 2 x 2, 2 = 2 x 1 (rows)
    const half8 *wt;     // packed [cout block of pbn][slice][tap][pbn][32] float16
    const half8 *wt_lo;  // the same layout of the float16 remainders (inexact weights), or null
    int pbn, cpad;       // the pack's block width and padded channel count
    int cout;
    const float *bias;
    const int *rows;  // GEMM row map (gather x rows, scatter y rows), or null
    int phc, phs, phh, phw;  // ConvTranspose phases: channels a phase, stride, y's size (0: off)
    int kw, pt, pl, act, chunks, taps;
    int slices;  // passes over the input's chunks: chunks, or 2 chunks with remainders
    int th, tw, mx;   // tile rows and columns; row tiles per tile row of blocks
    int hw, hwp, halo_px;  // halo columns, padded row length, halo pixels
    int tiles_x, tiles_y, tiles;
    int lin;  // 1: row tiles are 16 pixels of one row; 0: 2 x 8 blocks
};

__device__ inline float act_dev(float v, int act) {
    if (act == ACT_RELU) return fmaxf(v, 0.f);
    if (act == ACT_SIGMOID) return 1.f / (1.f + expf(-v));
    if (act == ACT_GELU) return 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    if (act == ACT_SILU) return v / (1.f + expf(-v));
    return v;
}

// Block b of G runs on XCD b % 8; tiles are handed out so that each XCD gets a contiguous run.
__device__ inline int xcd_tile(int b, int G) {
    const int q = G >> 3, rem = G & 7, x = b & 7;
    return x * q + min(x, rem) + (b >> 3);
}

template <int WM, int WN, int NT, int SI>
__global__ __launch_bounds__(256) void conv_igemm_kernel(IgParams p) {
    extern __shared__ __align__(16) _Float16 halo[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int g = lane >> 4, r = lane & 15;
    const int tile = xcd_tile(blockIdx.x, gridDim.x);
    const int tx = tile % p.tiles_x, rest = tile / p.tiles_x;
    const int ty = rest % p.tiles_y, img = rest / p.tiles_y;
    const int oy0 = ty * p.th, ox0 = tx * p.tw;
    const int co_w = blockIdx.y * (16 * NT * WN) + wn * 16 * NT;  // this wavefront's first channel

    // Halo slot of this lane's pixel in each row tile (tap 0) and the pixel's tile coordinates.
    int aslot[MT], py[MT], px[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int mi = wm * MT + mt;
        if (p.lin) {
            py[mt] = 0;
            px[mt] = mi * 16 + r;
        } else {
            const int mxi = mi % p.mx, myi = mi / p.mx, q = r & 3;
            py[mt] = 2 * myi + (q >> 1);
            px[mt] = 8 * mxi + 2 * (r >> 2) + (q & 1);
        }
        aslot[mt] = py[mt] * p.hwp + px[mt];
    }

    floatx4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int j = 0; j < NT; j++) acc[mt][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // B fragment of n-tile j for (slice, tap): lane (g, r) takes channel co + r, inputs 8g..8g+7.
    auto load_b = [&](half8 (&b)[NT], const half8 *wt, int c, int tap) {
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int co = co_w + 16 * j;
            if (co < p.cpad) {
                const int nbp = co / p.pbn, off = co - nbp * p.pbn;
                b[j] = wt[((size_t(nbp * p.chunks + c) * p.taps + tap) * p.pbn + off + r) * 4 + g];
            } else {
                b[j] = half8{};
            }
        }
    };

    const int iy0 = oy0 - p.pt, ix0 = ox0 - p.pl;
    // Slice sl: input chunk c against the float16 weights, then (inexact weights) every chunk
    // again against the remainders.
    for (int sl = 0; sl < p.slices; sl++) {
        const int c = sl < p.chunks ? sl : sl - p.chunks;
        const half8 *wt = sl < p.chunks ? p.wt : p.wt_lo;
        const int ci0 = c * 32;
        // Stage the halo: 8 threads per pixel, 4 channels each; zero outside the image.
        float4 st[SI];
#pragma unroll
        for (int s = 0; s < SI; s++) {
            const int i = tid + s * 256, hp = i >> 3, q = i & 7;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (hp < p.halo_px) {
                const int hy = hp / p.hw, hx = hp - hy * p.hw;
                const int iy = iy0 + hy, ix = ix0 + hx, ci = ci0 + 4 * q;
                if (iy >= 0 && iy < p.h && ix >= 0 && ix < p.w && ci < p.cin) {
                    const size_t pix = p.rows ? size_t(p.rows[ix]) : (size_t(img) * p.h + iy) * p.w + ix;
                    v = *reinterpret_cast<const float4 *>(p.x + pix * p.xcs + ci);
                }
            }
            st[s] = v;
        }
        half8 bcur[NT];
        load_b(bcur, wt, c, 0);
        if (sl > 0) __syncthreads();  // every wavefront is done with the previous slice
#pragma unroll
        for (int s = 0; s < SI; s++) {
            const int i = tid + s * 256, hp = i >> 3, q = i & 7;
            if (hp < p.halo_px) {
                const int hy = hp / p.hw, hx = hp - hy * p.hw;
                const float4 v = st[s];
                const half4 hi = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
                const half4 lo = {(_Float16)(v.x - (float)hi[0]), (_Float16)(v.y - (float)hi[1]),
                                  (_Float16)(v.z - (float)hi[2]), (_Float16)(v.w - (float)hi[3])};
                _Float16 *d = halo + (hy * p.hwp + hx) * PXS + 4 * q;
                *reinterpret_cast<half4 *>(d) = hi;
                *reinterpret_cast<half4 *>(d + 32) = lo;
            }
        }
        __syncthreads();
        for (int tap = 0; tap < p.taps; tap++) {
            half8 bnext[NT];
            if (tap + 1 < p.taps) load_b(bnext, wt, c, tap + 1);
            const int ky = tap / p.kw, kx = tap - ky * p.kw, toff = ky * p.hwp + kx;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const _Float16 *a = halo + (aslot[mt] + toff) * PXS + 8 * g;
                const half8 ahi = *reinterpret_cast<const half8 *>(a);
                const half8 alo = *reinterpret_cast<const half8 *>(a + 32);
#pragma unroll
                for (int j = 0; j < NT; j++) {
                    acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bcur[j], acc[mt][j], 0, 0, 0);
                    acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bcur[j], acc[mt][j], 0, 0, 0);
                }
            }
            if (tap + 1 < p.taps) {
#pragma unroll
                for (int j = 0; j < NT; j++) bcur[j] = bnext[j];
            }
        }
    }

    // Epilogue: lane (g, r) holds rows 4g..4g+3 of channel co_w + 16 j + r in each row tile.
#pragma unroll
    for (int j = 0; j < NT; j++) {
        int co = co_w + 16 * j + r;
        if (co >= p.cout) continue;
        // ConvTranspose phase k of channel co: its pixel offset in y and its own channel.
        size_t phoff = 0;
        int ppy = 0, ppx = 0;
        if (p.phc) {
            const int k = co / p.phc;
            co -= k * p.phc;
            ppy = k / p.phs, ppx = k % p.phs;
            phoff = size_t(ppy) * p.phw + size_t(ppx);
        }
        const float bv = p.bias ? p.bias[co] : 0.f;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = act_dev(acc[mt][j][i] + bv, p.act);
            if (p.lin) {
                // 4 consecutive pixels of one row: 4g..4g+3 of the row tile.
                if (p.y) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int ox = ox0 + (wm * MT + mt) * 16 + 4 * g + i;
                        if (ox >= p.ow) continue;
                        const size_t o = p.rows ? size_t(p.rows[ox])
                                                : size_t(img) * p.yn + size_t(oy0) * p.yy + size_t(ox) * p.yx;
                        p.y[o * p.ycs + co] = v[i];
                    }
                }
                continue;
            }
            // A 2 x 2 square: v[0] (y, x), v[1] (y, x+1), v[2] (y+1, x), v[3] (y+1, x+1).
            const int oy = oy0 + (py[mt] & ~1), ox = ox0 + 8 * ((wm * MT + mt) % p.mx) + 2 * g;
            if (p.y) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int yy = oy + (i >> 1), xx = ox + (i & 1);
                    if (yy < p.oh && xx < p.ow &&
                        (!p.phc || (yy * p.phs + ppy < p.phh && xx * p.phs + ppx < p.phw)))
                        p.y[(size_t(img) * p.yn + size_t(yy) * p.yy + size_t(xx) * p.yx + phoff) * p.ycs + co] = v[i];
                }
            }
            if (p.pool == 1) {
                const int qy = oy >> 1, qx = ox >> 1;
                if (qy < p.poh && qx < p.pow_)
                    p.yp[((size_t(img) * p.poh + qy) * p.pow_ + qx) * p.ypcs + co] =
                        fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
            } else if (p.pool == 2) {
                const int qy = oy >> 1;
                if (qy < p.poh) {
                    const size_t base = (size_t(img) * p.poh + qy) * p.pow_;
                    if (ox < p.pow_) p.yp[(base + ox) * p.ypcs + co] = fmaxf(v[0], v[2]);
                    if (ox + 1 < p.pow_) p.yp[(base + ox + 1) * p.ypcs + co] = fmaxf(v[1], v[3]);
                }
            }
        }
    }
}

template <int WM, int WN, int NT, int SI>
void launch(const IgParams &p, dim3 grid, size_t lds, hipStream_t s) {
    hipLaunchKernelGGL((conv_igemm_kernel<WM, WN, NT, SI>), grid, dim3(256), lds, s, p);
}

// SI (float4 staging loads per thread) for the halo sizes of a config.
template <int WM, int WN, int NT>
void launch_si(const IgParams &p, dim3 grid, size_t lds, hipStream_t s) {
    const int si = (p.halo_px * 8 + 255) / 256;
    if (si <= 4) launch<WM, WN, NT, 4>(p, grid, lds, s);
    else if (si <= 6) launch<WM, WN, NT, 6>(p, grid, lds, s);
    else if (si <= 8) launch<WM, WN, NT, 8>(p, grid, lds, s);
    else if (si <= 11) launch<WM, WN, NT, 11>(p, grid, lds, s);
    else fail("conv_igemm: halo too large");
}

}  // namespace

void pack_conv_frags(const ConvPack &pk, const uint16_t *hi, const uint16_t *lo, uint16_t *frag) {
    // hi, lo: [nblock][chunk][tap][bn][32]; frag: [n-tile][slice][tap][lane = 16 g + r][8], lane
    // (g, r) holding inputs 8g..8g+7 of channel 16 * tile + r; slice c >= chunks is lo's c - chunks.
    if (!pk.exact && !lo) fail("pack_conv_frags: inexact weights need their remainders");
    const int taps = pk.kh * pk.kw, ntiles = pk.nblocks * pk.bn / 16, slices = pk.frag_chunks();
    size_t o = 0;
    for (int nt = 0; nt < ntiles; nt++)
        for (int sl = 0; sl < slices; sl++) {
            const uint16_t *src_w = sl < pk.chunks ? hi : lo;
            const int c = sl < pk.chunks ? sl : sl - pk.chunks;
            for (int tap = 0; tap < taps; tap++)
                for (int l = 0; l < 64; l++, o += 8) {
                    const int g = l >> 4, r = l & 15, co = nt * 16 + r;
                    const int nb = co / pk.bn, off = co - nb * pk.bn;
                    const size_t src = (((size_t(nb) * pk.chunks + c) * taps + tap) * pk.bn + off) * 32 + 8 * g;
                    std::memcpy(frag + o, src_w + src, 8 * sizeof(uint16_t));
                }
        }
}

bool conv_igemm(const ConvArgs &a, hipStream_t s) {
    const ConvPack &pk = a.pk;
    if (a.nchw || a.in_scale || a.affine || a.amax_part || a.res) return false;
    if (!pk.exact && !a.wt_lo) return false;
    const bool phm = a.ph_cout > 0;
    if (phm) {
        // All s x s phases of a ConvTranspose: one conv over x (taps (a, b) read x[i - a][j - b],
        // leading pads kh - 1, kw - 1) on the grid of ceil(y.h / s) x ceil(y.w / s) positions.
        const int st = a.ph_s;
        if (st < 1 || pk.cout != st * st * a.ph_cout || a.y.c != a.ph_cout || a.pt != pk.kh - 1 ||
            a.pl != pk.kw - 1 || a.ypool.p || a.rows || a.y_px || a.y_row || a.y_img)
            return false;
    } else if (pk.cout != a.y.c) {
        return false;
    }
    if (pk.kh > 3 || pk.kw > 3 || pk.cin != a.x.c || a.y.n != a.x.n) return false;
    if (a.x.c % 4 || a.x.cs % 4 || (reinterpret_cast<uintptr_t>(a.x.p) & 15)) return false;
    const bool pooled = a.ypool.p != nullptr;
    int pool = 0;
    if (pooled) {
        if (a.ph == 2 && a.pw == 2) pool = 1;
        else if (a.ph == 2 && a.pw == 1) pool = 2;
        else return false;
        if (a.y_px || a.y_row || a.y_img) return false;
        if (a.ypool.h != a.y.h / a.ph || a.ypool.w != a.y.w / a.pw || a.ypool.c != a.y.c || a.ypool.n != a.y.n)
            fail("conv_igemm: pooled output shape");
    }
    if (a.rows && (pk.kh != 1 || pk.kw != 1 || a.x.n != 1 || a.x.h != 1 || pooled)) return false;
    const int cout = pk.cout;
    // Wavefront grid and channels per wavefront for this output width.
    int WM, WN, NT;
    if (cout <= 16) WM = 4, WN = 1, NT = 1;
    else if (cout <= 32) WM = 4, WN = 1, NT = 2;
    else if (cout <= 64) WM = 4, WN = 1, NT = 4;
    else WM = 2, WN = 2, NT = 4;
    const int bm = 64 * WM, bn = 16 * NT * WN;

    IgParams p{};
    p.x = a.x.p;
    p.n = a.x.n;
    p.h = a.x.h;
    p.w = a.x.w;
    p.cin = a.x.c;
    p.xcs = a.x.cs;
    p.oh = a.y.h;
    p.ow = a.y.w;
    p.ycs = a.y.cs;
    p.yx = a.y_px ? a.y_px : 1;
    p.yy = a.y_row ? a.y_row : long(p.ow) * p.yx;
    p.yn = a.y_img ? a.y_img : long(p.oh) * p.yy;
    if (phm) {
        // Grid position (i, j), phase (py, px) is y's pixel (s i + py, s j + px) when inside y.
        p.oh = (a.y.h + a.ph_s - 1) / a.ph_s;
        p.ow = (a.y.w + a.ph_s - 1) / a.ph_s;
        p.yx = a.ph_s;
        p.yy = long(a.ph_s) * a.y.w;
        p.yn = long(a.y.h) * a.y.w;
        p.phc = a.ph_cout;
        p.phs = a.ph_s;
        p.phh = a.y.h;
        p.phw = a.y.w;
    }
    p.y = pooled && !a.keep_full ? nullptr : a.y.p;
    p.yp = a.ypool.p;
    p.poh = a.ypool.h;
    p.pow_ = a.ypool.w;
    p.ypcs = a.ypool.cs;
    p.pool = pool;
    p.wt = reinterpret_cast<const half8 *>(a.wt_hi);
    p.wt_lo = pk.exact ? nullptr : reinterpret_cast<const half8 *>(a.wt_lo);
    p.pbn = pk.bn;
    p.cpad = pk.nblocks * pk.bn;
    p.cout = cout;
    p.bias = a.bias;
    p.rows = a.rows;
    p.kw = pk.kw;
    p.pt = a.pt;
    p.pl = a.pl;
    p.act = a.act;
    p.chunks = pk.chunks;
    p.slices = pk.exact ? pk.chunks : 2 * pk.chunks;
    p.taps = pk.kh * pk.kw;

    // Tile shape: one row of bm pixels for a one-row input (GEMM rows); otherwise 2 x 8 blocks,
    // the column count that wastes the fewest pixels (padding and halo) for this output.
    if (p.oh == 1 && p.h == 1 && pk.kh == 1 && !pooled && !phm) {
        p.lin = 1;
        p.th = 1;
        p.tw = bm;
        p.mx = 1;
    } else {
        p.lin = 0;
        const int nblk = bm / 16;  // 2 x 8 blocks per tile
        double best = 1e300;
        for (int mxc : {1, 2, 4, 8}) {
            if (nblk % mxc) continue;
            const int tw = 8 * mxc, th = 2 * (nblk / mxc);
            const int hwd = tw + pk.kw - 1, hh = th + pk.kh - 1;
            if (hh * hwd * 8 > 11 * 256) continue;
            const double cost = double((p.oh + th - 1) / th * th) * ((p.ow + tw - 1) / tw * tw) *
                                double(hh * hwd) / double(th * tw);
            if (cost < best) best = cost, p.tw = tw, p.th = th, p.mx = mxc;
        }
        if (best == 1e300) return false;
    }
    p.hw = p.tw + pk.kw - 1;
    const int hh = p.th + pk.kh - 1;
    p.hwp = p.lin ? p.hw : (p.hw + 3) / 8 * 8 + 4;  // row length = 4 mod 8 pixels: LDS banks spread
    p.halo_px = hh * p.hw;
    if (p.halo_px * 8 > 11 * 256) return false;
    p.tiles_x = (p.ow + p.tw - 1) / p.tw;
    p.tiles_y = (p.oh + p.th - 1) / p.th;
    const double tiles = double(p.tiles_x) * p.tiles_y * p.n;
    if (tiles > 0x7fffffff) return false;
    p.tiles = int(tiles);
    const int nblocks = (cout + bn - 1) / bn;
    const size_t lds = size_t(hh) * p.hwp * PXS * sizeof(_Float16);
    dim3 grid(unsigned(p.tiles), unsigned(nblocks));
    const double flops = 2.0 * p.n * p.oh * p.ow * cout * p.cin * pk.kh * pk.kw;
    const double bytes = 4.0 * (double(p.n) * p.h * p.w * p.cin + double(p.n) * p.oh * p.ow * cout) +
                         2.0 * double(pk.frag_halves());
    ProbeScope probe("conv_igemm", s, flops, bytes);
    if (WM == 4 && NT == 1) launch_si<4, 1, 1>(p, grid, lds, s);
    else if (WM == 4 && NT == 2) launch_si<4, 1, 2>(p, grid, lds, s);
    else if (WM == 4) launch_si<4, 1, 4>(p, grid, lds, s);
    else launch_si<2, 2, 4>(p, grid, lds, s);
    OCR_HIP(hipGetLastError());
    return true;
}

}  // namespace ocr
