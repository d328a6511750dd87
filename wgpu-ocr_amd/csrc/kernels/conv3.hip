// 3 x 3 stride-1 convolution (NHWC float32 activations, float32 weights) on the gfx950
// matrix cores with the operands fed by the LDS DMA path: the hot
// path of the recogniser trunk and the detector's deeper layers. Semantics of the reference's
// conv / conv_fast / conv128 programs (src/gpu.rs:37-350): y = act(sum x * w + b[c]), then an
// optional 2 x 2 or 2 x 1 MaxPool of the activated output (gpu.rs:462-482).
//
// Precision: each float32 activation is split into float16 hi and the float16 remainder lo
// (x = hi + lo to about 2^-22) and both go through v_mfma_f32_16x16x32_f16 against the float16
// weights with float32 accumulation. Weights that are not all float16 values are packed as
// further slices of their float16 remainders, and the input's slices are walked a second time
// against them: sum (hi + lo)(w_hi + w_lo), float32-class products at twice the matrix work.
//
// Data movement: nothing is staged through registers. global_load_lds_dwordx4 writes 16 bytes a
// lane straight into LDS (lane l at base + 16 l), so
// - weights: one stage is one kernel row (3 taps) of one 32-channel input slice for the block's
//   output channels; its MFMA B fragments (1 KiB each, lane-ordered in HBM) are copied as they
//   are into one of two stage buffers;
// - input: the tile's halo for the next slice lands float32 in a staging buffer (HF) while the
//   current slice is being computed, a pixel's eight 16-byte parts swapped in pairs on odd pixel
//   pairs; at the slice boundary all threads split it once into two planes, hi (HSH) and lo
//   (HSL), 64 bytes a pixel each: part g (channels 8g..8g+7) of halo pixel (y, x) at 16-byte
//   unit y * rs + 4 x + (g ^ 2 (y & 1)), rs a multiple of 16 units.
//   Why that layout: gfx950 serves a 16-byte LDS read in four passes of 16 lanes, and a pass is
//   not 16 consecutive lanes but the four lane quads of one half-wave whose quad index has the
//   same bit parity (quads 0, 3, 5, 6, then 1, 2, 4, 7 of each 32 lanes); a pass runs in one go
//   when its 16 addresses fall in distinct 16-byte groups modulo 256 bytes, and any collision
//   costs a second go (measured with the LDS bank-conflict counter over chosen lane patterns).
//   An A fragment is 16 pixels (2 rows x 8 columns, four 2 x 2 squares) x part g for lane group
//   g; with the layout above every pass of every tap and kernel row meets 16 distinct groups.
//   Every fragment address stays a fixed offset from the lane's base.
// While the matrix cores work on stage k, the weights of stage k+1 and (for two stages) the next
// slice's halo are in flight, their DMA instructions interleaved with the MFMAs; each stage ends
// with an explicit vmcnt wait and a barrier. The buffers are separate LDS objects used with
// compile-time parity, so the compiler adds no waits of its own between a DMA into one buffer and
// the reads of another. Tile bookkeeping is incremental and uniform, addresses are 32-bit
// offsets from per-tile bases: the VALU work per MFMA stays small.
//
// Work split: a persistent workgroup of 16 wavefronts (4 per SIMD, so the matrix core of a SIMD
// has another wavefront to serve while one waits on LDS or its DMA) per CU walks a contiguous
// run of TH x TW output tiles (runs of neighbouring tiles on one XCD) for one block of BN output
// channels; a tile is 16 row tiles of 2 x 8 pixels (each four 2 x 2 squares, so a fused MaxPool
// reduces a lane's own accumulators), and wavefront (wm, wn) of the WM x WN grid computes 16 / WM
// of them x 16 * NT channels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "../kernels.h"
#include "../runtime.h"
#include "lds_dma.h"

namespace ocr {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int RTT = 16;              // row tiles (of 16 pixels) per tile
constexpr int HMAX = 51;             // halo staging size in 1 KiB blocks (8 pixels of 32 channels)
constexpr int HPX = HMAX * 8;        // halo pixels at most
constexpr int HSP = 1632;            // units (16 bytes) of each hi / lo plane: halo rows x rs at most

// One segment: a tensor of n images of width w (output width ow, pooled pow_); every segment of
// a launch has the same height, channels and weights (the width batches of one recogniser pass).
struct C3Seg {
    const float *x;
    float *y, *yp;
    int n, w, ow, pow_, tiles_x, t0;  // t0: the segment's first tile in the launch
    int noff;                         // pool mode 3: the segment's first line in tm
};
constexpr int C3MAXSEG = 32;

struct C3Params {
    int h, cin, xcs;
    int oh, ycs;
    int poh, ypcs, pool;  // pool: 0 none, 1 = 2 x 2, 2 = 2 x 1, 3 = 2 x 1 then mean of 2 rows into tm
    float *tm;
    int tm_ntot;
    const half8 *wt;  // fragments [n-tile][slice][tap][64 lanes] of 8 halves
    int ntiles, cout, chunks;  // chunks: weight slices (twice the input's for inexact weights)
    int xchunks;               // input slices of 32 channels
    const float *bias;
    int th, tw, mx, hw, hh, rs, npx, hblocks;
    int tiles_y, tiles, nblocks, runs, nseg;
    const float4 *zero;  // 16 zero bytes (the DMA source for padding)
    C3Seg seg[C3MAXSEG];
};

__device__ inline float act3(float v, int act) {
    if (act == ACT_RELU) return fmaxf(v, 0.f);
    if (act == ACT_SIGMOID) return 1.f / (1.f + expf(-v));
    return v;
}

__device__ inline int xcd_index3(int b, int G) {
    const int q = G >> 3, rem = G & 7, x = b & 7;
    return x * q + min(x, rem) + (b >> 3);
}



// A (tile, slice) position of the workgroup's walk, all values uniform.
struct Seq {
    int t, c, tx, ty, img, sg;
};

// RC = 0: the weights stream through two stage buffers (W0, W1), one kernel row of one slice at a
// time. RC > 0 (layers of at most RC slices whose weights fit beside the halo buffers): every
// tap of every slice is copied into W0 once, a slice's three kernel rows run without a barrier
// between them, and the next slice's halo has the whole slice to land.
template <int WM, int WN, int NT, int ACT, int RC>
__global__ __launch_bounds__(64 * WM * WN, 1) void conv3_dma_kernel(C3Params p) {
    constexpr int NW = WM * WN, MT = RTT / WM;  // wavefronts; row tiles per wavefront
    constexpr int NTW = NT * WN, WBLK = 3 * NTW, NWI = (WBLK + NW - 1) / NW;
    constexpr int WRB = RC ? 9 * RC * NTW : WBLK, NRI = (WRB + NW - 1) / NW;
    constexpr int NHI = (HMAX + NW - 1) / NW;         // halo DMA instructions per wavefront and slice
    constexpr int NSI = (HPX + 16 * NW - 1) / (16 * NW);  // split items (pixel, 8 channels) per thread
    static_assert(NW == 8 || NW == 16, "8 or 16 wavefronts");
    static_assert(RTT % WM == 0 && MT % 2 == 0, "whole row-tile pairs per wavefront");
    static_assert(NWI + NHI <= 3 * MT, "a stage's DMA instructions fit its steps");
    __shared__ __align__(16) half8 W0[WRB * 64];
    __shared__ __align__(16) half8 W1[RC ? 64 : WBLK * 64];
    __shared__ __align__(16) float4 HF[HMAX * 64];  // float32 staging of the next slice
    __shared__ __align__(16) half8 HSH[HSP];        // hi plane of the current slice
    __shared__ __align__(16) half8 HSL[HSP];        // lo plane

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const int g = lane >> 4, r = lane & 15;
    const int v = xcd_index3(blockIdx.x, gridDim.x);
    const int nb = v % p.nblocks, run = v / p.nblocks;
    if (run >= p.runs) return;
    const int t_begin = int((long(run) * p.tiles) / p.runs), t_end = int((long(run + 1) * p.tiles) / p.runs);
    if (t_begin >= t_end) return;
    const int nt0 = nb * NTW, co_w = (nt0 + wn * NT) * 16;

    // This lane's pixel in each row tile: its plane unit for tap (0, 0) at kernel row 0 and its
    // square's corner.
    int abase[MT], pyb[MT], pxb[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        // Row tiles run along rows; in pool mode 3 (four output rows) down columns instead, so
        // a lane's row tiles mt and mt + 1 are the same columns' rows 0-1 and 2-3.
        const int mi = wm * MT + mt, q = r & 3;
        const int mxi = p.pool == 3 ? mi >> 1 : mi % p.mx, myi = p.pool == 3 ? mi & 1 : mi / p.mx;
        pyb[mt] = 2 * myi, pxb[mt] = 8 * mxi;
        abase[mt] = (pyb[mt] + (q >> 1)) * p.rs + (pxb[mt] + 2 * (r >> 2) + (q & 1)) * 4 + (g ^ (q & 2));
    }
    // One kernel row down flips the row parity and with it bit 1 of the lane's part: +2 or -2.
    const int kodd = (((lane >> 5) ^ (lane >> 1)) & 1) ? -2 : 2;
    // This lane's halo slot (row, column, channel part) for each halo DMA instruction; row -1
    // for padding slots. Unit U = 8 P + (u ^ ((P >> 1) & 1)) of HF holds channels 4u..4u+3 of
    // slot P = row * hw + column.
    // Packed in one register: column (bits 0-7), row (8-15), channel quad (16-18); -1: padding.
    int dhs[NHI];
#pragma unroll
    for (int i = 0; i < NHI; i++) {
        const int b = min(i * NW + wave, p.hblocks - 1), U = b * 64 + lane, P = U >> 3;
        const int hy = P / p.hw, hx = P - hy * p.hw;
        dhs[i] = P < p.npx ? hx | hy << 8 | ((U & 7) ^ ((P >> 1) & 1)) << 16 : -1;
    }
    // This thread's split items: item k of lane l in wavefront w covers pixel
    // (l & 3) + 4 (l >> 4) + 16 (w + 8 k), channels 8q..8q+7 with q = (l >> 2) & 3: the four
    // quads of every 16-byte access pass take four different parts, so the reads of HF and the
    // writes within a halo row meet distinct groups. sf: its HF unit, ss: its unit in each plane
    // (-1: none).
    int sf[NSI], ss[NSI];
#pragma unroll
    for (int k = 0; k < NSI; k++) {
        const int P = (lane & 3) + 4 * (lane >> 4) + 16 * (wave + NW * k), q = (lane >> 2) & 3;
        const int hy = P / p.hw, hx = P - hy * p.hw;
        sf[k] = 8 * P + ((2 * q) ^ ((P >> 1) & 1));
        ss[k] = P < p.npx ? hy * p.rs + hx * 4 + (q ^ ((hy & 1) << 1)) : -1;
    }
    // Bias of this lane's output channel in each n-tile.
    const int co_l = co_w + r;
    float bv[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) bv[j] = (p.bias && co_l + 16 * j < p.cout) ? p.bias[co_l + 16 * j] : 0.f;

    auto advance = [&](Seq s) __attribute__((always_inline)) {
        if (++s.c == p.chunks) {
            s.c = 0, s.t++;
            if (++s.tx == p.seg[s.sg].tiles_x) {
                s.tx = 0;
                if (++s.ty == p.tiles_y) {
                    s.ty = 0;
                    if (++s.img == p.seg[s.sg].n) s.img = 0, s.sg = min(s.sg + 1, C3MAXSEG - 1);
                }
            }
        }
        return s;
    };
    Seq cur;
    cur.sg = 0;
    while (cur.sg + 1 < p.nseg && t_begin >= p.seg[cur.sg + 1].t0) cur.sg++;
    {
        const int l = t_begin - p.seg[cur.sg].t0, tx_n = p.seg[cur.sg].tiles_x;
        cur.t = t_begin, cur.c = 0, cur.tx = l % tx_n;
        cur.ty = (l / tx_n) % p.tiles_y, cur.img = l / (tx_n * p.tiles_y);
    }

    // Weights of slice c, kernel row ky: block b = kx * NTW + j (n-tile nt0 + j); instruction i.
    // The lane's byte offset of each instruction's fragment is fixed (n-tile, tap column, lane);
    // a stage only moves the uniform base by its slice and kernel row. An n-tile past the last
    // (16-channel layers in a 32-channel block) reads the last one's weights: its outputs are
    // never stored.
    unsigned woff[NWI];
#pragma unroll
    for (int i = 0; i < NWI; i++) {
        const int b = min(i * NW + wave, WBLK - 1), kx = b / NTW, j = b - kx * NTW, nt = min(nt0 + j, p.ntiles - 1);
        woff[i] = (unsigned(nt * p.chunks * 9 + kx) * 64u + unsigned(lane)) * 16u;
    }
    // LDS byte addresses of the DMA destinations (the copies take them, not pointers).
    const unsigned w0a = lds_addr(W0), w1a = lds_addr(W1), hfa = lds_addr(HF);
    auto dma_w = [&](unsigned dst, int c, int ky, int i) __attribute__((always_inline)) {
        const int b = min(i * NW + wave, WBLK - 1);
        const char *base = reinterpret_cast<const char *>(p.wt) + size_t(c * 9 + ky * 3) * 1024;
        dma16s_to(base, woff[i], dst + unsigned(b) * 1024u);
    };
    // The halo of a position: its image's slice base, corner and width, computed once for the
    // position's NHI copies; instruction i copies this lane's slot (zeros outside the image and
    // past the input channels), the choice made by a select rather than a branch.
    struct Halo {
        const float *base;
        int iy0, ix0, w, cleft;
    };
    // Weight slice c reads input slice c, or c - xchunks for the remainder slices of inexact
    // weights (the input is walked a second time against them).
    auto halo_of = [&](const Seq &s) __attribute__((always_inline)) {
        const C3Seg &sd = p.seg[s.sg];
        const int ci = s.c >= p.xchunks ? s.c - p.xchunks : s.c;
        return Halo{sd.x + size_t(s.img) * p.h * sd.w * p.xcs + ci * 32, s.ty * p.th - 1, s.tx * p.tw - 1, sd.w,
                    p.cin - ci * 32};
    };
    auto dma_h = [&](const Halo &hl, int i) __attribute__((always_inline)) {
        const int b = min(i * NW + wave, p.hblocks - 1);
        const int d = dhs[i], ch = 4 * ((d >> 16) & 7);
        const int iy = hl.iy0 + ((d >> 8) & 255), ix = hl.ix0 + (d & 255);
        const bool ok = d >= 0 && unsigned(iy) < unsigned(p.h) && unsigned(ix) < unsigned(hl.w) && ch < hl.cleft;
        const int off = ok ? (iy * hl.w + ix) * p.xcs + ch : 0;
        const void *src = ok ? static_cast<const void *>(hl.base + unsigned(off)) : static_cast<const void *>(p.zero);
        dma16_to(src, hfa + unsigned(b) * 1024u);
    };
    // HF -> HSH / HSL, once a slice: hi and lo of part q (channels 8q..8q+7) of a pixel at the
    // same unit of each plane; lo = x - hi rounded to float16 (x = hi + lo to about 2^-22).
    auto split = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < NSI; k++) {
            if (ss[k] < 0) continue;
            const float4 a = HF[sf[k]], b = HF[sf[k] ^ 1];
            const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            half8 hi, lo;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                hi[e] = (_Float16)xs[e];
                lo[e] = (_Float16)__builtin_fmaf(-1.f, (float)hi[e], xs[e]);
            }
            HSH[ss[k]] = hi;
            HSL[ss[k]] = lo;
        }
    };

    floatx4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int j = 0; j < NT; j++) acc[mt][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // One kernel row of one slice: 3 taps x MT row tiles x NT n-tiles x (hi, lo), as 12 steps
    // (tap, row tile). Each step's A fragments (and at a new tap its B fragments) are read one
    // step ahead into a second register set; `issue(step)` puts this step's share of the next
    // stage's DMA between the MFMAs.
    auto compute = [&](const half8 *Wb, int ky, auto &&issue) __attribute__((always_inline)) {
        int base[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            base[mt] = abase[mt] + ky * p.rs + (ky & 1 ? kodd : 0);
            asm volatile("" : "+v"(base[mt]));  // per stage, not hoisted out of the stage loop
        }
        half8 ah[2], al[2], bb[2][NT];
        auto read_a = [&](int kx, int mt, half8 &hi, half8 &lo) __attribute__((always_inline)) {
            hi = HSH[base[mt] + kx * 4];
            lo = HSL[base[mt] + kx * 4];
        };
        auto read_b = [&](int kx, half8 (&b)[NT]) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < NT; j++) b[j] = Wb[(kx * NTW + wn * NT + j) * 64 + lane];
        };
        read_b(0, bb[0]);
        read_a(0, 0, ah[0], al[0]);
#pragma unroll
        for (int st = 0; st < 3 * MT; st++) {
            const int kx = st / MT, mt = st % MT, ca = st & 1, cb = kx & 1;
            issue(st);
            if (st + 1 < 3 * MT) {
                const int kx1 = (st + 1) / MT, mt1 = (st + 1) % MT;
                if (mt1 == 0) read_b(kx1, bb[cb ^ 1]);
                read_a(kx1, mt1, ah[ca ^ 1], al[ca ^ 1]);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < NT; j++) acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[ca], bb[cb][j], acc[mt][j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < NT; j++) acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[ca], bb[cb][j], acc[mt][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // The tile's outputs: bias, activation, then the full output (when p.y is set) and the
    // pooled output (POOL 1: 2 x 2, 2: 2 x 1). Offsets are 32-bit from the tile's corner; CHECK
    // bounds-checks every store (tiles on the image's or the channels' edge).
    auto epi = [&](const Seq &s, auto POOLc, auto CHECKc) __attribute__((always_inline)) {
        constexpr int POOL = decltype(POOLc)::value;
        constexpr bool CHECK = decltype(CHECKc)::value;
        const int oy0 = s.ty * p.th, ox0 = s.tx * p.tw;
        const C3Seg &sd = p.seg[s.sg];
        const int ow = sd.ow, pow_ = sd.pow_;
        float *yt = sd.y ? sd.y + (size_t(s.img) * p.oh * ow + size_t(oy0) * ow + ox0) * p.ycs : nullptr;
        float *pt = nullptr;
        if (POOL == 1) pt = sd.yp + (size_t(s.img) * p.poh * pow_ + size_t(oy0 / 2) * pow_ + ox0 / 2) * p.ypcs;
        if (POOL == 2) pt = sd.yp + (size_t(s.img) * p.poh * pow_ + size_t(oy0 / 2) * pow_ + ox0) * p.ypcs;
        if (POOL == 3) {
            // Row tiles mt (rows 0-1) and mt + 1 (rows 2-3) of the same columns: max over each
            // pair of rows, then the mean of the two maxima, summed in row order as the
            // average pool does.
            const size_t line = size_t(sd.noff + s.img);
#pragma unroll
            for (int mt = 0; mt < MT; mt += 2) {
                const int t = ox0 + pxb[mt] + 2 * g;
#pragma unroll
                for (int j = 0; j < NT; j++) {
                    float v[4], u[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        v[i] = act3(acc[mt][j][i] + bv[j], ACT);
                        u[i] = act3(acc[mt + 1][j][i] + bv[j], ACT);
                    }
                    acc[mt][j] = floatx4{0.f, 0.f, 0.f, 0.f};
                    acc[mt + 1][j] = floatx4{0.f, 0.f, 0.f, 0.f};
                    const int co = co_l + 16 * j;
                    if (CHECK && co >= p.cout) continue;
                    float *dst = p.tm + (size_t(t) * p.tm_ntot + line) * p.cout + co;
                    if (!CHECK || t < ow) dst[0] = (fmaxf(v[0], v[2]) + fmaxf(u[0], u[2])) / 2.f;
                    if (!CHECK || t + 1 < ow)
                        dst[size_t(p.tm_ntot) * p.cout] = (fmaxf(v[1], v[3]) + fmaxf(u[1], u[3])) / 2.f;
                }
            }
            return;
        }
        // The lane's parts of the offsets, computed here (not kept live across the tile loop).
        int lf = 2 * g * p.ycs + co_l, lp = (POOL == 1 ? g : 2 * g) * p.ypcs + co_l;
        asm volatile("" : "+v"(lf), "+v"(lp));
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int dy = pyb[mt], dx = pxb[mt] + 2 * g;
            const unsigned fo = unsigned((dy * ow + pxb[mt]) * p.ycs + lf);
            const unsigned po = POOL == 1 ? unsigned(((dy >> 1) * pow_ + (pxb[mt] >> 1)) * p.ypcs + lp)
                                          : unsigned(((dy >> 1) * pow_ + pxb[mt]) * p.ypcs + lp);
#pragma unroll
            for (int j = 0; j < NT; j++) {
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = act3(acc[mt][j][i] + bv[j], ACT);
                acc[mt][j] = floatx4{0.f, 0.f, 0.f, 0.f};
                const bool cok = !CHECK || co_l + 16 * j < p.cout;
                if (yt) {
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const bool in = !CHECK || (cok && oy0 + dy + (i >> 1) < p.oh && ox0 + dx + (i & 1) < ow);
                        if (in) yt[fo + unsigned(((i >> 1) * ow + (i & 1)) * p.ycs + 16 * j)] = v[i];
                    }
                }
                if (POOL == 1) {
                    const bool in = !CHECK || (cok && (oy0 + dy) / 2 < p.poh && (ox0 + dx) / 2 < pow_);
                    if (in) pt[po + 16 * j] = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
                }
                if (POOL == 2) {
                    const bool iny = !CHECK || (cok && (oy0 + dy) / 2 < p.poh);
                    if (iny && (!CHECK || ox0 + dx < pow_)) pt[po + 16 * j] = fmaxf(v[0], v[2]);
                    if (iny && (!CHECK || ox0 + dx + 1 < pow_)) pt[po + unsigned(p.ypcs) + 16 * j] = fmaxf(v[1], v[3]);
                }
            }
        }
    };
    auto epilogue = [&](const Seq &s) __attribute__((always_inline)) {
        const int oy0 = s.ty * p.th, ox0 = s.tx * p.tw;
        const C3Seg &sd = p.seg[s.sg];
        const bool cin_ = co_w + 16 * NT <= p.cout && (!sd.y || (oy0 + p.th <= p.oh && ox0 + p.tw <= sd.ow));
        auto run = [&](auto POOLc, bool inside) __attribute__((always_inline)) {
            if (inside) epi(s, POOLc, std::false_type{});
            else epi(s, POOLc, std::true_type{});
        };
        if (p.pool == 3)
            run(std::integral_constant<int, 3>{}, cin_ && ox0 + p.tw <= sd.ow);
        else if (p.pool == 1)
            run(std::integral_constant<int, 1>{}, cin_ && (oy0 + p.th) / 2 <= p.poh && (ox0 + p.tw) / 2 <= sd.pow_);
        else if (p.pool == 2)
            run(std::integral_constant<int, 2>{}, cin_ && (oy0 + p.th) / 2 <= p.poh && ox0 + p.tw <= sd.pow_);
        else
            run(std::integral_constant<int, 0>{}, cin_);
    };

    Seq nxt = advance(cur);
    // Resident weights: kernel row KY of the current slice. The next position's halo goes out in
    // the first row's steps; at the third the tile's outputs are stored (last slice), and after
    // one wait and barrier the halo becomes the next slice's hi / lo.
    auto stage_r = [&](auto KYc) __attribute__((always_inline)) -> bool {
        constexpr int KY = decltype(KYc)::value;
        const bool more = nxt.t < t_end, hnext = KY == 0 && more;
        Halo hn{};
        if (hnext) hn = halo_of(nxt);
        compute(W0 + (cur.c * 3 + KY) * 3 * NTW * 64, KY, [&](int st) __attribute__((always_inline)) {
            if (st < NHI && hnext) dma_h(hn, st);
        });
        if (KY < 2) return true;
        // The wait is for the halo; the outputs are stored after it (stores count in vmcnt too)
        // and stay in flight through the split and the next slice.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (cur.c == p.chunks - 1) epilogue(cur);
        lds_barrier();
        if (!more) return false;
        split();
        lds_barrier();
        cur = nxt;
        nxt = advance(nxt);
        return true;
    };

    // Stage (position cur, kernel row KY); weight buffer (KY + HP) & 1 with HP the parity of the
    // slice sequence (three stages a slice). Returns false after the last stage.
    auto stage = [&](auto KYc, auto HPc) __attribute__((always_inline)) -> bool {
        constexpr int KY = decltype(KYc)::value, HP = decltype(HPc)::value;
        constexpr int WP = (KY + HP) & 1;
        half8 *Wc = WP ? W1 : W0;
        const unsigned Wna = WP ? w0a : w1a;
        const bool more = nxt.t < t_end;
        // The next stage's weights (steps 0..NWI-1), then at a slice's first row the next slice's
        // halo (steps NWI..NWI+NHI-1), one DMA instruction per step between the MFMAs.
        const bool wnext = KY < 2 || more, hnext = KY == 0 && more;
        const int wc = KY < 2 ? cur.c : nxt.c, wky = KY < 2 ? KY + 1 : 0;
        Halo hn{};
        if (hnext) hn = halo_of(nxt);
        compute(Wc, KY, [&](int st) __attribute__((always_inline)) {
            if (st < NWI) {
                if (wnext) dma_w(Wna, wc, wky, st);
            } else if (st < NWI + NHI) {
                if (hnext) dma_h(hn, st - NWI);
            }
        });
        if (hnext) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NHI) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (KY == 2 && cur.c == p.chunks - 1) epilogue(cur);  // stored after the wait, left in flight
        lds_barrier();
        if (KY == 2) {
            if (!more) return false;
            split();  // the next slice's halo, landed in HF, becomes its hi / lo
            lds_barrier();
            cur = nxt;
            nxt = advance(nxt);
        }
        return true;
    };

    if constexpr (RC > 0) {
        // Every weight block of the layer's slices: block ((c * 3 + ky) * 3 + kx) * NTW + j.
        const int nwb = 9 * p.chunks * NTW;
#pragma unroll
        for (int i = 0; i < NRI; i++) {
            const int b = min(i * NW + wave, nwb - 1), j = b % NTW, tap = b / NTW;
            const int c = tap / 9, t9 = tap - c * 9, nt = min(nt0 + j, p.ntiles - 1);
            dma16_to(p.wt + (size_t(nt * p.chunks + c) * 9 + t9) * 64 + lane, w0a + unsigned(b) * 1024u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NWI; i++) dma_w(w0a, 0, 0, i);
    }
    {
        const Halo h0 = halo_of(cur);
#pragma unroll
        for (int i = 0; i < NHI; i++) dma_h(h0, i);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();
    split();
    lds_barrier();
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    if constexpr (RC > 0) {
        for (;;) {
            if (!stage_r(I0{}) || !stage_r(I1{}) || !stage_r(I2{})) break;
        }
    } else {
        for (;;) {
            if (!stage(I0{}, I0{}) || !stage(I1{}, I0{}) || !stage(I2{}, I0{})) break;
            if (!stage(I0{}, I1{}) || !stage(I1{}, I1{}) || !stage(I2{}, I1{})) break;
        }
    }
}

int cu_count3() {
    static int n = 0;
    if (!n) {
        int dev = 0;
        OCR_HIP(hipGetDevice(&dev));
        OCR_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        if (n <= 0) n = 256;
    }
    return n;
}

const float4 *zero_block() { return static_cast<const float4 *>(zero_block64()); }

}  // namespace

namespace {

// The checks of one segment; pool mode out (0 none, 1 = 2 x 2, 2 = 2 x 1), -1 when not taken.
int c3_accepts(const ConvArgs &a) {
    const ConvPack &pk = a.pk;
    if (!a.wt_frag || a.nchw || a.in_scale || a.affine || a.amax_part || a.res || a.rows) return -1;
    if (pk.kh != 3 || pk.kw != 3 || a.pt != 1 || a.pl != 1 || pk.cin != a.x.c || pk.cout != a.y.c) return -1;
    if (a.y.n != a.x.n || a.y.h != a.x.h || a.y.w != a.x.w || a.y_px || a.y_row || a.y_img) return -1;
    if (a.x.c % 4 || a.x.cs % 4 || (reinterpret_cast<uintptr_t>(a.x.p) & 15)) return -1;
    if (a.act != ACT_NONE && a.act != ACT_RELU && a.act != ACT_SIGMOID) return -1;
    // 32-bit offsets within one image of the input, the output and the pooled output.
    if (double(a.x.h) * a.x.w * a.x.cs >= 2147483647.0 || double(a.y.h) * a.y.w * a.y.cs >= 2147483647.0) return -1;
    if (a.tm) {
        // Max pool (2, 1) and the mean of the two pooled rows, time-major; nothing else written.
        if (a.ph != 2 || a.pw != 1 || a.y.h != 4 || a.ypool.p || a.keep_full || a.tm_ntot < 1 || a.tm_noff < 0 ||
            a.tm_noff + a.y.n > a.tm_ntot)
            return -1;
        return 3;
    }
    if (!a.ypool.p) return 0;
    int pool;
    if (a.ph == 2 && a.pw == 2) pool = 1;
    else if (a.ph == 2 && a.pw == 1) pool = 2;
    else return -1;
    if (a.ypool.h != a.y.h / a.ph || a.ypool.w != a.y.w / a.pw || a.ypool.c != a.y.c || a.ypool.n != a.y.n)
        fail("conv3x3_dma: pooled output shape");
    return pool;
}

// Segments [0, count) of one launch (count <= C3MAXSEG), all accepted and alike.
void c3_launch(const ConvArgs *args, int count, int pool, hipStream_t s) {
    const ConvArgs &a = args[0];
    const ConvPack &pk = a.pk;
    const int cout = a.y.c;
    const int nt_max = cout > 64 ? 4 : cout > 32 ? 2 : 1;
    int nt = nt_max;
    C3Params p{};
    p.h = a.x.h;
    p.cin = a.x.c;
    p.xcs = a.x.cs;
    p.oh = a.y.h;
    p.ycs = a.y.cs;
    p.poh = a.ypool.h;
    p.ypcs = a.ypool.cs;
    p.pool = pool;
    p.wt = reinterpret_cast<const half8 *>(a.wt_frag);
    p.ntiles = pk.nblocks * pk.bn / 16;
    p.cout = cout;
    p.chunks = pk.frag_chunks();
    p.xchunks = pk.chunks;
    p.bias = a.bias;
    // Tile shape (16 blocks of 2 x 8 pixels) and channel block (32 nt channels) chosen
    // together. A workgroup walks ceil(tiles / runs) tiles, runs = CUs / blocks, so the launch
    // takes that many rounds of a tile each; a tile costs about (1.5 + nt) units (per-stage
    // overhead, then matrix work per 32 channels: measured on the detector's 256 -> 128 layer) times
    // its halo's share of extra pixels. Few tiles (the detector's deep levels at a few pages)
    // favour narrower blocks and shapes whose count fits one round; many tiles the widest block.
    p.tm = a.tm;
    p.tm_ntot = a.tm_ntot;
    const int cus = cu_count3();
    double best = 1e300;
    bool fits = false;
    for (int mxc : {1, 2, 4, 8}) {
        if (pool == 3 && mxc != 8) continue;  // four rows: the whole output height in one tile
        const int tw = 8 * mxc, th = 2 * (16 / mxc), hw = tw + 2, hh = th + 2;
        const int rs = (4 * hw + 15) / 16 * 16;  // a multiple of 16 units
        if (hh * hw > HPX || hh * rs > HSP) continue;
        fits = true;
        double ntl = 0;
        for (int k = 0; k < count; k++)
            ntl += double(args[k].y.n) * ((p.oh + th - 1) / th) * ((args[k].y.w + tw - 1) / tw);
        if (ntl < 1) continue;
        for (int q = nt_max; q >= 1; q /= 2) {
            const double blocks = (cout + 32 * q - 1) / (32 * q);
            const double runs = std::max(1.0, std::min(ntl, std::floor(cus / blocks)));
            const double cost = std::ceil(ntl / runs) * (1.5 + q) * double(hh * hw) / (th * tw);
            if (cost < best) best = cost, p.tw = tw, p.th = th, p.mx = mxc, p.rs = rs, nt = q;
        }
    }
    if (!fits) fail("conv3x3_dma: no tile fits");
    if (best == 1e300) return;  // no output pixels
    p.hw = p.tw + 2;
    p.hh = p.th + 2;
    p.npx = p.hh * p.hw;
    p.hblocks = (p.npx + 7) / 8;
    p.tiles_y = (p.oh + p.th - 1) / p.th;
    double tiles = 0, flops = 0, bytes = 2.0 * double(pk.frag_halves());
    for (int k = 0; k < count; k++) {
        const ConvArgs &b = args[k];
        C3Seg &sg = p.seg[k];
        sg.x = b.x.p;
        sg.y = (b.ypool.p && !b.keep_full) || pool == 3 ? nullptr : b.y.p;
        sg.yp = b.ypool.p;
        sg.noff = b.tm_noff;
        sg.n = b.x.n;
        sg.w = b.x.w;
        sg.ow = b.y.w;
        sg.pow_ = b.ypool.w;
        sg.tiles_x = (sg.ow + p.tw - 1) / p.tw;
        sg.t0 = int(tiles);
        tiles += double(sg.tiles_x) * p.tiles_y * sg.n;
        flops += 2.0 * b.y.n * b.y.h * b.y.w * cout * p.cin * 9;
        // Algorithmic bytes: the input once and every output actually stored.
        double out = 0;
        if (sg.y) out += double(b.y.n) * b.y.h * b.y.w;
        if (sg.yp) out += double(b.ypool.n) * b.ypool.h * b.ypool.w;
        if (pool == 3) out += double(b.y.n) * b.y.w;
        bytes += 4.0 * (double(b.x.n) * b.x.h * b.x.w * p.cin + out * cout);
        if (tiles > 0x7fffffff) fail("conv3x3_dma: too many tiles");
    }
    p.nseg = count;
    p.tiles = int(tiles);
    if (p.tiles == 0) return;
    const int bn = 32 * nt;
    p.nblocks = (cout + bn - 1) / bn;
    p.runs = std::max(1, std::min(p.tiles, cus / p.nblocks));
    p.zero = zero_block();
    const int grid = p.runs * p.nblocks;
    ProbeScope probe("conv3x3_dma", s, flops, bytes);
    auto launch = [&](auto ACTc) {
        constexpr int A = decltype(ACTc)::value;
        // 16 wavefronts (4 a SIMD): 128-channel blocks as 4 x 4 wavefronts of 2 n-tiles, 64-channel
        // blocks as 4 x 4 of one, 32-channel blocks as 8 x 2 of one (two row tiles each).
        const dim3 gd{unsigned(grid)}, bd{1024};
        if (nt == 4) hipLaunchKernelGGL((conv3_dma_kernel<4, 4, 2, A, 0>), gd, bd, 0, s, p);
        else if (nt == 2 && p.chunks == 1) hipLaunchKernelGGL((conv3_dma_kernel<4, 4, 1, A, 1>), gd, bd, 0, s, p);
        else if (nt == 2) hipLaunchKernelGGL((conv3_dma_kernel<4, 4, 1, A, 0>), gd, bd, 0, s, p);
        else if (p.chunks == 1) hipLaunchKernelGGL((conv3_dma_kernel<8, 2, 1, A, 1>), gd, bd, 0, s, p);
        else if (p.chunks == 2) hipLaunchKernelGGL((conv3_dma_kernel<8, 2, 1, A, 2>), gd, bd, 0, s, p);
        else hipLaunchKernelGGL((conv3_dma_kernel<8, 2, 1, A, 0>), gd, bd, 0, s, p);
    };
    if (a.act == ACT_RELU) launch(std::integral_constant<int, ACT_RELU>{});
    else if (a.act == ACT_SIGMOID) launch(std::integral_constant<int, ACT_SIGMOID>{});
    else launch(std::integral_constant<int, ACT_NONE>{});
    OCR_HIP(hipGetLastError());
}

}  // namespace

bool conv3x3_dma(const ConvArgs &a, hipStream_t s) {
    const int pool = c3_accepts(a);
    if (pool < 0) return false;
    c3_launch(&a, 1, pool, s);
    return true;
}

bool conv3x3_dma_multi(const ConvArgs *args, int count, hipStream_t s) {
    if (count < 1) return true;
    const ConvArgs &a = args[0];
    const int pool = c3_accepts(a);
    if (pool < 0) return false;
    for (int k = 1; k < count; k++) {
        const ConvArgs &b = args[k];
        if (c3_accepts(b) != pool || b.tm != a.tm || b.tm_ntot != a.tm_ntot || b.wt_frag != a.wt_frag ||
            b.bias != a.bias || b.act != a.act ||
            b.x.h != a.x.h || b.x.c != a.x.c || b.x.cs != a.x.cs || b.y.c != a.y.c || b.y.cs != a.y.cs ||
            b.ypool.cs != a.ypool.cs || (b.ypool.p && !b.keep_full) != (a.ypool.p && !a.keep_full) ||
            b.pk.chunks != a.pk.chunks || b.pk.exact != a.pk.exact)
            return false;
    }
    for (int k = 0; k < count; k += C3MAXSEG) c3_launch(args + k, std::min(C3MAXSEG, count - k), pool, s);
    return true;
}

}  // namespace ocr
