// 3 x 3, pad 1 convolution of a one-channel image (the first layer of the ocrs detector and
// recogniser) on the matrix cores, with bias, activation and an optional fused 2 x 2 MaxPool:
// semantics of the reference's conv_direct program (src/gpu.rs:385-422).
//
// One v_mfma_f32_16x16x32_f16 gives 16 output channels of 16 pixels: the K = 32 side holds the
// pixel's 3 x 3 patch twice, as float16 hi parts (k 0-15) and float16 remainders lo (k 16-31) of
// the float32 input (x = hi + lo to about 2^-22), against the exact float16 weights. Each half
// holds the patch's three rows as (left, centre, right, 0) quadruples and a fourth quadruple the
// zero weights cancel. The weights are the A operand, so a lane's 4 accumulators are 4
// neighbouring output channels of one pixel and leave as one 16-byte NHWC store; for a pooled-only
// output the patches are the A operand instead, so a lane's 4 accumulators are one channel of a
// 2 x 2 window.
//
// A workgroup (4 wavefronts) owns a 16 x 64 pixel tile. The input window (18 x 66) is loaded once,
// then rewritten in LDS as a hi and a lo plane of row quadruples: entry (row, x) holds window
// values x, x + 1, x + 2 of that row, so lane (g, r), which holds k = 8 g .. 8 g + 7 of pixel r,
// reads two entries (rows py + 2 (g & 1) and the next) of plane g >> 1 with one aligned 16-byte
// LDS read. Planes and rows are spaced so that the 64 lanes of a read touch each bank at most
// twice. A wavefront takes groups of 16 pixels laid out as four 2 x 2 squares (a fused pool is a
// max over 4 neighbouring lanes, or over a lane's own accumulators in the pooled-only form).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>

#include "../kernels.h"
#include "../runtime.h"

namespace ocr {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int TY = 16, TX = 64;  // pixels of a tile
constexpr int WW = TX + 2;       // the input window: TY + 2 rows of WW values
constexpr int WROWS = TY + 2;
constexpr int QROWS = TY + 3;    // quadruple rows (the last one zero: read against zero weights)
constexpr int QSTRIDE = 72;      // quadruples per row: consecutive rows 16 banks apart
constexpr int QPLANE = QROWS * QSTRIDE;

template <int ACT> __device__ inline float act1(float v) {
    if (ACT == ACT_RELU) return fmaxf(v, 0.f);
    if (ACT == ACT_SIGMOID) return 1.f / (1.f + expf(-v));
    return v;
}

// Lane l receives the value of lane l ^ 1 (quad_perm [1,0,3,2]) or lane l ^ 2 ([2,3,0,1]).
__device__ inline float xor1(float v) { return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false)); }
__device__ inline float xor2(float v) { return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false)); }

// One launch covers up to C1MAXSEG inputs of the same height (the width batches of a
// recognition pass): segment s owns blocks [blk0, blk0 + tiles_x * tiles_y * n).
struct C1Seg {
    const float *x;
    float *y, *yp;
    int n, w, ow, pow_, tiles_x, blk0;
};
constexpr int C1MAXSEG = 32;
struct C1Params {
    int h, xcs, oh, ycs, poh, ypcs, tiles_y, nseg;
    const half8 *wf;
    const float *bias;
    C1Seg seg[C1MAXSEG];
};

constexpr int FILL = (WROWS * WW + 255) / 256;  // window values a thread loads

// POOL 0: the output y only; 1: the 2 x 2 pooled output only (in yp); 2: both, the full output
// in y and the pooled one in yp.
template <int NT, int POOL, int ACT>
__global__ __launch_bounds__(256) void conv1_kernel(const C1Params p) {
    __shared__ float s_win[WROWS * WW];
    __shared__ uint2 s_q[2 * QPLANE];  // hi plane, then lo plane; an entry is 4 halves
    static_assert(TY / 2 * (TX / 8) % 8 == 0, "groups come in pairs per wavefront");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r = lane & 15;
    int sg = 0;
    while (sg + 1 < p.nseg && int(blockIdx.x) >= p.seg[sg + 1].blk0) sg++;
    const C1Seg &sd = p.seg[sg];
    const int h = p.h, w = sd.w, xcs = p.xcs;
    const int b = int(blockIdx.x) - sd.blk0, per_img = sd.tiles_x * p.tiles_y;
    const int img = b / per_img, tb = b - img * per_img;
    const int ty = tb / sd.tiles_x, tx = tb - ty * sd.tiles_x;
    const int y0 = ty * TY, x0 = tx * TX;
    const float *xi = sd.x + size_t(img) * h * w * xcs;
    // The input window (rows y0 - 1 .., columns x0 - 1 ..), zero outside the image; every load
    // is issued before the first LDS write.
    float v[FILL];
#pragma unroll
    for (int k = 0; k < FILL; k++) {
        const int i = tid + 256 * k;
        const int wy = i / WW, wx = i - wy * WW;
        const int iy = y0 - 1 + wy, ix = x0 - 1 + wx;
        v[k] = 0.f;
        if (i < WROWS * WW && iy >= 0 && iy < h && ix >= 0 && ix < w) v[k] = xi[(size_t(iy) * w + ix) * xcs];
    }
#pragma unroll
    for (int k = 0; k < FILL; k++) {
        const int i = tid + 256 * k;
        if (i < WROWS * WW) s_win[i] = v[k];
    }
    __syncthreads();
    // The quadruples: (x, x + 1, x + 2, 0) of each window row, split into hi and lo.
    for (int e = tid; e < QROWS * TX; e += 256) {
        const int row = e / TX, x = e - row * TX;
        float t[3] = {0.f, 0.f, 0.f};
        if (row < WROWS)
#pragma unroll
            for (int c = 0; c < 3; c++) t[c] = s_win[row * WW + x + c];
        _Float16 hi[4], lo[4];
#pragma unroll
        for (int c = 0; c < 3; c++) {
            hi[c] = (_Float16)t[c];
            lo[c] = (_Float16)(t[c] - (float)hi[c]);
        }
        hi[3] = lo[3] = (_Float16)0.f;
        uint2 qh, ql;
        __builtin_memcpy(&qh, hi, 8);
        __builtin_memcpy(&ql, lo, 8);
        s_q[row * QSTRIDE + x] = qh;
        s_q[QPLANE + row * QSTRIDE + x] = ql;
    }
    // Weights of the NT 16-channel tiles (the A operand, or B in the pooled-only form), bias of
    // this lane's 4 channels per tile.
    half8 a[NT];
    float4 b4[NT];
    float bc[NT];  // the bias of channel 16 j + r (pooled-only form)
#pragma unroll
    for (int j = 0; j < NT; j++) {
        a[j] = p.wf[j * 64 + lane];
        const int co = j * 16 + 4 * g;
        b4[j] = p.bias ? *reinterpret_cast<const float4 *>(p.bias + co) : make_float4(0.f, 0.f, 0.f, 0.f);
        bc[j] = p.bias ? p.bias[j * 16 + r] : 0.f;
    }
    __syncthreads();
    // This lane's pixel in a group: square r >> 2 (2 columns each), position r & 3.
    const int q = r & 3, sq = r >> 2;
    const int pdy = q >> 1, pdx = 2 * sq + (q & 1);
    // This lane's plane (hi for g < 2) and first quadruple row (patch row 0, or row 2 for odd g).
    const int lbase = (g >= 2 ? QPLANE : 0) + ((g & 1) ? 2 * QSTRIDE : 0) + pdy * QSTRIDE + pdx;
    constexpr int NG = TY / 2 * (TX / 8);  // groups of 16 pixels in the tile
    const int oh = p.oh, ow = sd.ow, poh = p.poh, pow_ = sd.pow_;
    float *const y = sd.y, *const yp = sd.yp;
    // Two groups at a time (G and G + 4): the second's MFMAs issue while the first's results
    // are on their way.
    for (int G0 = wave; G0 < NG; G0 += 8) {
        floatx4 acc[2][NT];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int G = G0 + 4 * u;
            const int gy = G / (TX / 8), gx = G - gy * (TX / 8);
            const uint2 *src = s_q + lbase + 2 * gy * QSTRIDE + 8 * gx;
            const uint4 q4 = make_uint4(src[0].x, src[0].y, src[QSTRIDE].x, src[QSTRIDE].y);
            half8 bf;
            __builtin_memcpy(&bf, &q4, 16);
            // Pooled output only: the patches are the A operand, so a lane's 4 accumulators are
            // one channel of the 4 pixels of one 2 x 2 window and the pool is a max over them.
#pragma unroll
            for (int j = 0; j < NT; j++)
                acc[u][j] = POOL == 1
                                ? __builtin_amdgcn_mfma_f32_16x16x32_f16(bf, a[j], floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0)
                                : __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], bf, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int G = G0 + 4 * u;
            const int gy = G / (TX / 8), gx = G - gy * (TX / 8);
            if (POOL == 1) {
                // Lane (g, r): channel 16 j + r of pooled pixel (y0 / 2 + gy, x0 / 2 + 4 gx + g);
                // max(relu(v + b)) = relu(max(v) + b) exactly (rounded addition is monotone).
                const int qy = (y0 >> 1) + gy, qx = (x0 >> 1) + 4 * gx + g;
                if (qy < poh && qx < pow_) {
                    float *dst = yp + ((size_t(img) * poh + qy) * pow_ + qx) * p.ypcs + r;
#pragma unroll
                    for (int j = 0; j < NT; j++) {
                        const floatx4 v = acc[u][j];
                        if (ACT == ACT_SIGMOID)
                            dst[16 * j] = fmaxf(fmaxf(act1<ACT>(v[0] + bc[j]), act1<ACT>(v[1] + bc[j])),
                                                fmaxf(act1<ACT>(v[2] + bc[j]), act1<ACT>(v[3] + bc[j])));
                        else
                            dst[16 * j] = act1<ACT>(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])) + bc[j]);
                    }
                }
                continue;
            }
            // Output: lane (g, r) holds channels 16 j + 4 g .. + 3 of the group's pixel r.
            const int oy = y0 + 2 * gy + pdy, ox = x0 + 8 * gx + pdx;
#pragma unroll
            for (int j = 0; j < NT; j++) {
                float o[4] = {act1<ACT>(acc[u][j][0] + b4[j].x), act1<ACT>(acc[u][j][1] + b4[j].y),
                              act1<ACT>(acc[u][j][2] + b4[j].z), act1<ACT>(acc[u][j][3] + b4[j].w)};
                if (POOL != 1 && oy < oh && ox < ow)
                    *reinterpret_cast<float4 *>(y + ((size_t(img) * oh + oy) * ow + ox) * p.ycs + j * 16 + 4 * g) =
                        make_float4(o[0], o[1], o[2], o[3]);
                if (POOL) {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        o[e] = fmaxf(o[e], xor1(o[e]));
                        o[e] = fmaxf(o[e], xor2(o[e]));
                    }
                    const int qy = oy >> 1, qx = ox >> 1;
                    if (q == 0 && qy < poh && qx < pow_)
                        *reinterpret_cast<float4 *>(yp + ((size_t(img) * poh + qy) * pow_ + qx) * p.ypcs + j * 16 +
                                                    4 * g) = make_float4(o[0], o[1], o[2], o[3]);
                }
            }
        }
    }
}

}  // namespace

void pack_conv1_frags(const float *w, int cout, uint16_t *frag) {
    // frag [cout / 16][64 lanes][8]: lane (g, r) holds k = 8 g .. 8 g + 7 of channel 16 t + r.
    // Each 16-k half (hi side, lo side) is rows 0, 1, 2 of the 3 x 3 kernel as (left, centre,
    // right, 0) quadruples, then a zero quadruple.
    for (int t = 0; t < cout / 16; t++)
        for (int lane = 0; lane < 64; lane++)
            for (int e = 0; e < 8; e++) {
                const int g = lane >> 4, r = lane & 15;
                const int row = 2 * (g & 1) + (e >> 2), col = e & 3;
                const float v = row < 3 && col < 3 ? w[size_t(t * 16 + r) * 9 + row * 3 + col] : 0.f;
                const _Float16 hv = (_Float16)v;
                std::memcpy(&frag[(size_t(t) * 64 + lane) * 8 + e], &hv, 2);
            }
}

bool conv1_mfma_multi(const Act *x, const Act *y, const Act *ypool, int count, const uint16_t *frag, const float *b,
                      int act, int ph, int pw, hipStream_t s) {
    if (!frag || count < 1) return false;
    if (act != ACT_NONE && act != ACT_RELU && act != ACT_SIGMOID) return false;
    if (b && (reinterpret_cast<uintptr_t>(b) & 15)) return false;
    auto aligned = [](const Act &a) { return a.cs % 4 == 0 && (reinterpret_cast<uintptr_t>(a.p) & 15) == 0; };
    const int cout = y[0].c;
    if (cout % 16 || cout > 64 || cout < 16) return false;
    // pool 0: y only; 1: y is the pooled output; 2: y full and ypool pooled.
    const int pool = ypool ? 2 : (ph == 2 && pw == 2) ? 1 : (ph == 1 && pw == 1) ? 0 : -1;
    if (pool < 0 || (pool == 2 && (ph != 2 || pw != 2))) return false;
    double flops = 0, bytes = 0;
    for (int k = 0; k < count; k++) {
        const Act &xk = x[k], &yk = y[k];
        if (xk.c != 1 || yk.c != cout || yk.n != xk.n || xk.h != x[0].h || xk.cs != x[0].cs || yk.cs != y[0].cs ||
            !aligned(yk))
            return false;
        if (pool == 2) {
            const Act &pk = ypool[k];
            if (yk.h != xk.h || yk.w != xk.w || pk.h != xk.h / 2 || pk.w != xk.w / 2 || pk.c != cout || pk.n != yk.n ||
                pk.cs != ypool[0].cs || !aligned(pk))
                return false;
        } else if (yk.h != xk.h / ph || yk.w != xk.w / pw) {
            return false;
        }
        flops += 2.0 * double(xk.pixels()) * cout * 9;
        bytes += 4.0 * double(xk.pixels() + yk.count() + (pool == 2 ? ypool[k].count() : 0));
    }
    const int tiles_y = (x[0].h + TY - 1) / TY;
    ProbeScope probe("conv_direct", s, flops, bytes);
    const int nt = cout / 16;
    for (int k0 = 0; k0 < count; k0 += C1MAXSEG) {
        const int cnt = std::min(C1MAXSEG, count - k0);
        C1Params p{};
        p.h = x[0].h;
        p.xcs = x[0].cs;
        p.tiles_y = tiles_y;
        p.nseg = cnt;
        p.wf = reinterpret_cast<const half8 *>(frag);
        p.bias = b;
        // POOL 1 writes the pooled output through (yp, poh, pow_, ypcs) = y.
        const Act &y0 = y[k0];
        const Act &yp0 = pool == 2 ? ypool[k0] : y0;
        p.oh = y0.h;
        p.ycs = y0.cs;
        p.poh = yp0.h;
        p.ypcs = yp0.cs;
        long long blocks = 0;
        for (int k = 0; k < cnt; k++) {
            const Act &xk = x[k0 + k], &yk = y[k0 + k];
            const Act &pk = pool == 2 ? ypool[k0 + k] : yk;
            C1Seg &sg = p.seg[k];
            sg.x = xk.p;
            sg.y = yk.p;
            sg.yp = pk.p;
            sg.n = xk.n;
            sg.w = xk.w;
            sg.ow = yk.w;
            sg.pow_ = pk.w;
            sg.tiles_x = (xk.w + TX - 1) / TX;
            sg.blk0 = int(blocks);
            blocks += (long long)sg.tiles_x * tiles_y * xk.n;
            if (blocks > 2147483647LL) fail("conv1_mfma: grid too large");
        }
        if (blocks == 0) continue;
        const dim3 grid{unsigned(blocks)};
#define C1_LAUNCH(NT, P, A) hipLaunchKernelGGL((conv1_kernel<NT, P, A>), grid, dim3(256), 0, s, p)
#define C1_ACT(NT, P)                                   \
    if (act == ACT_RELU) C1_LAUNCH(NT, P, ACT_RELU);     \
    else if (act == ACT_SIGMOID) C1_LAUNCH(NT, P, ACT_SIGMOID); \
    else C1_LAUNCH(NT, P, ACT_NONE)
#define C1_NT(P)                  \
    if (nt == 1) C1_ACT(1, P);     \
    else if (nt == 2) C1_ACT(2, P); \
    else if (nt == 3) C1_ACT(3, P); \
    else C1_ACT(4, P)
        if (pool == 2) {
            C1_NT(2);
        } else if (pool == 1) {
            C1_NT(1);
        } else {
            C1_NT(0);
        }
#undef C1_NT
#undef C1_ACT
#undef C1_LAUNCH
        OCR_HIP(hipGetLastError());
    }
    return true;
}

bool conv1_mfma(const Act &x, const Act &y, const uint16_t *frag, const float *b, int act, int ph, int pw,
                hipStream_t s, const Act *ypool) {
    return conv1_mfma_multi(&x, &y, ypool, 1, frag, b, act, ph, pw, s);
}

}  // namespace ocr
