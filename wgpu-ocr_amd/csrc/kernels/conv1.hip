// 3 x 3, pad 1 convolution of a one-channel image (the first layer of the ocrs detector and
// recogniser) on the matrix cores, with bias, activation and an optional fused 2 x 2 MaxPool:
// semantics of the reference's conv_direct program (src/gpu.rs:385-422).
//
// One v_mfma_f32_16x16x32_f16 gives 16 output channels of 16 pixels: the K = 32 side holds the
// pixel's 3 x 3 patch twice, as float16 hi parts (k 0-8) and float16 remainders lo (k 16-24) of
// the float32 input (x = hi + lo to about 2^-22), against the exact float16 weights (k 9-15 and
// 25-31 are zero weights). The weights are the A operand, so a lane's 4 accumulators are 4
// neighbouring output channels of one pixel and leave as one 16-byte NHWC store.
//
// A workgroup (4 wavefronts) owns a 16 x 64 pixel tile: the input window (18 x 66) is split once
// into hi and lo planes in LDS. A wavefront takes groups of 16 pixels laid out as four 2 x 2
// squares (so a fused pool is a max over 4 neighbouring lanes, two DPP steps); each lane reads its
// 8 patch values with immediate-offset LDS loads: lane (g, r) holds k = 8 g .. 8 g + 7 of pixel r,
// i.e. taps 0-7 (g even) or tap 8 followed by values the zero weights cancel (g odd), of the hi
// (g < 2) or the lo plane.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>

#include "../kernels.h"
#include "../runtime.h"

namespace ocr {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int TY = 16, TX = 64;               // pixels of a tile
constexpr int WW = TX + 2;                    // LDS row of the input window
constexpr int WROWS = TY + 6;                 // window rows (+ rows the cancelled reads may touch)
constexpr int PLANE = WROWS * WW;             // halves per plane

__device__ inline float act1(float v, int act) {
    if (act == ACT_RELU) return fmaxf(v, 0.f);
    if (act == ACT_SIGMOID) return 1.f / (1.f + expf(-v));
    return v;
}

// Lane l receives the value of lane l ^ 1 (quad_perm [1,0,3,2]) or lane l ^ 2 ([2,3,0,1]).
__device__ inline float xor1(float v) { return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false)); }
__device__ inline float xor2(float v) { return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false)); }

// POOL 0: the output y only; 1: the 2 x 2 pooled output only (in y); 2: both, the full output in
// y and the pooled one in yp.
template <int NT, int POOL>
__global__ __launch_bounds__(256) void conv1_kernel(const float *__restrict__ x, int h, int w, int xcs,
                                                    float *__restrict__ y, int oh, int ow, int ycs,
                                                    float *__restrict__ yp, int poh, int pow_, int ypcs,
                                                    const half8 *__restrict__ wf, const float *__restrict__ bias,
                                                    int act, int tiles_x) {
    __shared__ _Float16 s_in[2 * PLANE];  // hi plane, then lo plane
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int tx = blockIdx.x % tiles_x, ty = blockIdx.x / tiles_x, img = blockIdx.y;
    const int y0 = ty * TY, x0 = tx * TX;
    const float *xi = x + size_t(img) * h * w * xcs;
    // The input window (rows y0 - 1 .., columns x0 - 1 ..), zero outside the image and in the
    // spare rows, split into hi / lo.
    for (int i = tid; i < PLANE; i += 256) {
        const int wy = i / WW, wx = i - wy * WW;
        const int iy = y0 - 1 + wy, ix = x0 - 1 + wx;
        float v = 0.f;
        if (wy < TY + 2 && iy >= 0 && iy < h && ix >= 0 && ix < w) v = xi[(size_t(iy) * w + ix) * xcs];
        const _Float16 hi = (_Float16)v;
        s_in[i] = hi;
        s_in[PLANE + i] = (_Float16)(v - (float)hi);
    }
    // Weights (A operand) of the NT 16-channel tiles, bias of this lane's 4 channels per tile.
    half8 a[NT];
    float4 b4[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
        a[j] = wf[j * 64 + lane];
        const int co = j * 16 + 4 * g;
        b4[j] = bias ? *reinterpret_cast<const float4 *>(bias + co) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
    // This lane's pixel in a group: square r >> 2 (2 columns each), position r & 3.
    const int q = r & 3, sq = r >> 2;
    const int pdy = q >> 1, pdx = 2 * sq + (q & 1);
    // Plane and tap of this lane's first k: hi (g < 2) or lo, tap 0 (g even) or tap 8.
    const int lbase = (g >= 2 ? PLANE : 0) + ((g & 1) ? 2 * WW + 2 : 0) + pdy * WW + pdx;
    const int NG = TY / 2 * (TX / 8);  // groups of 16 pixels in the tile
    for (int G = wave; G < NG; G += 4) {
        const int gy = G / (TX / 8), gx = G - gy * (TX / 8);
        const int py = 2 * gy + pdy, px = 8 * gx + pdx;  // this lane's pixel (its B column)
        const _Float16 *src = s_in + lbase + 2 * gy * WW + 8 * gx;
        half8 bf;
#pragma unroll
        for (int k = 0; k < 8; k++) bf[k] = src[(k / 3) * WW + k % 3];
        // Output: lane (g, r) holds channels 16 j + 4 g .. + 3 of the group's pixel r.
        const int oy = y0 + py, ox = x0 + px;
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const floatx4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], bf, floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            float v[4] = {act1(acc[0] + b4[j].x, act), act1(acc[1] + b4[j].y, act), act1(acc[2] + b4[j].z, act),
                          act1(acc[3] + b4[j].w, act)};
            if (POOL != 1 && oy < oh && ox < ow)
                *reinterpret_cast<float4 *>(y + ((size_t(img) * oh + oy) * ow + ox) * ycs + j * 16 + 4 * g) =
                    make_float4(v[0], v[1], v[2], v[3]);
            if (POOL) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    v[e] = fmaxf(v[e], xor1(v[e]));
                    v[e] = fmaxf(v[e], xor2(v[e]));
                }
                const int qy = oy >> 1, qx = ox >> 1;
                if (q == 0 && qy < poh && qx < pow_)
                    *reinterpret_cast<float4 *>(yp + ((size_t(img) * poh + qy) * pow_ + qx) * ypcs + j * 16 + 4 * g) =
                        make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
}

}  // namespace

void pack_conv1_frags(const float *w, int cout, uint16_t *frag) {
    // frag [cout / 16][64 lanes][8]: lane (g, r) holds k = 8 g .. 8 g + 7 of channel 16 t + r;
    // k 0-8 and 16-24 are taps 0-8 (hi and lo sides), the rest zero.
    for (int t = 0; t < cout / 16; t++)
        for (int lane = 0; lane < 64; lane++)
            for (int e = 0; e < 8; e++) {
                const int g = lane >> 4, r = lane & 15, k = 8 * g + e, kk = k & 15;
                const float v = kk < 9 ? w[size_t(t * 16 + r) * 9 + kk] : 0.f;
                const _Float16 hv = (_Float16)v;
                std::memcpy(&frag[(size_t(t) * 64 + lane) * 8 + e], &hv, 2);
            }
}

bool conv1_mfma(const Act &x, const Act &y, const uint16_t *frag, const float *b, int act, int ph, int pw,
                hipStream_t s, const Act *ypool) {
    if (!frag || x.c != 1 || y.c % 16 || y.c > 64 || y.c < 16 || y.n != x.n) return false;
    if (act != ACT_NONE && act != ACT_RELU && act != ACT_SIGMOID) return false;
    auto aligned = [](const Act &a) { return a.cs % 4 == 0 && (reinterpret_cast<uintptr_t>(a.p) & 15) == 0; };
    int pool;
    if (ypool) {
        if (ph != 2 || pw != 2 || y.h != x.h || y.w != x.w || ypool->h != x.h / 2 || ypool->w != x.w / 2 ||
            ypool->c != y.c || ypool->n != y.n || !aligned(*ypool))
            return false;
        pool = 2;
    } else {
        pool = (ph == 2 && pw == 2) ? 1 : (ph == 1 && pw == 1) ? 0 : -1;
        if (pool < 0 || y.h != x.h / ph || y.w != x.w / pw) return false;
    }
    if (!aligned(y) || (b && (reinterpret_cast<uintptr_t>(b) & 15))) return false;
    const int tiles_x = (x.w + TX - 1) / TX, tiles_y = (x.h + TY - 1) / TY;
    if (double(tiles_x) * tiles_y > 2147483647.0 || y.n > 65535) return false;
    dim3 grid(unsigned(tiles_x * tiles_y), unsigned(y.n));
    ProbeScope probe("conv_direct", s, 2.0 * double(x.pixels()) * y.c * 9,
                     4.0 * double(x.pixels() + y.count() + (ypool ? ypool->count() : 0)));
    const half8 *wf = reinterpret_cast<const half8 *>(frag);
    // POOL 1 writes the pooled output through (yp, poh, pow_, ypcs) = y.
    const Act &yp = ypool ? *ypool : y;
#define C1_LAUNCH(NT, P)                                                                                              \
    hipLaunchKernelGGL((conv1_kernel<NT, P>), grid, dim3(256), 0, s, x.p, x.h, x.w, x.cs, y.p, y.h, y.w, y.cs, yp.p,  \
                       yp.h, yp.w, yp.cs, wf, b, act, tiles_x)
#define C1_NT(P)                  \
    if (nt == 1) C1_LAUNCH(1, P);  \
    else if (nt == 2) C1_LAUNCH(2, P); \
    else if (nt == 3) C1_LAUNCH(3, P); \
    else C1_LAUNCH(4, P)
    const int nt = y.c / 16;
    if (pool == 2) {
        C1_NT(2);
    } else if (pool == 1) {
        C1_NT(1);
    } else {
        C1_NT(0);
    }
#undef C1_NT
#undef C1_LAUNCH
    OCR_HIP(hipGetLastError());
    return true;
}

}  // namespace ocr
