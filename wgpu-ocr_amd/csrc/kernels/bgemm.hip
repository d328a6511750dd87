// Batched GEMM on the gfx950 matrix cores for products of two computed tensors (the SVTR
// attention's Q K^T and A V; the reference's nd_bgemm, src/nd.rs:291-358, in float32 FMA).
//
// Both operands are float32 activations, so each is split on the fly into float16 hi and the
// float16 remainder lo, and C = Ahi Bhi + Ahi Blo + Alo Bhi is accumulated in float32 with
// v_mfma_f32_16x16x32_f16 (the dropped Alo Blo term is below 2^-22 relative). A workgroup of 4
// wavefronts owns a 64 x 64 tile of C; each wavefront a 32 x 32 quarter (2 x 2 MFMA tiles). K
// advances in slices of 32, staged in LDS as hi/lo halves: A row-major [m][k], B transposed
// [n][k], so both MFMA operands are 16-byte LDS reads.
#include <hip/hip_runtime.h>

#include "../nd_kernels.h"
#include "../runtime.h"

namespace ocr {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int BT = 64, KT = 32, KS = 40;  // tile, K slice, LDS row (32 halves + 8 padding)

__global__ __launch_bounds__(256) void bgemm_kernel(BgemmArgs g) {
    __shared__ __align__(16) _Float16 a_hi[BT][KS], a_lo[BT][KS], b_hi[BT][KS], b_lo[BT][KS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gq = lane >> 4, r = lane & 15;
    const int n0 = blockIdx.x * BT, m0 = blockIdx.y * BT, bb = blockIdx.z;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const float *A = g.a + size_t(bb) * g.sab;
    const float *B = g.b + size_t(bb) * g.sbb;
    floatx4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < g.k; k0 += KT) {
        for (int i = tid; i < BT * KT; i += 256) {
            const int m = i / KT, k = i - m * KT;  // k fastest: rows of A are contiguous in k
            float v = 0.f;
            if (m0 + m < g.m && k0 + k < g.k) v = A[size_t(m0 + m) * g.sam + size_t(k0 + k) * g.sak];
            const _Float16 h = (_Float16)v;
            a_hi[m][k] = h;
            a_lo[m][k] = (_Float16)(v - (float)h);
        }
        for (int i = tid; i < BT * KT; i += 256) {
            const int k = i / BT, n = i - k * BT;  // n fastest: rows of B are contiguous in n
            float v = 0.f;
            if (n0 + n < g.n && k0 + k < g.k) v = B[size_t(k0 + k) * g.sbk + size_t(n0 + n) * g.sbn];
            const _Float16 h = (_Float16)v;
            b_hi[n][k] = h;
            b_lo[n][k] = (_Float16)(v - (float)h);
        }
        __syncthreads();
        half8 ah[2], al[2], bh[2], bl[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            ah[i] = *reinterpret_cast<const half8 *>(&a_hi[wm + i * 16 + r][8 * gq]);
            al[i] = *reinterpret_cast<const half8 *>(&a_lo[wm + i * 16 + r][8 * gq]);
            bh[i] = *reinterpret_cast<const half8 *>(&b_hi[wn + i * 16 + r][8 * gq]);
            bl[i] = *reinterpret_cast<const half8 *>(&b_lo[wn + i * 16 + r][8 * gq]);
        }
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bh[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[i], bl[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bh[j], acc[i][j], 0, 0, 0);
            }
        __syncthreads();
    }
    // Lane (gq, r) holds rows 4 gq .. 4 gq + 3 of column r of each 16 x 16 tile.
    float *C = g.c + size_t(bb) * g.scb;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn + j * 16 + r;
            if (n >= g.n) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm + i * 16 + 4 * gq + e;
                if (m < g.m) C[size_t(m) * g.scm + size_t(n) * g.scn] = acc[i][j][e];
            }
        }
}

}  // namespace

void nd_bgemm(const BgemmArgs &g, hipStream_t s) {
    if (g.batch <= 0 || g.m <= 0 || g.n <= 0) return;
    if (g.batch > 65535) fail("nd_bgemm: batch above 65535");
    ProbeScope probe("nd_bgemm", s, 2.0 * g.batch * double(g.m) * g.n * g.k,
                     4.0 * g.batch * (double(g.m) * g.k + double(g.k) * g.n + double(g.m) * g.n));
    dim3 grid(unsigned((g.n + BT - 1) / BT), unsigned((g.m + BT - 1) / BT), unsigned(g.batch));
    hipLaunchKernelGGL(bgemm_kernel, grid, dim3(256), 0, s, g);
    OCR_HIP(hipGetLastError());
}

}  // namespace ocr
