// The bidirectional GRU recurrence (ONNX GRU, linear_before_reset = 1, hidden 256, gate order
// z, r, h), one persistent dispatch per layer for all lines; each line walks its own length and
// the backward direction starts at the line's own end. Semantics of the reference's recurrence
// programs (src/gpu.rs:680-819):
//   z = s(G_z + R_z h + Rb_z), r = s(G_r + R_r h + Rb_r), c = tanh(G_h + r (R_h h + Rb_h)),
//   h' = (1 - z) c + z h, h0 = 0,  with G = W x + Wb precomputed for all steps by one GEMM.
//
// Mapping to gfx950: a workgroup owns one direction and 8 lines. R (768 x 256 per direction,
// float16 values) is loaded once into VGPRs as MFMA A-operand fragments and stays resident for
// every time step. The hidden state of the 8 lines is the MFMA B operand: 16 columns, columns
// 0-7 its float16 "hi" part and columns 8-15 the float16 remainder "lo" (h = hi + lo to about
// 2^-22), so one v_mfma_f32_16x16x32_f16 per 16 rows and 32 hidden units gives R h for all 8
// lines at float32-class accuracy. Each wavefront owns UPW hidden units (all three gate rows of
// them), so the gate nonlinearity needs no exchange: after adding the hi and lo columns, lane
// (r < 8) holds 4 units of line r for z, r and h and keeps that line's state in registers. The
// new state goes to a double-buffered LDS copy of the B operand: one barrier per step.
#include <hip/hip_runtime.h>

#include <cmath>

#include "../kernels.h"
#include "../runtime.h"

namespace ocr {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int H = 256, LINES = 8, HROW = H + 8;  // LDS row of the B operand: 256 units + padding

__device__ inline float sigm(float v) { return 1.f / (1.f + expf(-v)); }

template <int UPW>
__global__ __launch_bounds__(H / UPW * 64) void gru_kernel(const float *__restrict__ G, const half8 *__restrict__ R,
                                                           const float *__restrict__ Rb, float *__restrict__ Y,
                                                           const uint32_t *__restrict__ lens, int ntot) {
    constexpr int RT = UPW / 16;  // 16-row tiles per gate per wavefront
    __shared__ __align__(16) _Float16 hbuf[2][16][HROW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int dir = blockIdx.y, n0 = blockIdx.x * LINES;

    // R fragments: rows gate * 256 + unit, unit = wave * UPW + rt * 16 + r; k = kt * 32 + 8g .. +7.
    half8 rf[3][RT][8];
#pragma unroll
    for (int q = 0; q < 3; q++)
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int kt = 0; kt < 8; kt++)
                rf[q][rt][kt] = R[(size_t(dir) * 768 + q * 256 + wave * UPW + rt * 16 + r) * 32 + kt * 4 + g];

    for (int i = tid; i < 2 * 16 * HROW; i += blockDim.x) (&hbuf[0][0][0])[i] = (_Float16)0.f;

    int maxlen = 0;
    for (int j = 0; j < LINES; j++)
        if (n0 + j < ntot) maxlen = max(maxlen, int(lens[n0 + j]));
    const int line = n0 + r;
    const bool owner = r < LINES;
    const int len = (owner && line < ntot) ? int(lens[line]) : 0;
    float h[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int i = 0; i < 4; i++) h[rt][i] = 0.f;
    __syncthreads();

    __shared__ float s_rb[768];  // this direction's recurrent bias [z | r | h]
    for (int i = tid; i < 768; i += blockDim.x) s_rb[i] = Rb[dir * 768 + i];
    __syncthreads();

    for (int s = 0; s < maxlen; s++) {
        const int cur = s & 1;
        floatx4 acc[3][RT];
#pragma unroll
        for (int q = 0; q < 3; q++)
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
                acc[q][rt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < 8; kt++) {
            const half8 b = *reinterpret_cast<const half8 *>(&hbuf[cur][r][kt * 32 + 8 * g]);
#pragma unroll
            for (int q = 0; q < 3; q++)
#pragma unroll
                for (int rt = 0; rt < RT; rt++)
                    acc[q][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(rf[q][rt][kt], b, acc[q][rt], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        // Column r + 8 holds the lo contribution of line r: add it in (DPP row_ror:8 brings lane
        // r + 8 of each 16-lane row to lane r).
#pragma unroll
        for (int q = 0; q < 3; q++)
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[q][rt][i] += __int_as_float(
                        __builtin_amdgcn_mov_dpp(__float_as_int(acc[q][rt][i]), 0x128, 0xf, 0xf, false));
        if (owner) {
            const bool on = s < len;
            const int t = dir == 0 ? s : len - 1 - s;
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const int u0 = wave * UPW + rt * 16 + 4 * g;
                if (on) {
                    const float *gb = G + (size_t(t) * ntot + line) * 1536 + dir * 768 + u0;
                    float *yo = Y + (size_t(t) * ntot + line) * 512 + dir * 256 + u0;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float z = sigm(gb[i] + (acc[0][rt][i] + s_rb[u0 + i]));
                        const float rr = sigm(gb[256 + i] + (acc[1][rt][i] + s_rb[256 + u0 + i]));
                        const float c = tanhf(gb[512 + i] + rr * (acc[2][rt][i] + s_rb[512 + u0 + i]));
                        h[rt][i] = (1.f - z) * c + z * h[rt][i];
                        yo[i] = h[rt][i];
                    }
                }
                // The next step's B operand (the unchanged state when this line has ended).
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const _Float16 hi = (_Float16)h[rt][i];
                    hbuf[cur ^ 1][r][u0 + i] = hi;
                    hbuf[cur ^ 1][r + 8][u0 + i] = (_Float16)(h[rt][i] - (float)hi);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();
    }
}

}  // namespace

void gru_recurrence(const float *G, const uint16_t *R, const float *Rb, float *Y, const uint32_t *lens, int ntot,
                    int tmax, long long steps, hipStream_t s) {
    (void)tmax;
    if (ntot <= 0) return;
    dim3 grid(unsigned((ntot + LINES - 1) / LINES), 2);
    // Per line step and direction: R h (768 x 256), G read (768 floats), Y written (256 floats).
    ProbeScope probe("gru", s, 2.0 * 2.0 * double(steps) * 768 * 256,
                     2.0 * double(steps) * (768 + 256) * 4 + 2.0 * 768 * 256 * 2);
    hipLaunchKernelGGL((gru_kernel<32>), grid, dim3(H / 32 * 64), 0, s, G, reinterpret_cast<const half8 *>(R), Rb, Y,
                       lens, ntot);
    OCR_HIP(hipGetLastError());
}

}  // namespace ocr
