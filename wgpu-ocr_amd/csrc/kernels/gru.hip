// The bidirectional GRU recurrence (ONNX GRU, linear_before_reset = 1, hidden 256, gate order
// z, r, h), one persistent dispatch per layer for all lines; each line walks its own length and
// the backward direction starts at the line's own end. Semantics of the reference's recurrence
// programs (src/gpu.rs:680-819):
//   z = s(G_z + R_z h + Rb_z), r = s(G_r + R_r h + Rb_r), c = tanh(G_h + r (R_h h + Rb_h)),
//   h' = (1 - z) c + z h, h0 = 0,  with G = W x + Wb precomputed for all steps by one GEMM.
//
// Mapping to gfx950: a workgroup owns one direction and 8 lines. R (768 x 256 per direction,
// float16 values) is loaded once as MFMA A-operand fragments, mostly into VGPRs and the rest
// into LDS, and stays resident for every time step. The hidden state of the 8 lines is the MFMA B operand: 16 columns, columns
// 0-7 its float16 "hi" part and columns 8-15 the float16 remainder "lo" (h = hi + lo to about
// 2^-22), so one v_mfma_f32_16x16x32_f16 per 16 rows and 32 hidden units gives R h for all 8
// lines at float32-class accuracy. Each wavefront owns UPW hidden units (all three gate rows of
// them), so the gate nonlinearity needs no exchange across wavefronts.
//
// Per step, after the MFMAs, lane (g, r) of a 16-lane row holds rows 4g..4g+3 of column r. The
// hi and lo columns of a line are summed with one DPP rotation by 8, arranged so that lane r < 8
// ends with units 4g, 4g+1 of line r and lane r + 8 with units 4g+2, 4g+3 of the same line:
// every lane does gate arithmetic for two units. The step's G values are loaded at the end of
// the previous step, so the HBM latency hides behind the barrier (an LDS-only one: the loads and
// the Y stores stay in flight) and the MFMA phase. The new state goes to a double-buffered LDS
// copy of the B operand: one barrier per step.
#include <hip/hip_runtime.h>

#include <cmath>

#include "../kernels.h"
#include "../runtime.h"
#include "lds_dma.h"

namespace ocr {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

// LDS row of the B operand: 256 units + 16 of padding (34 16-byte units, so the B reads of a step
// meet distinct bank groups in every access pass and the state writes distinct banks).
constexpr int H = 256, LINES = 8, HROW = H + 16;

// exp through the hardware base-2 exponential; 1/x through the hardware reciprocal (1 ulp).
__device__ inline float fast_exp(float v) { return __builtin_amdgcn_exp2f(v * 1.4426950408889634f); }
__device__ inline float sigm(float v) { return __builtin_amdgcn_rcpf(1.f + fast_exp(-v)); }
__device__ inline float tanh_f(float v) { return 1.f - 2.f * __builtin_amdgcn_rcpf(1.f + fast_exp(2.f * v)); }

// a where the mask's bits are set, b elsewhere (v_bfi_b32): a per-lane choice of a register.
__device__ inline float sel_bits(unsigned m, float a, float b) {
    return __uint_as_float((m & __float_as_uint(a)) | (~m & __float_as_uint(b)));
}

// Lane r of each 16-lane row receives the value of lane (r + 8) mod 16 (DPP row_ror:8).
__device__ inline float ror8(float v) {
    // (a row rotation has no out-of-row lanes, so bound_ctrl changes nothing; with it the
    // compiler folds the move into the add that uses it)
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, true));
}

template <int UPW>
__global__ __launch_bounds__(H / UPW * 64) void gru_kernel(const float *__restrict__ G, const half8 *__restrict__ R,
                                                           const float *__restrict__ Rb, float *__restrict__ Y,
                                                           const uint32_t *__restrict__ lens, int ntot) {
    constexpr int RT = UPW / 16;  // 16-row tiles per gate per wavefront
    constexpr int KL = 2;         // k-slices of R kept in LDS ...
    constexpr int KLQ = UPW == 16 ? 3 : 1;  // ... for the last KLQ gates
    __shared__ __align__(16) _Float16 hbuf[2][16][HROW];
    __shared__ float s_rb[768];  // this direction's recurrent bias [z | r | h]
    __shared__ half8 s_rf[H / UPW][KLQ * RT * KL][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r = lane & 15;
    const int dir = blockIdx.y, n0 = blockIdx.x * LINES;

    // R fragments: rows gate * 256 + unit, unit = wave * UPW + rt * 16 + r; k = kt * 32 + 8g .. +7.
    // All are held in VGPRs except the last KL k-slices of the last KLQ gates, which live in LDS
    // (the register file holds the rest of the step's state without spilling).
    half8 rf[3][RT][8];
#pragma unroll
    for (int q = 0; q < 3; q++)
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int kt = 0; kt < 8; kt++) {
                const half8 v = R[(size_t(dir) * 768 + q * 256 + wave * UPW + rt * 16 + r) * 32 + kt * 4 + g];
                if (q >= 3 - KLQ && kt >= 8 - KL) s_rf[wave][((q - (3 - KLQ)) * RT + rt) * KL + kt - (8 - KL)][lane] = v;
                else rf[q][rt][kt] = v;
            }

    for (int i = tid; i < 2 * 16 * HROW; i += blockDim.x) (&hbuf[0][0][0])[i] = (_Float16)0.f;
    for (int i = tid; i < 768; i += blockDim.x) s_rb[i] = Rb[dir * 768 + i];

    int maxlen = 0;
    for (int j = 0; j < LINES; j++)
        if (n0 + j < ntot) maxlen = max(maxlen, int(lens[n0 + j]));
    // This lane's line and the two units (of each 16-row tile) it updates: lane r < 8 takes
    // units 4g, 4g+1 of line r, lane r >= 8 units 4g+2, 4g+3 of line r - 8.
    const bool upper = r >= LINES;
    const unsigned umask = upper ? ~0u : 0u;
    const int lr = upper ? r - LINES : r;
    const int line = n0 + lr;
    const int len = line < ntot ? int(lens[line]) : 0;
    const int usub = upper ? 2 : 0;
    float h[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) h[rt][0] = h[rt][1] = 0.f;
    __syncthreads();
    // G of the step about to run, [gate][rt] pairs of units; loaded one step ahead.
    auto load_g = [&](int s, float2 (&gv)[3][RT]) {
        const int t = dir == 0 ? s : len - 1 - s;
        if (s < len) {
            const float *gb = G + (size_t(t) * ntot + line) * 1536 + dir * 768 + wave * UPW + 4 * g + usub;
#pragma unroll
            for (int q = 0; q < 3; q++)
#pragma unroll
                for (int rt = 0; rt < RT; rt++)
                    gv[q][rt] = *reinterpret_cast<const float2 *>(gb + q * 256 + rt * 16);
        }
    };
    float2 gcur[3][RT];
    load_g(0, gcur);
    // The recurrent bias of the lane's units, the same every step.
    float rbv[3][RT][2];
#pragma unroll
    for (int q = 0; q < 3; q++)
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int i = 0; i < 2; i++) rbv[q][rt][i] = s_rb[q * 256 + wave * UPW + rt * 16 + 4 * g + usub + i];

    typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
    for (int s = 0; s < maxlen; s++) {
        const int cur = s & 1;
        const bool on = s < len;
        floatx4 acc[3][RT];
#pragma unroll
        for (int q = 0; q < 3; q++)
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
                acc[q][rt] = floatx4{0.f, 0.f, 0.f, 0.f};
        // R h for row tile rt of the three gates (8 k-slices); the B fragment of k-slice kt + 1
        // is read from LDS before k-slice kt's MFMAs, so its latency hides behind them.
        auto mfmas = [&](int rt, int q0 = 0, int q1 = 3) __attribute__((always_inline)) {
            half8 bb[2];
            bb[0] = *reinterpret_cast<const half8 *>(&hbuf[cur][r][8 * g]);
#pragma unroll
            for (int kt = 0; kt < 8; kt++) {
                if (kt < 7) bb[(kt + 1) & 1] = *reinterpret_cast<const half8 *>(&hbuf[cur][r][(kt + 1) * 32 + 8 * g]);
                const half8 b = bb[kt & 1];
#pragma unroll
                for (int q = q0; q < q1; q++) {
                    const half8 a = (q >= 3 - KLQ && kt >= 8 - KL)
                                        ? s_rf[wave][((q - (3 - KLQ)) * RT + rt) * KL + kt - (8 - KL)][lane]
                                        : rf[q][rt][kt];
                    acc[q][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[q][rt], 0, 0, 0);
                }
            }
        };
        // The new state of row tile rt's units (also the step's Y).
        float hn[RT][2];
        float zv[RT][2], rv[RT][2];
        // hi + lo of R h for gate q of row tile rt: lane r < 8 keeps rows 0, 1 and sends rows 2, 3
        // to lane r + 8 (and the reverse).
        auto rh_of = [&](int q, int rt, float (&o)[2]) __attribute__((always_inline)) {
            // The lane's choice between rows 0, 1 and 2, 3 as bit selects on the upper-lane
            // mask (one bitfield insert each; a ternary on `upper` is compiled as a dynamic
            // index into the accumulator, a chain of compares and selects).
            const float send0 = sel_bits(umask, acc[q][rt][0], acc[q][rt][2]);
            const float send1 = sel_bits(umask, acc[q][rt][1], acc[q][rt][3]);
            const float keep0 = sel_bits(umask, acc[q][rt][2], acc[q][rt][0]);
            const float keep1 = sel_bits(umask, acc[q][rt][3], acc[q][rt][1]);
            o[0] = keep0 + ror8(send0);
            o[1] = keep1 + ror8(send1);
        };
        // The update and reset gates of row tile rt (they need only their own rows' MFMAs).
        auto gates_zr = [&](int rt) __attribute__((always_inline)) {
            float rz[2], rr2[2];
            rh_of(0, rt, rz);
            rh_of(1, rt, rr2);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const float gz = i ? gcur[0][rt].y : gcur[0][rt].x;
                const float gr = i ? gcur[1][rt].y : gcur[1][rt].x;
                zv[rt][i] = sigm(gz + (rz[i] + rbv[0][rt][i]));
                rv[rt][i] = sigm(gr + (rr2[i] + rbv[1][rt][i]));
            }
        };
        // The candidate and the new state of row tile rt, branch-free (a line past its end keeps
        // its state), and the next step's B operand: units u0 and u0 + 1 as one 32-bit word of
        // hi parts and one of lo parts.
        auto gates_h = [&](int rt) __attribute__((always_inline)) {
            float rhh[2];
            rh_of(2, rt, rhh);
            const int u0 = wave * UPW + rt * 16 + 4 * g + usub;
            half2_t hi2, lo2;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const float gh = i ? gcur[2][rt].y : gcur[2][rt].x;
                const float z = zv[rt][i], rr = rv[rt][i];
                const float c = tanh_f(gh + rr * (rhh[i] + rbv[2][rt][i]));
                hn[rt][i] = (1.f - z) * c + z * h[rt][i];
                h[rt][i] = on ? hn[rt][i] : h[rt][i];
                hi2[i] = (_Float16)h[rt][i];
                lo2[i] = (_Float16)(h[rt][i] - (float)hi2[i]);
            }
            *reinterpret_cast<half2_t *>(&hbuf[cur ^ 1][lr][u0]) = hi2;
            *reinterpret_cast<half2_t *>(&hbuf[cur ^ 1][lr + LINES][u0]) = lo2;
        };
        auto gates = [&](int rt) __attribute__((always_inline)) {
            gates_zr(rt);
            gates_h(rt);
        };
        // Two row tiles: row tile 0's MFMAs; then row tile 1's MFMAs with row tile 0's gate
        // arithmetic between them (the vector ALU works while the matrix core does); then row
        // tile 1's gates. One row tile: the update and reset rows' MFMAs, then the candidate
        // rows' MFMAs with the update and reset gates between them, then the candidate and the
        // new state.
        static_assert(RT == 1 || RT == 2, "one or two row tiles a wavefront");
        if constexpr (RT == 2) {
            mfmas(0);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(1);
            gates(0);
#pragma unroll
            for (int i = 0; i < 24; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (RT == 1) {
            mfmas(0, 0, 2);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(0, 2, 3);
            gates_zr(0);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // five VALU
            }
            __builtin_amdgcn_sched_barrier(0);
            gates_h(0);
        } else {
            gates(RT - 1);
        }
        if (on) {
            const int t = dir == 0 ? s : len - 1 - s;
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                const int u0 = wave * UPW + rt * 16 + 4 * g + usub;
                *reinterpret_cast<float2 *>(Y + (size_t(t) * ntot + line) * 512 + dir * 256 + u0) =
                    make_float2(hn[rt][0], hn[rt][1]);
            }
        }
        // The next step's G, in flight across the barrier (which waits for LDS only) and the
        // next MFMA phase.
        load_g(s + 1, gcur);
        lds_barrier();
    }
}

// Float32 recurrent weights (the reference's recurrence with F16 off, gpu.rs:858, 1476-1486):
// for R that is not float16-valued when rounding it is not allowed. R is too large to stay on
// chip next to its remainders, so this kernel streams it from L2 every step: one workgroup per
// (direction, 8 lines), thread u owns hidden unit u of all 8 lines, and R^T [dir][k][768] makes
// the 256 threads' reads of one (k, gate) row one coalesced 1 KiB access. h lives in LDS
// (double-buffered, one barrier a step); the gates use expf and a true division.
constexpr int FL = 8;  // lines per workgroup

__global__ __launch_bounds__(256) void gru_f32_kernel(const float *__restrict__ G, const float *__restrict__ Rt,
                                                      const float *__restrict__ Rb, float *__restrict__ Y,
                                                      const uint32_t *__restrict__ lens, int ntot) {
    __shared__ float hs[2][FL][H];
    const int u = threadIdx.x, dir = blockIdx.y, n0 = blockIdx.x * FL;
    const float *rt = Rt + size_t(dir) * H * 768;
    int len[FL], maxlen = 0;
#pragma unroll
    for (int l = 0; l < FL; l++) {
        len[l] = n0 + l < ntot ? int(lens[n0 + l]) : 0;
        maxlen = max(maxlen, len[l]);
        hs[0][l][u] = 0.f;
    }
    const float rbz = Rb[dir * 768 + u], rbr = Rb[dir * 768 + 256 + u], rbh = Rb[dir * 768 + 512 + u];
    float h[FL];
#pragma unroll
    for (int l = 0; l < FL; l++) h[l] = 0.f;
    __syncthreads();
    for (int s = 0; s < maxlen; s++) {
        const int cur = s & 1;
        float az[FL], ar[FL], ah[FL];
#pragma unroll
        for (int l = 0; l < FL; l++) az[l] = ar[l] = ah[l] = 0.f;
        for (int k = 0; k < H; k++) {
            const float wz = rt[size_t(k) * 768 + u], wr = rt[size_t(k) * 768 + 256 + u], wh = rt[size_t(k) * 768 + 512 + u];
#pragma unroll
            for (int l = 0; l < FL; l++) {
                const float hk = hs[cur][l][k];
                az[l] = fmaf(wz, hk, az[l]);
                ar[l] = fmaf(wr, hk, ar[l]);
                ah[l] = fmaf(wh, hk, ah[l]);
            }
        }
#pragma unroll
        for (int l = 0; l < FL; l++) {
            if (s < len[l]) {
                const int t = dir == 0 ? s : len[l] - 1 - s;
                const float *gr = G + (size_t(t) * ntot + n0 + l) * 1536 + dir * 768;
                const float z = 1.f / (1.f + expf(-(gr[u] + az[l] + rbz)));
                const float r = 1.f / (1.f + expf(-(gr[256 + u] + ar[l] + rbr)));
                const float c = tanhf(gr[512 + u] + r * (ah[l] + rbh));
                h[l] = (1.f - z) * c + z * h[l];
                Y[(size_t(t) * ntot + n0 + l) * 512 + dir * 256 + u] = h[l];
            }
            hs[cur ^ 1][l][u] = h[l];
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
    // 16 wavefronts of 16 hidden units (4 a SIMD): the matrix core always has a wavefront to
    // serve while others do their gate arithmetic (11 % faster per step than 8 of 32 units).
    constexpr int UPW = 16;
    hipLaunchKernelGGL((gru_kernel<UPW>), grid, dim3(H / UPW * 64), 0, s, G, reinterpret_cast<const half8 *>(R), Rb,
                       Y, lens, ntot);
    OCR_HIP(hipGetLastError());
}

void gru_recurrence_f32(const float *G, const float *Rt, const float *Rb, float *Y, const uint32_t *lens, int ntot,
                        long long steps, hipStream_t s) {
    if (ntot <= 0) return;
    dim3 grid(unsigned((ntot + FL - 1) / FL), 2);
    ProbeScope probe("gru", s, 2.0 * 2.0 * double(steps) * 768 * 256,
                     2.0 * double(steps) * (768 + 256) * 4 + 2.0 * 768 * 256 * 4);
    hipLaunchKernelGGL(gru_f32_kernel, grid, dim3(H), 0, s, G, Rt, Rb, Y, lens, ntot);
    OCR_HIP(hipGetLastError());
}

}  // namespace ocr
