// Dense 1 x 1 convolution / GEMM on the gfx950 matrix cores: y[m][n] = act(sum_k x[m][k] w[k][n]
// + b[n]) with float32 x (NHWC pixels, or GEMM rows picked by a row map) and float32 w.
// The recogniser's GRU input projections (src/gpu.rs:1538-1566: [rows][256 or 512] x
// [.][1536]) and its output layer run here, as does any NHWC 1 x 1 convolution of the executor
// with at least 128 input channels.
//
// Precision: each float32 activation is split into float16 hi and the float16 remainder lo
// (x = hi + lo to about 2^-22); both go through v_mfma_f32_16x16x32_f16 against the float16
// weights with float32 accumulation. Weights that are not all float16 values come as further K
// slices of their float16 remainders, against which the activations' K slices are read again.
//
// Roles: the weights are the MFMA's A operand and the activations its B operand, so a lane's four
// accumulators are four neighbouring output channels of one row and leave as one 16-byte store.
//
// Pipeline (one 32-wide K chunk a stage, three LDS stages): between the MFMAs of stage s the
// weights of chunk s + 2 arrive by LDS DMA (lane-ordered fragments copied as they are), the
// float32 activations of chunk s + 2 (loaded during stage s - 1) are split into hi / lo and
// written to LDS, those of chunk s + 3 are loaded into registers, and in the last step the
// fragments of chunk s + 1 are read into registers, so the next stage starts on the matrix cores
// right after the barrier.
// A workgroup (8 wavefronts, 256 rows x 32 NT columns) is persistent: it keeps one block of
// output channels (its bias and the row map of its tiles sit in LDS) and walks a contiguous run of
// row tiles with the pipeline running on across tile boundaries.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "../kernels.h"
#include "../runtime.h"
#include "lds_dma.h"

namespace ocr {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int GBM = 256;        // rows per tile
constexpr int RSU = 9;          // LDS units (16 bytes) per row: 4 hi, 4 lo, 1 of padding
constexpr int ASU = GBM * RSU;  // activation stage size in units



struct GParams {
    const float *x;
    long xcs;
    int K, chunks;  // chunks: weight slices of 32 (twice K's for inexact weights)
    int xchunks;    // slices of K
    const int *rows;  // row map (row i of the GEMM reads x row rows[i], writes y row rows[i]) or null
    int M;
    float *y;
    long ycs;
    int N;
    const half8 *wt;  // fragments [n-tile][chunk][64 lanes] of 8 halves
    int ntiles;
    const float *bias;
    int act;
    int mtiles, nblocks, runs;
    int vec;            // 16-byte output stores (N and the row stride multiples of 4, y aligned)
    const float *zero;  // 64 zero bytes
};

__device__ inline float gact(float v, int act) {
    if (act == ACT_RELU) return fmaxf(v, 0.f);
    if (act == ACT_SIGMOID) return 1.f / (1.f + expf(-v));
    return v;
}

__device__ inline int gxcd_index(int b, int G) {
    const int q = G >> 3, rem = G & 7, x = b & 7;
    return x * q + min(x, rem) + (b >> 3);
}

template <int NT, int ACT>
__global__ __launch_bounds__(512, 1) void gemm_dma_kernel(GParams p) {
    constexpr int WM = 4, WN = 2, MT = 4, NTW = NT * WN;
    constexpr int NWI = (NTW + 7) / 8;  // weight DMA instructions per wavefront and chunk
    __shared__ __align__(16) half8 AS0[ASU];
    __shared__ __align__(16) half8 AS1[ASU];
    __shared__ __align__(16) half8 AS2[ASU];
    __shared__ __align__(16) half8 WB0[NTW * 64];
    __shared__ __align__(16) half8 WB1[NTW * 64];
    __shared__ __align__(16) half8 WB2[NTW * 64];
    __shared__ __align__(16) float BIAS[NTW * 16];
    __shared__ int ROWS[2][GBM];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const int g = lane >> 4, r = lane & 15;
    const int v = gxcd_index(blockIdx.x, gridDim.x);
    const int nb = v % p.nblocks, run = v / p.nblocks;
    if (run >= p.runs) return;
    const int tb = int((long(run) * p.mtiles) / p.runs), te = int((long(run + 1) * p.mtiles) / p.runs);
    if (tb >= te) return;
    const int S = (te - tb) * p.chunks;  // stages of this run
    const int nt0 = nb * NTW;

    // Loader role: rows lr and lr + 128 of a tile, floats 8 lq..8 lq + 7 of a chunk.
    const int lr = tid >> 2, lq = tid & 3;
    auto row_of = [&](int tile, int h) __attribute__((always_inline)) -> int {
        const int m = tile * GBM + lr + 128 * h;
        if (tile >= te || m >= p.M) return -1;
        return p.rows ? p.rows[m] : m;
    };
    int ld_row[2], nx_row[2];
    // The loader moves to tile `tile`: its rows (prefetched in nx_row, also written to ROWS for
    // the epilogue) and the prefetch of the next tile's (gathered earlier into nx2).
    auto enter_tile = [&](int tile, const int (&nx2)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            ld_row[h] = nx_row[h];
            if (lq == 0) ROWS[tile & 1][lr + 128 * h] = ld_row[h];
            nx_row[h] = nx2[h];
        }
    };
    float4 R0[4], R1[4];
    // Activations of chunk c of the loader's tile (zeros outside the rows or K).
    auto load_a = [&](float4(&R)[4], int c, bool live) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int k0 = (c >= p.xchunks ? c - p.xchunks : c) * 32 + 8 * lq + 4 * e;
                const float4 *src = reinterpret_cast<const float4 *>(p.zero);
                if (live && ld_row[h] >= 0 && k0 < p.K) src = reinterpret_cast<const float4 *>(p.x + size_t(ld_row[h]) * p.xcs + k0);
                R[2 * h + e] = *src;
            }
    };
    // Row lr + 128 h of the loaded chunk, split into hi / lo, into an LDS stage.
    auto convert = [&](const float4(&R)[4], half8 *as, int h) __attribute__((always_inline)) {
        const float xs[8] = {R[2 * h].x, R[2 * h].y, R[2 * h].z, R[2 * h].w,
                             R[2 * h + 1].x, R[2 * h + 1].y, R[2 * h + 1].z, R[2 * h + 1].w};
        half8 hi, lo;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            hi[e] = (_Float16)xs[e];
            lo[e] = (_Float16)(xs[e] - (float)hi[e]);
        }
        const int u = (lr + 128 * h) * RSU + lq;
        as[u] = hi;
        as[u + 4] = lo;
    };
    // Weights of chunk c: fragment b = n-tile nt0 + b, instruction i.
    auto dma_w = [&](half8 *dst, int c, int i) __attribute__((always_inline)) {
        const int b = min(i * 8 + wave, NTW - 1), nt = nt0 + b;
        const half8 *src = reinterpret_cast<const half8 *>(p.zero);
        if (nt < p.ntiles) src = p.wt + (size_t(nt) * p.chunks + c) * 64 + lane;
        dma16(src, dst + b * 64);
    };

    // Prologue: rows of the first tile, chunks 0 and 1 in LDS, chunk 2 in R0, bias.
    {
        int nx2[2];
#pragma unroll
        for (int h = 0; h < 2; h++) nx_row[h] = row_of(tb, h), nx2[h] = row_of(tb + 1, h);
        enter_tile(tb, nx2);
    }
    for (int i = tid; i < NTW * 16; i += 512) {
        const int n = nt0 * 16 + i;
        BIAS[i] = (p.bias && n < p.N) ? p.bias[n] : 0.f;
    }
    load_a(R0, 0, true);
    load_a(R1, 1, true);
#pragma unroll
    for (int i = 0; i < NWI; i++) dma_w(WB0, 0, i);
#pragma unroll
    for (int i = 0; i < NWI; i++) dma_w(WB1, 1, i);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    convert(R0, AS0, 0);
    convert(R0, AS0, 1);
    convert(R1, AS1, 0);
    convert(R1, AS1, 1);
    // The loader's position: chunk la_c of tile la_t (stage s + 3 of the run).
    int la_t = tb, la_c = 2;
    load_a(R0, la_c, 2 < S);
    la_c++;  // at least four chunks a tile: still tile tb
    lds_barrier();

    floatx4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int j = 0; j < NT; j++) acc[mt][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    half8 wf[NT], ah[2], al[2];
    auto read_a = [&](const half8 *as, int mt, int set) __attribute__((always_inline)) {
        const int u = (wm * 64 + mt * 16 + r) * RSU + g;
        ah[set] = as[u];
        al[set] = as[u + 4];
    };
#pragma unroll
    for (int j = 0; j < NT; j++) wf[j] = WB0[(wn * NT + j) * 64 + lane];
    read_a(AS0, 0, 0);

    // Output of the tile that ended with the previous stage; orow: its rows for this lane (read
    // from ROWS before that stage's barrier).
    int orow[MT];
    auto epilogue = [&]() __attribute__((always_inline)) {
        const int n_w = (nt0 + wn * NT) * 16 + 4 * g;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            float *yr = p.y + size_t(orow[mt] < 0 ? 0 : orow[mt]) * p.ycs;
#pragma unroll
            for (int j = 0; j < NT; j++) {
                const float4 b4 = *reinterpret_cast<const float4 *>(&BIAS[(wn * NT + j) * 16 + 4 * g]);
                float4 o;
                o.x = gact(acc[mt][j][0] + b4.x, ACT);
                o.y = gact(acc[mt][j][1] + b4.y, ACT);
                o.z = gact(acc[mt][j][2] + b4.z, ACT);
                o.w = gact(acc[mt][j][3] + b4.w, ACT);
                acc[mt][j] = floatx4{0.f, 0.f, 0.f, 0.f};
                const int n = n_w + 16 * j;
                if (orow[mt] < 0 || n >= p.N) continue;
                if (p.vec) {
                    *reinterpret_cast<float4 *>(yr + n) = o;
                } else {
                    yr[n] = o.x;
                    if (n + 1 < p.N) yr[n + 1] = o.y;
                    if (n + 2 < p.N) yr[n + 2] = o.z;
                    if (n + 3 < p.N) yr[n + 3] = o.w;
                }
            }
        }
    };

    int ct = tb, cc = 0;  // the compute position: chunk cc of tile ct
    int wc = 2 % p.chunks;  // chunk index of the weights for stage s + 2
    bool pend = false;
    int s = 0;
    // Stage s with LDS stage S3 = s % 3 and register set S2 = s % 2.
    auto stage = [&](auto S3c, auto S2c) __attribute__((always_inline)) -> bool {
        constexpr int S3 = decltype(S3c)::value, S2 = decltype(S2c)::value;
        half8 *ASc = S3 == 0 ? AS0 : S3 == 1 ? AS1 : AS2;
        half8 *ASn = S3 == 0 ? AS1 : S3 == 1 ? AS2 : AS0;
        half8 *AS2n = S3 == 0 ? AS2 : S3 == 1 ? AS0 : AS1;
        half8 *WBn = S3 == 0 ? WB1 : S3 == 1 ? WB2 : WB0;
        half8 *WB2n = S3 == 0 ? WB2 : S3 == 1 ? WB0 : WB1;
        float4(&Rc)[4] = S2 == 0 ? R0 : R1;  // chunk s + 2, loaded during stage s - 1
        float4(&Rn)[4] = S2 == 0 ? R1 : R0;  // chunk s + 3, loaded now
        // The activations of chunk s + 2 are the previous stage's last loads.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (pend) {
            epilogue();
            pend = false;
        }
        // Rows of the tile after the next one, when the loader moves on in this stage (gathered
        // before this stage's activation loads: those must be its last loads).
        const bool entering = s + 3 < S && la_c == p.chunks - 1;
        int nx2[2] = {-1, -1};
        if (entering) {
#pragma unroll
            for (int h = 0; h < 2; h++) nx2[h] = row_of(la_t + 2, h);
        }
        // Chunk s: MT row tiles x NT n-tiles x (hi, lo); the next row tile's fragments are read
        // one step ahead. Between the MFMAs: the weights of chunk s + 2 (DMA), the hi / lo split
        // of chunk s + 2, the loads of chunk s + 3, and in the last step the next stage's
        // weights (each fragment after its last use) and first row tile.
        const bool more = s + 1 < S, conv = s + 2 < S;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int ca = mt & 1;
            if (mt + 1 < MT) read_a(ASc, mt + 1, ca ^ 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < NT; j++) acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[j], ah[ca], acc[mt][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (mt == 0 && conv) {
#pragma unroll
                for (int i = 0; i < NWI; i++) dma_w(WB2n, wc, i);
            }
            if (mt < 2 && conv) convert(Rc, AS2n, mt);
            __builtin_amdgcn_sched_barrier(0);
            if (mt + 1 < MT) {
#pragma unroll
                for (int j = 0; j < NT; j++) acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[j], al[ca], acc[mt][j], 0, 0, 0);
            } else {
#pragma unroll
                for (int j = 0; j < NT; j++) {
                    acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[j], al[ca], acc[mt][j], 0, 0, 0);
                    if (more) wf[j] = WBn[(wn * NT + j) * 64 + lane];
                }
                if (more) read_a(ASn, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (mt == 0) {
                // Chunk s + 3 into registers (zeros past the run), always four loads: the end of
                // the stage leaves exactly these outstanding.
                load_a(Rn, la_c, s + 3 < S);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (++wc == p.chunks) wc = 0;
        if (++cc == p.chunks) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) orow[mt] = ROWS[ct & 1][wm * 64 + mt * 16 + r];
            pend = true;
            cc = 0, ct++;
        }
        if (s + 3 < S && ++la_c == p.chunks) la_c = 0, enter_tile(++la_t, nx2);
        // The weights of chunk s + 2 have landed (the loads of chunk s + 3 may be in flight).
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        lds_barrier();
        return ++s < S;
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    for (;;) {
        if (!stage(I0{}, I0{}) || !stage(I1{}, I1{}) || !stage(I2{}, I0{})) break;
        if (!stage(I0{}, I1{}) || !stage(I1{}, I0{}) || !stage(I2{}, I1{})) break;
    }
    if (pend) epilogue();
}

int gcu_count() {
    static int n = 0;
    if (!n) {
        int dev = 0;
        OCR_HIP(hipGetDevice(&dev));
        OCR_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        if (n <= 0) n = 256;
    }
    return n;
}

const float *gzero() { return static_cast<const float *>(zero_block64()); }

}  // namespace

bool gemm_dma(const ConvArgs &a, hipStream_t s) {
    const ConvPack &pk = a.pk;
    if (!a.wt_frag || a.nchw || a.in_scale || a.affine || a.amax_part || a.res) return false;
    if (pk.kh != 1 || pk.kw != 1 || a.pt || a.pl || a.ypool.p || a.y_px || a.y_row || a.y_img) return false;
    if (pk.cin != a.x.c || pk.cout != a.y.c) return false;
    if (a.x.n != a.y.n || a.x.h != a.y.h || a.x.w != a.y.w) return false;
    if (a.act != ACT_NONE && a.act != ACT_RELU && a.act != ACT_SIGMOID) return false;
    if (a.rows && (a.x.n != 1 || a.x.h != 1)) return false;
    const int K = a.x.c, N = a.y.c;
    // Four or more K chunks: the row map of a tile stays in LDS until its epilogue.
    if (K % 4 || a.x.cs % 4 || (reinterpret_cast<uintptr_t>(a.x.p) & 15) || pk.frag_chunks() < 4 || N < 1) return false;
    const double m = double(a.x.n) * a.x.h * a.x.w;
    if (m >= 2147483647.0 - GBM) return false;
    GParams p{};
    p.x = a.x.p;
    p.xcs = a.x.cs;
    p.K = K;
    p.chunks = pk.frag_chunks();
    p.xchunks = pk.chunks;
    p.rows = a.rows;
    p.M = int(m);
    p.y = a.y.p;
    p.ycs = a.y.cs;
    p.N = N;
    p.wt = reinterpret_cast<const half8 *>(a.wt_frag);
    p.ntiles = pk.nblocks * pk.bn / 16;
    p.bias = a.bias;
    p.act = a.act;
    const int nt = N > 128 ? 8 : 4, bn = 32 * nt;
    p.mtiles = (p.M + GBM - 1) / GBM;
    p.nblocks = (N + bn - 1) / bn;
    p.runs = std::max(1, std::min(p.mtiles, gcu_count() / p.nblocks));
    p.vec = (N % 4 == 0 && a.y.cs % 4 == 0 && (reinterpret_cast<uintptr_t>(a.y.p) & 15) == 0) ? 1 : 0;
    p.zero = gzero();
    if (p.M == 0) return true;
    const int grid = p.runs * p.nblocks;
    const double flops = 2.0 * p.M * double(N) * K;
    const double bytes = 4.0 * (double(p.M) * K + double(p.M) * N) + 2.0 * double(pk.frag_halves());
    ProbeScope probe("gemm_dma", s, flops, bytes);
    auto launch = [&](auto ACTc) {
        constexpr int A = decltype(ACTc)::value;
        if (nt == 8) hipLaunchKernelGGL((gemm_dma_kernel<8, A>), dim3(unsigned(grid)), dim3(512), 0, s, p);
        else hipLaunchKernelGGL((gemm_dma_kernel<4, A>), dim3(unsigned(grid)), dim3(512), 0, s, p);
    };
    if (a.act == ACT_RELU) launch(std::integral_constant<int, ACT_RELU>{});
    else if (a.act == ACT_SIGMOID) launch(std::integral_constant<int, ACT_SIGMOID>{});
    else launch(std::integral_constant<int, ACT_NONE>{});
    OCR_HIP(hipGetLastError());
    return true;
}

}  // namespace ocr
