// Run-length labelling of the detection masks on the GPU: the first half of word_rects
// (ocr-bench.rs:40-60; the components the host restatement in geometry.cpp finds), so the host
// only turns each component's row extremes into a rectangle.
//
// For every page of a detection pass: (1) a wavefront per mask row counts the row's runs (set
// pixels whose left neighbour is clear); (2) a workgroup per page turns the counts into row
// offsets; (3) a wavefront per row writes its runs, left to right, each run its own parent; (4)
// every run is joined with every run of the row above that touches it with 8-connectivity
// (x ranges overlapping or adjacent; the runs above found by binary search), linking the larger
// root under the smaller with a compare-and-swap, so every component's root is its smallest run
// index: its first run in row-major order, the order the host lists components in (within bands
// of rows in LDS first, then across the bands' edges); (5) a thread per run replaces its
// parent by its root and raises its root's bottom row; (6) a thread per root gives its component
// a record and a block of row slots, one a row from top to bottom (an 8-connected component has
// pixels in every row of its span); (7) a thread per run folds its first and last pixel into its
// row's slot with atomic min / max (only the first and last of neighbouring runs of one component
// in a row). The host then reads each component's leftmost and rightmost
// pixel per row, the points its rectangle needs. A page with more runs, components or row slots
// than the buffers hold gets none of them (its totals say so) and the host labels it from the
// bits instead.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../kernels.h"
#include "../runtime.h"

namespace ocr {

namespace {

constexpr int CCL_MAXPAGES = 16;
struct CclParams {
    CclPage pg[CCL_MAXPAGES];
};

// Word wi of a row, zero past the last one and past the mask width w.
__device__ inline uint32_t mask_word(const uint32_t *row, int wi, int words, int w) {
    if (wi < 0 || wi >= words) return 0u;
    uint32_t v = row[wi];
    if (wi == words - 1 && (w & 31)) v &= (1u << (w & 31)) - 1u;
    return v;
}

// Exclusive prefix sum over the wavefront's lanes, and the wavefront total.
__device__ inline int wave_scan(int v, int lane, int &total) {
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    total = __shfl(x, 63);
    return x - v;
}

__global__ __launch_bounds__(256) void ccl_count_kernel(const CclParams p) {
    const CclPage &g = p.pg[blockIdx.y];
    const int lane = threadIdx.x & 63, y = int(blockIdx.x) * 4 + int(threadIdx.x >> 6);
    if (y >= g.h) return;
    const int words = (g.w + 31) / 32;
    const uint32_t *row = g.bits + size_t(y) * words;
    int n = 0;
    for (int c0 = 0; c0 < words; c0 += 64) {
        const int wi = c0 + lane;
        const uint32_t v = mask_word(row, wi, words, g.w), prev = mask_word(row, wi - 1, words, g.w);
        n += __popc(v & ~((v << 1) | (prev >> 31)));
    }
    int total;
    wave_scan(n, lane, total);
    if (lane == 0) g.row_off[y + 1] = total;
}

// Row offsets: row_off[0] = 0, row_off[y + 1] = runs in rows 0 .. y; total = row_off[h].
__global__ __launch_bounds__(1024) void ccl_scan_kernel(const CclParams p) {
    const CclPage &g = p.pg[blockIdx.x];
    __shared__ int s_wave[16];
    __shared__ int s_carry;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) s_carry = 0;
    __syncthreads();
    for (int b = 0; b < g.h; b += 1024) {
        const int y = b + tid;
        const int v = y < g.h ? g.row_off[y + 1] : 0;
        int wt;
        const int ex = wave_scan(v, lane, wt);
        if (lane == 0) s_wave[wave] = wt;
        __syncthreads();
        int before = s_carry;
        for (int k = 0; k < wave; k++) before += s_wave[k];
        if (y < g.h) g.row_off[y + 1] = before + ex + v;
        __syncthreads();
        if (tid == 1023) s_carry = before + ex + v;
        __syncthreads();
    }
    if (tid == 0) {
        g.row_off[0] = 0;
        g.total[0] = s_carry;
        g.total[1] = 0;
        g.total[2] = 0;
    }
}

__global__ __launch_bounds__(256) void ccl_runs_kernel(const CclParams p) {
    const CclPage &g = p.pg[blockIdx.y];
    const int lane = threadIdx.x & 63, y = int(blockIdx.x) * 4 + int(threadIdx.x >> 6);
    if (y >= g.h || g.row_off[g.h] > g.cap) return;
    const int words = (g.w + 31) / 32;
    const uint32_t *row = g.bits + size_t(y) * words;
    int ks = g.row_off[y], ke = ks;  // next start / end index of the row
    for (int c0 = 0; c0 < words; c0 += 64) {
        const int wi = c0 + lane;
        const uint32_t v = mask_word(row, wi, words, g.w), prev = mask_word(row, wi - 1, words, g.w),
                       next = mask_word(row, wi + 1, words, g.w);
        uint32_t st = v & ~((v << 1) | (prev >> 31));  // run starts
        uint32_t en = v & ~((v >> 1) | (next << 31));  // run ends (last pixel)
        int ts, te;
        int is = ks + wave_scan(__popc(st), lane, ts), ie = ke + wave_scan(__popc(en), lane, te);
        while (st) {
            const int b = __ffs(int(st)) - 1;
            st &= st - 1;
            g.x0[is] = uint16_t(wi * 32 + b);
            g.ry[is] = uint16_t(y);
            g.cbot[is] = y;
            g.root[is] = is;
            is++;
        }
        while (en) {
            const int b = __ffs(int(en)) - 1;
            en &= en - 1;
            g.x1[ie++] = uint16_t(wi * 32 + b);
        }
        ks += ts;
        ke += te;
    }
}

// The root of x, read only (the flatten step: its stores of final roots must not be replaced by
// a concurrent walk's shortcut).
__device__ inline int ccl_root(const int32_t *parent, int x) {
    for (;;) {
        const int q = __atomic_load_n(parent + x, __ATOMIC_RELAXED);
        if (q == x) return x;
        x = q;
    }
}

// The root of x, halving the path on the way (x's parent becomes its grandparent: an ancestor
// either way, and only roots are ever linked, so the store never undoes a link). Union step only.
__device__ inline int ccl_find(int32_t *parent, int x) {
    for (;;) {
        const int q = __atomic_load_n(parent + x, __ATOMIC_RELAXED);
        if (q == x) return x;
        const int qq = __atomic_load_n(parent + q, __ATOMIC_RELAXED);
        if (qq != q) __atomic_store_n(parent + x, qq, __ATOMIC_RELAXED);
        x = qq;
    }
}

// Joins run j (row y > 0) with every run of the row above that touches it, on the global
// parents: the larger root linked under the smaller with a compare-and-swap.
__device__ inline void ccl_join_above(const CclPage &g, int j, int y) {
    const int lo = g.row_off[y - 1], hi = g.row_off[y];
    const int a0 = g.x0[j], a1 = g.x1[j];
    // First run above whose right end reaches a0 - 1 (right ends increase along a row).
    int l = lo, r = hi;
    while (l < r) {
        const int m = (l + r) >> 1;
        if (int(g.x1[m]) + 1 >= a0) r = m;
        else l = m + 1;
    }
    for (int i = l; i < hi && int(g.x0[i]) <= a1 + 1; i++) {
        int u = i, v = j;
        for (;;) {
            u = ccl_find(g.root, u);
            v = ccl_find(g.root, v);
            if (u == v) break;
            if (u > v) {
                const int t = u;
                u = v;
                v = t;
            }
            // Link root v under the smaller root u, if v is still a root.
            if (atomicCAS(g.root + v, v, u) == v) break;
        }
    }
}

// Step (4) in two parts. Bands of CCL_BAND rows first: a workgroup a band joins every run with
// the runs of the row above inside the band, with the runs' ranges and parents in LDS (binary
// searches, parent walks and compare-and-swaps at LDS latency instead of a chain of dependent
// global loads), then sets each run's parent to its band root, the band's smallest run index of
// its component. A band with more runs than CCL_BAND_CAP does the same on the global parents.
// Then ccl_union_bounds_kernel joins the first row of each band with the row above it.
constexpr int CCL_BAND = 32, CCL_BAND_CAP = 4096;

// The root of local run x in the LDS parents, halving the path (as ccl_find).
__device__ inline int ccl_find_lds(int *par, int x) {
    for (;;) {
        const int q = __hip_atomic_load(par + x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (q == x) return x;
        const int qq = __hip_atomic_load(par + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (qq != q) __hip_atomic_store(par + x, qq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        x = qq;
    }
}

__global__ __launch_bounds__(512) void ccl_union_band_kernel(const CclParams p) {
    const CclPage &g = p.pg[blockIdx.y];
    const int n = g.row_off[g.h];
    const int y0 = int(blockIdx.x) * CCL_BAND;
    if (n > g.cap || y0 >= g.h) return;
    const int y1 = min(g.h, y0 + CCL_BAND), r0 = g.row_off[y0], nb = g.row_off[y1] - r0;
    const int tid = threadIdx.x;
    if (nb > CCL_BAND_CAP) {
        for (int j = r0 + tid; j < r0 + nb; j += 512) {
            const int y = g.ry[j];
            if (y > y0) ccl_join_above(g, j, y);
        }
        return;
    }
    __shared__ uint16_t s_x0[CCL_BAND_CAP], s_x1[CCL_BAND_CAP];
    __shared__ uint8_t s_row[CCL_BAND_CAP];  // row within the band
    __shared__ int s_par[CCL_BAND_CAP];
    __shared__ int s_off[CCL_BAND + 1];      // band-local index of each row's first run
    for (int k = tid; k < nb; k += 512) {
        s_x0[k] = g.x0[r0 + k];
        s_x1[k] = g.x1[r0 + k];
        s_row[k] = uint8_t(g.ry[r0 + k] - y0);
        s_par[k] = k;
    }
    for (int t = tid; t <= y1 - y0; t += 512) s_off[t] = g.row_off[y0 + t] - r0;
    __syncthreads();
    for (int k = tid; k < nb; k += 512) {
        const int yl = s_row[k];
        if (yl == 0) continue;
        const int lo = s_off[yl - 1], hi = s_off[yl];
        const int a0 = s_x0[k], a1 = s_x1[k];
        int l = lo, r = hi;
        while (l < r) {
            const int m = (l + r) >> 1;
            if (int(s_x1[m]) + 1 >= a0) r = m;
            else l = m + 1;
        }
        for (int i = l; i < hi && int(s_x0[i]) <= a1 + 1; i++) {
            int u = i, v = k;
            for (;;) {
                u = ccl_find_lds(s_par, u);
                v = ccl_find_lds(s_par, v);
                if (u == v) break;
                if (u > v) {
                    const int t = u;
                    u = v;
                    v = t;
                }
                if (atomicCAS(s_par + v, v, u) == v) break;
            }
        }
    }
    __syncthreads();
    // No links are made any more: a plain walk to the band root.
    for (int k = tid; k < nb; k += 512) {
        int x = k;
        while (s_par[x] != x) x = s_par[x];
        g.root[r0 + k] = r0 + x;
    }
}

// The first row of every band but the first, joined with the last row of the band above (the
// parents are then at most one link from a band root within each band).
__global__ __launch_bounds__(256) void ccl_union_bounds_kernel(const CclParams p) {
    const CclPage &g = p.pg[blockIdx.y];
    const int n = g.row_off[g.h];
    const int y = (int(blockIdx.x) + 1) * CCL_BAND;
    if (n > g.cap || y >= g.h) return;
    for (int j = g.row_off[y] + int(threadIdx.x); j < g.row_off[y + 1]; j += 256) ccl_join_above(g, j, y);
}

__global__ __launch_bounds__(256) void ccl_flatten_kernel(const CclParams p) {
    const CclPage &g = p.pg[blockIdx.y];
    const int n = g.row_off[g.h];
    if (n > g.cap) return;
    for (int j = int(blockIdx.x) * 256 + int(threadIdx.x); j < n; j += int(gridDim.x) * 256) {
        const int r = ccl_root(g.root, j);
        g.root[j] = r;
        // The root's bottom row, from the last of neighbouring runs of one component in a row
        // (a neighbour's parent equal to r means the same component: r is a root).
        const int y = g.ry[j];
        const bool last = j + 1 == n || int(g.ry[j + 1]) != y || __atomic_load_n(g.root + j + 1, __ATOMIC_RELAXED) != r;
        if (r != j && last) atomicMax(g.cbot + r, y);
    }
}

// Component records and row slots: slot blocks are handed out in whatever order the roots come,
// the records carry each block's start, and the host orders the records by first run.
__global__ __launch_bounds__(256) void ccl_comps_kernel(const CclParams p) {
    const CclPage &g = p.pg[blockIdx.y];
    const int n = g.row_off[g.h];
    if (n > g.cap) return;
    for (int j = int(blockIdx.x) * 256 + int(threadIdx.x); j < n; j += int(gridDim.x) * 256) {
        if (g.root[j] != j) continue;
        const int top = g.ry[j], rows = g.cbot[j] - top + 1;
        const int k = atomicAdd(g.total + 1, 1), b = atomicAdd(g.total + 2, rows);
        g.cbot[j] = b;
        if (k < g.ccap) {
            int4 rec;
            rec.x = j, rec.y = top, rec.z = rows, rec.w = b;
            reinterpret_cast<int4 *>(g.comps)[k] = rec;
        }
        if (b + rows <= g.scap)
            for (int i = b; i < b + rows; i++) g.xmin[i] = 0xffffu, g.xmax[i] = 0u;
    }
}

__global__ __launch_bounds__(256) void ccl_extremes_kernel(const CclParams p) {
    const CclPage &g = p.pg[blockIdx.y];
    const int n = g.row_off[g.h];
    if (n > g.cap || g.total[1] > g.ccap || g.total[2] > g.scap) return;
    for (int j = int(blockIdx.x) * 256 + int(threadIdx.x); j < n; j += int(gridDim.x) * 256) {
        const int r = g.root[j], y = g.ry[j];
        // Runs of a row go left to right: of neighbouring runs of one component in one row only
        // the first can hold its leftmost pixel and only the last its rightmost.
        const bool first = j == 0 || int(g.ry[j - 1]) != y || g.root[j - 1] != r;
        const bool last = j + 1 == n || int(g.ry[j + 1]) != y || g.root[j + 1] != r;
        if (!first && !last) continue;
        const int slot = g.cbot[r] + y - int(g.ry[r]);
        if (first) atomicMin(g.xmin + slot, uint32_t(g.x0[j]));
        if (last) atomicMax(g.xmax + slot, uint32_t(g.x1[j]));
    }
}

}  // namespace

void ccl_runs(const CclPage *pages, int count, hipStream_t s) {
    for (int k0 = 0; k0 < count; k0 += CCL_MAXPAGES) {
        CclParams p{};
        const int cnt = std::min(CCL_MAXPAGES, count - k0);
        int maxh = 0, maxcap = 0;
        double bytes = 0;
        for (int k = 0; k < cnt; k++) {
            const CclPage &g = pages[k0 + k];
            if (g.w < 1 || g.h < 1 || g.w > 65536 || g.h > 65536 || g.cap < 1 || g.ccap < 1 || g.scap < 1)
                fail("ccl_runs: page size or capacity");
            p.pg[k] = g;
            maxh = std::max(maxh, g.h);
            maxcap = std::max(maxcap, g.cap);
            bytes += 4.0 * double((g.w + 31) / 32) * g.h;
        }
        ProbeScope probe("ccl", s, 0, bytes);
        const dim3 rows(unsigned((maxh + 3) / 4), unsigned(cnt));
        hipLaunchKernelGGL(ccl_count_kernel, rows, dim3(256), 0, s, p);
        hipLaunchKernelGGL(ccl_scan_kernel, dim3(unsigned(cnt)), dim3(1024), 0, s, p);
        hipLaunchKernelGGL(ccl_runs_kernel, rows, dim3(256), 0, s, p);
        // A thread per run (up to the capacity; threads past a page's run count return).
        const dim3 runs_grid(unsigned(std::min(2048, (maxcap + 255) / 256)), unsigned(cnt));
        const unsigned bands = unsigned((maxh + CCL_BAND - 1) / CCL_BAND);
        hipLaunchKernelGGL(ccl_union_band_kernel, dim3(bands, unsigned(cnt)), dim3(512), 0, s, p);
        if (bands > 1) hipLaunchKernelGGL(ccl_union_bounds_kernel, dim3(bands - 1, unsigned(cnt)), dim3(256), 0, s, p);
        hipLaunchKernelGGL(ccl_flatten_kernel, runs_grid, dim3(256), 0, s, p);
        hipLaunchKernelGGL(ccl_comps_kernel, runs_grid, dim3(256), 0, s, p);
        hipLaunchKernelGGL(ccl_extremes_kernel, runs_grid, dim3(256), 0, s, p);
        OCR_HIP(hipGetLastError());
    }
}

}  // namespace ocr
