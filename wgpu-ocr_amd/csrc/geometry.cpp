#include "geometry.h"

#include "host_util.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <string>
#include <thread>

namespace ocr {

// ocr-bench.rs:31: class k > 0 is this string's character k - 1 (96 characters; class 0 blank).
const char *const OCRS_ALPHABET =
    " 0123456789!\"#$%&'()*+,-./:;<=>?@[\\]^_`{|}~EABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz";

void RRect::corners(float xs[4], float ys[4]) const {
    const float hx = ux * h / 2, hy = uy * h / 2, wx = rx() * w / 2, wy = ry() * w / 2;
    xs[0] = cx + hx - wx, ys[0] = cy + hy - wy;  // top-left
    xs[1] = cx + hx + wx, ys[1] = cy + hy + wy;  // top-right
    xs[2] = cx - hx + wx, ys[2] = cy - hy + wy;  // bottom-right
    xs[3] = cx - hx - wx, ys[3] = cy - hy - wy;  // bottom-left
}

void RRect::bbox(float &l, float &t, float &r, float &b) const {
    float xs[4], ys[4];
    corners(xs, ys);
    l = *std::min_element(xs, xs + 4);
    r = *std::max_element(xs, xs + 4);
    t = *std::min_element(ys, ys + 4);
    b = *std::max_element(ys, ys + 4);
}

bool RRect::upright() const { return std::fabs(uy) >= std::fabs(ux); }

namespace {

struct Pt {
    float x, y;
};

// ---- Word boxes: outer contours, simplification, minimum-area rectangles -------------------
// The steps of ocr-bench.rs:47-58 (find_contours External, simplify_polygon(2), min_area_rect of
// rten-imageproc 0.26.0), restated from the algorithms they publish (the crate is not vendored):
// Suzuki-Abe border following, Ramer-Douglas-Peucker, and the rectangle with a side on a convex
// hull edge. The arithmetic is float32 in a fixed order, the same rectangles bit for bit as the
// oracle's independent restatement.

// Directions 0 E, 1 NE, 2 N, 3 NW, 4 W, 5 SW, 6 S, 7 SE (y down); +1 turns counter-clockwise on
// the page.
constexpr int DIR_X[8] = {1, 1, 0, -1, -1, -1, 0, 1};
constexpr int DIR_Y[8] = {0, -1, -1, -1, 0, 1, 1, 1};

// A bit mask copied with a frame of zeros: one row above and below, one word left and right,
// and the bits past the mask width cleared (the padding of the border following), so a pixel's
// neighbours are read with no bounds checks.
struct PaddedMask {
    std::vector<uint32_t> p;
    size_t stride = 0;  // words a padded row
    void build(const uint32_t *bits, int w, int h) {
        const int words = (w + 31) / 32;
        stride = size_t(words) + 2;
        p.assign(stride * (size_t(h) + 2) + 1, 0u);  // one spare word for the last 64-bit read
        const uint32_t last = (w & 31) ? (1u << (w & 31)) - 1u : ~0u;
        for (int y = 0; y < h; y++) {
            uint32_t *dst = p.data() + (size_t(y) + 1) * stride + 1;
            std::memcpy(dst, bits + size_t(y) * size_t(words), size_t(words) * 4);
            dst[words - 1] &= last;
        }
    }
    // The 3 x 3 block around (x, y): row y - 1 in bits 0..2, row y in 3..5, row y + 1 in 6..8
    // (pixel x - 1 first in each).
    uint32_t block(int x, int y) const {
        const int b = x + 31;  // bit of pixel x - 1 in the padded row
        const uint32_t *row = p.data() + (size_t(y) + 1) * stride + size_t(b >> 5);
        const int sh = b & 31;
        uint64_t u, m, d;
        std::memcpy(&u, row - stride, 8);
        std::memcpy(&m, row, 8);
        std::memcpy(&d, row + stride, 8);
        return (uint32_t(u >> sh) & 7u) | (uint32_t(m >> sh) & 7u) << 3 | (uint32_t(d >> sh) & 7u) << 6;
    }
};

// The neighbour ring (bits 0..7 in direction order) of a 3 x 3 block.
constexpr uint32_t block_ring(uint32_t b) {
    return ((b >> 5) & 1u) | ((b >> 2) & 1u) << 1 | ((b >> 1) & 1u) << 2 | (b & 1u) << 3 | ((b >> 3) & 1u) << 4 |
           ((b >> 6) & 1u) << 5 | ((b >> 7) & 1u) << 6 | ((b >> 8) & 1u) << 7;
}

// Steps (3.3)-(3.4) of the border following as one table lookup: for a pixel's 3 x 3 block and
// the direction dprev of the pixel it came from, the first set neighbour counter-clockwise after
// dprev, given as the move there (dx + 1 in bits 0-1, dy + 1 in bits 2-3) and the direction from
// that neighbour back to the pixel (bits 4-6), the next step's dprev. The ring always holds dprev;
// entries where it does not are never read.
struct BorderStep {
    uint8_t t[512 * 8];
    BorderStep() {
        for (uint32_t b = 0; b < 512; b++) {
            const uint32_t r = block_ring(b);
            for (int d = 0; d < 8; d++) {
                int n = d;
                for (int k = 1; k <= 8; k++)
                    if ((r >> ((d + k) & 7)) & 1u) {
                        n = (d + k) & 7;
                        break;
                    }
                t[b * 8 + uint32_t(d)] = uint8_t((DIR_X[n] + 1) | (DIR_Y[n] + 1) << 2 | ((n + 4) & 7) << 4);
            }
        }
    }
};
const BorderStep BORDER_STEP;

// The outer borders of the 8-connected components seeds[lo, hi), each given by its raster-first
// pixel (fx, fy): the pixels Suzuki-Abe border following visits (steps 3.1-3.5: from the west
// neighbour clockwise to the first set pixel, then from each pixel counter-clockwise after the
// one it came from), x, y pairs in visiting order, starting at the first pixel; a lone pixel is
// its own border. done(i, xy) gets component i's border as it closes (in no fixed order; xy is
// reused afterwards). TRACE_LANES borders are followed side by side on the calling thread: each
// is a chain of dependent loads, and independent chains interleaved keep the core busy.
constexpr int TRACE_LANES = 4;
template <class Seeds, class F>
void trace_outer_many(const PaddedMask &m, const Seeds &seeds, int lo, int hi,
                      std::vector<int32_t> (&buf)[TRACE_LANES], F &&done) {
    struct Lane {
        int i, x0, y0, x1, y1, x, y;
        uint32_t dprev, b;
        std::vector<int32_t> *xy;
    };
    Lane lane[TRACE_LANES];
    int nl = 0, next = lo;
    // Puts the next component with more than one border pixel on l (the others are done at
    // once); false when none is left.
    auto start = [&](Lane &l, std::vector<int32_t> *xy) {
        while (next < hi) {
            const int i = next++;
            const int x0 = seeds[size_t(i)].fx, y0 = seeds[size_t(i)].fy;
            xy->clear();
            xy->push_back(x0), xy->push_back(y0);
            const uint32_t b0 = m.block(x0, y0), r0 = block_ring(b0);
            if (!r0) {
                done(i, *xy);
                continue;
            }
            int d1 = 4;
            while (!((r0 >> d1) & 1u)) d1 = (d1 + 7) & 7;  // clockwise from the west
            l = Lane{i, x0, y0, x0 + DIR_X[d1], y0 + DIR_Y[d1], x0, y0, uint32_t(d1), b0, xy};
            return true;
        }
        return false;
    };
    for (int k = 0; k < TRACE_LANES; k++)
        if (start(lane[nl], &buf[k])) nl++;
    while (nl > 0) {
        for (int k = 0; k < nl; k++) {
            Lane &l = lane[k];
            const uint32_t e = BORDER_STEP.t[l.b * 8 + l.dprev];
            const int x = l.x + int(e & 3u) - 1, y = l.y + int((e >> 2) & 3u) - 1;
            if (x == l.x0 && y == l.y0 && l.x == l.x1 && l.y == l.y1) {
                // Back at the start, about to take the first step again: the border is closed.
                done(l.i, *l.xy);
                if (!start(l, l.xy)) lane[k--] = lane[--nl];
                continue;
            }
            l.dprev = e >> 4, l.x = x, l.y = y;
            l.xy->push_back(x), l.xy->push_back(y);
            l.b = m.block(x, y);
        }
    }
}

// Squared distances from the points k in (s, e) (coordinates px, py) to the segment between
// points s and e (from point s when the segment is a point), into d2[k]: the float operations of
// the distance itself up to its square root, so sqrt(d2[k]) is that distance bit for bit. Eight
// points at a time, the last block running up to 7 points past e (px, py and d2 hold them; their
// lanes are left out of the maximum). Returns the largest d2 of (s, e), 0 when it is empty (max is
// exact in any order). Built for AVX2 and for the baseline ISA (the loader picks one); the same
// IEEE operations either way, no fused multiply-adds. (Host code only: the device pass of this
// file compiles nothing.)
#if defined(__HIP_DEVICE_COMPILE__)
#define OCR_HOST_CLONES
#else
#define OCR_HOST_CLONES __attribute__((target_clones("avx2", "default")))
#endif
typedef float F8 __attribute__((vector_size(32)));
typedef int I8 __attribute__((vector_size(32)));
constexpr int SEG_PAD = 8;  // readable floats past the last point of px, py and d2

OCR_HOST_CLONES
float seg_dist2_max(const float *__restrict px, const float *__restrict py, int s, int e, float *__restrict d2) {
#if defined(__clang__)
#pragma clang fp contract(off)
#endif
    const float ax = px[s], ay = py[s], bx = px[e], by = py[e];
    const int k0 = s + 1, cnt = e - s - 1;
    const F8 zero = {}, vax = ax + zero, vay = ay + zero, vbx = bx + zero, vby = by + zero;
    const I8 lane = {0, 1, 2, 3, 4, 5, 6, 7};
    const bool point = ax == bx && ay == by;
    const float abx = bx - ax, aby = by - ay, den = abx * abx + aby * aby;
    const F8 vabx = abx + zero, vaby = aby + zero, vden = den + zero;
    F8 mx = zero;
    for (int i = 0; i < cnt; i += 8) {
        F8 x, y, d;
        std::memcpy(&x, px + k0 + i, sizeof x);
        std::memcpy(&y, py + k0 + i, sizeof y);
        if (point) {
            const F8 dx = x - vax, dy = y - vay;
            d = dx * dx + dy * dy;
        } else {
            // Both ends and the projection computed, then selected.
            const F8 acx = x - vax, acy = y - vay;
            const F8 t = (acx * vabx + acy * vaby) / vden;
            F8 qx = vax + vabx * t, qy = vay + vaby * t;
            qx = t >= 1.f ? vbx : qx, qy = t >= 1.f ? vby : qy;
            qx = t <= 0.f ? vax : qx, qy = t <= 0.f ? vay : qy;
            const F8 dx = x - qx, dy = y - qy;
            d = dx * dx + dy * dy;
        }
        std::memcpy(d2 + k0 + i, &d, sizeof d);
        const F8 dm = lane < cnt - i ? d : zero;
        mx = dm > mx ? dm : mx;
    }
    float m = mx[0];
    for (int j = 1; j < 8; j++) m = mx[j] > m ? mx[j] : m;
    return m;
}

// Scratch of simplify_closed, kept per thread.
struct SimplifyScratch {
    std::vector<float> px, py, d2;
    std::vector<unsigned char> keep;
    std::vector<std::pair<int, int>> stack;
};

// simplify_polygon(points, eps): Ramer-Douglas-Peucker on the closed polygon (the first point
// appended, then dropped): a run splits at its farthest inner point from the segment between its
// ends (distance to the segment, from its first point when it is a point; the last of equally
// far points) when that is farther than eps. The largest distance is the root of the largest
// squared one; the points as far as it are those whose squared distance has that same root,
// which (sqrt being monotonic and correctly rounded) are the ones at or above the smallest float
// with that root: the split is the last of them.
void simplify_closed(const std::vector<int32_t> &xy, float eps, std::vector<Pt> &out, SimplifyScratch &S) {
    const int n = int(xy.size() / 2);
    out.clear();
    if (n == 0) return;
    const size_t len = size_t(n) + 1 + SEG_PAD;
    S.px.resize(len), S.py.resize(len), S.d2.resize(len);
    float *px = S.px.data(), *py = S.py.data(), *d2 = S.d2.data();
    for (int k = 0; k < n; k++) px[k] = float(xy[size_t(2 * k)]), py[k] = float(xy[size_t(2 * k + 1)]);
    for (size_t k = size_t(n); k < len; k++) px[k] = px[0], py[k] = py[0];
    S.keep.assign(size_t(n) + 1, 0);
    S.stack.assign(1, {0, n});
    while (!S.stack.empty()) {
        const auto [s, e] = S.stack.back();
        S.stack.pop_back();
        S.keep[size_t(s)] = S.keep[size_t(e)] = 1;
        if (e - s < 2) continue;
        const float m2 = seg_dist2_max(px, py, s, e, d2);
        const float dmax = std::sqrt(m2);
        if (!(dmax > eps)) continue;
        // The smallest float whose root is dmax: step down one ulp at a time (a root's preimage
        // spans a few floats); below a positive float lies its bit pattern less one.
        float lo = m2;
        while (lo > 0.f) {
            uint32_t u;
            std::memcpy(&u, &lo, 4);
            float below;
            u -= 1;
            std::memcpy(&below, &u, 4);
            if (std::sqrt(below) != dmax) break;
            lo = below;
        }
        // The last point at or above lo: eight at a time from the end while every lane is below.
        // One exists (the largest), so the scan stops inside (s, e).
        int best = e - 1;
        while (best - 7 > s) {
            F8 v;
            std::memcpy(&v, d2 + best - 7, sizeof v);
            const I8 hit = v >= lo;
            int any = 0;
            for (int j = 0; j < 8; j++) any |= hit[j];
            if (any) break;
            best -= 8;
        }
        while (d2[best] < lo) best--;
        S.stack.push_back({best, e});
        S.stack.push_back({s, best});
    }
    for (int k = 0; k < n; k++)
        if (S.keep[size_t(k)]) out.push_back({px[k], py[k]});
}

double cross(const Pt &o, const Pt &a, const Pt &b) {
    return (double(a.x) - o.x) * (double(b.y) - o.y) - (double(a.y) - o.y) * (double(b.x) - o.x);
}

// Convex hull (Andrew's monotone chain): counter-clockwise in the sense cross > 0 from the point
// with the smallest (x, y), collinear points dropped, the first point not repeated.
void convex_hull(std::vector<Pt> p, std::vector<Pt> &h) {
    std::sort(p.begin(), p.end(), [](const Pt &a, const Pt &b) { return a.x < b.x || (a.x == b.x && a.y < b.y); });
    p.erase(std::unique(p.begin(), p.end(), [](const Pt &a, const Pt &b) { return a.x == b.x && a.y == b.y; }),
            p.end());
    h.clear();
    if (p.size() <= 2) {
        h = p;
        return;
    }
    h.resize(2 * p.size());
    size_t k = 0;
    for (size_t i = 0; i < p.size(); i++) {
        while (k >= 2 && cross(h[k - 2], h[k - 1], p[i]) <= 0) k--;
        h[k++] = p[i];
    }
    for (size_t i = p.size() - 1, t = k + 1; i-- > 0;) {
        while (k >= t && cross(h[k - 2], h[k - 1], p[i]) <= 0) k--;
        h[k++] = p[i];
    }
    h.resize(k - 1);
}

// min_area_rect: of the rectangles with a side on an edge of the convex hull (edges in hull
// order), the first of the smallest area, then turned by a multiple of 90 degrees so its up axis
// points most towards -y (the last of equally good turns: up, +90, +180, +270). False when the
// points hold fewer than two distinct positions.
bool min_area_rect(const std::vector<Pt> &pts, std::vector<Pt> &hull, RRect &out) {
    convex_hull(pts, hull);
    const size_t m = hull.size();
    bool found = false;
    float best = INFINITY;
    for (size_t i = 0; i < m && m >= 2; i++) {
        const float ax = hull[i].x, ay = hull[i].y, bx = hull[(i + 1) % m].x, by = hull[(i + 1) % m].y;
        float ex = bx - ax, ey = by - ay;
        const float len = std::sqrt(ex * ex + ey * ey);
        if (len == 0.f) continue;
        ex /= len, ey /= len;
        const float nx = -ey, ny = ex;  // into the hull
        float pmin = INFINITY, pmax = -INFINITY, qmax = -INFINITY;
        for (size_t k = 0; k < m; k++) {
            const float dx = hull[k].x - ax, dy = hull[k].y - ay;
            const float par = dx * ex + dy * ey, perp = dx * nx + dy * ny;
            if (par < pmin) pmin = par;
            if (par > pmax) pmax = par;
            if (perp > qmax) qmax = perp;
        }
        const float width = pmax - pmin, height = qmax, area = width * height;
        if (area < best) {
            best = area;
            found = true;
            const float mid = (pmin + pmax) / 2.f, half = height / 2.f;
            out.cx = ax + ex * mid + nx * half;
            out.cy = ay + ey * mid + ny * half;
            out.ux = nx, out.uy = ny, out.w = width, out.h = height;
        }
    }
    if (!found) return false;
    const float ux = out.ux, uy = out.uy, w = out.w, h = out.h;
    const float cand[4][2] = {{ux, uy}, {uy, -ux}, {-ux, -uy}, {-uy, ux}};
    int k = 0;
    for (int c = 1; c < 4; c++)
        if (-cand[c][1] >= -cand[k][1]) k = c;
    out.ux = cand[k][0], out.uy = cand[k][1];
    out.w = (k & 1) ? h : w;
    out.h = (k & 1) ? w : h;
    return true;
}

struct Run {
    int y, x0, x1;  // inclusive pixel range in row y
};

int find(std::vector<int> &parent, int a) {
    while (parent[a] != a) a = parent[a] = parent[parent[a]];
    return a;
}

}  // namespace

namespace {

// The 8-connected components of rows [y0, y1) of a bit mask (ceil(w / 32) words a row), each as
// its rows' leftmost and rightmost pixels, rows ascending (its first pixel and bounding box), in
// order of their first run; and the runs of the first and last rows with their components, for
// joining neighbouring bands.
struct BandComps {
    std::vector<std::vector<Pt>> pts;
    std::vector<Run> first, last;
    std::vector<int> first_c, last_c;
};

BandComps band_components(const uint32_t *bits, int w, int y0, int y1) {
    const int words = (w + 31) / 32, h = y1 - y0;
    const uint32_t last_mask = (w & 31) ? (1u << (w & 31)) - 1 : ~0u;
    std::vector<Run> runs;
    runs.reserve(size_t(h) * 16);
    std::vector<int> row_start(size_t(h) + 1, 0);
    for (int y = y0; y < y1; y++) {
        row_start[size_t(y - y0)] = int(runs.size());
        const uint32_t *row = bits + size_t(y) * words;
        uint32_t any = row[words - 1] & last_mask;
        for (int wi = 0; wi + 1 < words; wi++) any |= row[wi];
        if (!any) continue;
        // Runs from the row's bit transitions: bit b of t is set where pixel b differs from
        // pixel b - 1 (pixel -1 and pixels past w are background).
        int start = -1;
        uint32_t prev = 0;
        for (int wi = 0; wi < words; wi++) {
            const uint32_t word = wi + 1 == words ? row[wi] & last_mask : row[wi];
            uint32_t t = word ^ ((word << 1) | prev);
            prev = word >> 31;
            while (t) {
                const int b = __builtin_ctz(t);
                t &= t - 1;
                const int x = (wi << 5) + b;
                if ((word >> b) & 1u) {
                    start = x;
                } else {
                    runs.push_back({y, start, x - 1});
                    start = -1;
                }
            }
        }
        if (start >= 0) runs.push_back({y, start, w - 1});
    }
    row_start[size_t(h)] = int(runs.size());
    // Union the runs of neighbouring rows that touch with 8-connectivity. A parent always has a
    // smaller index than its child (roots link to the smaller root; a run still alone joins
    // the root of the run above it).
    std::vector<int> parent(runs.size());
    std::iota(parent.begin(), parent.end(), 0);
    for (int y = 1; y < h; y++) {
        int i = row_start[size_t(y) - 1], j = row_start[size_t(y)];
        const int ie = row_start[size_t(y)], je = row_start[size_t(y) + 1];
        while (i < ie && j < je) {
            const Run &a = runs[size_t(i)], &b = runs[size_t(j)];
            if (a.x1 + 1 >= b.x0 && b.x1 + 1 >= a.x0) {
                if (parent[size_t(j)] == j) {
                    parent[size_t(j)] = find(parent, i);
                } else {
                    const int ra = find(parent, i), rb = find(parent, j);
                    if (ra != rb) parent[size_t(std::max(ra, rb))] = std::min(ra, rb);
                }
            }
            if (a.x1 < b.x1) i++;
            else j++;
        }
    }
    // Every run's root in one forward pass (its parent's root is already final).
    for (size_t r = 0; r < runs.size(); r++) parent[r] = parent[size_t(parent[r])];
    // Row extremes per component (components in order of their first run). Runs are listed row
    // by row and left to right, so a component's later run in the same row only moves its right
    // end.
    BandComps out;
    std::vector<int> comp(runs.size(), -1), run_comp(runs.size());
    // Component ids in order of first run, and room for two points a row.
    std::vector<int> npts, last_y;
    for (size_t r = 0; r < runs.size(); r++) {
        const int root = parent[r];
        if (comp[size_t(root)] < 0) {
            comp[size_t(root)] = int(npts.size());
            npts.push_back(0);
            last_y.push_back(-1);
        }
        const int c = comp[size_t(root)];
        run_comp[r] = c;
        if (last_y[size_t(c)] != runs[r].y) npts[size_t(c)] += 2, last_y[size_t(c)] = runs[r].y;
    }
    out.pts.resize(npts.size());
    for (size_t c = 0; c < npts.size(); c++) out.pts[c].reserve(size_t(npts[c]));
    for (size_t r = 0; r < runs.size(); r++) {
        auto &v = out.pts[size_t(run_comp[r])];
        const float y = float(runs[r].y), x0 = float(runs[r].x0), x1 = float(runs[r].x1);
        const bool same_row = !v.empty() && v.back().y == y;
        if (same_row) {
            // the row holds (left) or (left, right): the new right end replaces the old one
            if (v.size() >= 2 && v[v.size() - 2].y == y) v.back().x = x1;
            else if (x1 != v.back().x) v.push_back({x1, y});
        } else {
            v.push_back({x0, y});
            if (x1 != x0) v.push_back({x1, y});
        }
    }
    if (h > 0) {
        for (int r = row_start[0]; r < row_start[1]; r++) out.first.push_back(runs[size_t(r)]), out.first_c.push_back(run_comp[size_t(r)]);
        for (int r = row_start[size_t(h) - 1]; r < row_start[size_t(h)]; r++)
            out.last.push_back(runs[size_t(r)]), out.last_c.push_back(run_comp[size_t(r)]);
    }
    return out;
}

// Row extremes of one component made of several band components: per row the leftmost and the
// rightmost pixel of all of them (the right one only when it differs), rows ascending.
std::vector<Pt> merge_rows(std::vector<Pt> all) {
    std::stable_sort(all.begin(), all.end(), [](const Pt &a, const Pt &b) { return a.y < b.y; });
    std::vector<Pt> out;
    for (size_t i = 0; i < all.size();) {
        size_t j = i;
        float lo = all[i].x, hi = all[i].x;
        for (; j < all.size() && all[j].y == all[i].y; j++) lo = std::min(lo, all[j].x), hi = std::max(hi, all[j].x);
        out.push_back({lo, all[i].y});
        if (hi != lo) out.push_back({hi, all[i].y});
        i = j;
    }
    return out;
}

thread_local int t_loop_prio = 0;

// fn(lo, hi) over contiguous ranges covering [0, n): the whole range on the calling thread when
// threads is 1, else up to 4 ranges a thread (for balance) on the caller and the shared loop pool,
// at this thread's loop priority.
template <class F> void parallel_ranges(int n, int threads, F fn) {
    threads = std::max(1, std::min(threads, n));
    if (threads == 1) {
        if (n > 0) fn(0, n);
        return;
    }
    const int chunks = std::min(n, 4 * threads);
    LoopPool::get().run(
        chunks, [&](int t) { fn(int(long(n) * t / chunks), int(long(n) * (t + 1) / chunks)); }, t_loop_prio);
}

// fn(i) for i in [0, n), as parallel_ranges cuts it.
template <class F> void parallel_for(int n, int threads, F fn) {
    parallel_ranges(n, threads, [&](int lo, int hi) {
        for (int i = lo; i < hi; i++) fn(i);
    });
}

}  // namespace

void set_loop_priority(int prio) { t_loop_prio = prio; }

// Every 8-connected component of a bit mask (h rows of ceil(w / 32) words) as its rows'
// leftmost and rightmost pixels, rows ascending, in order of its first run (row-major). With
// several threads the rows are cut into bands labelled on their own, then the components that
// meet across a cut are joined (the same components, in the same order).
static std::vector<std::vector<Pt>> component_points(const uint32_t *bits, int w, int h, int threads = 1) {
    const int bands = std::max(1, std::min(threads, h / 64));
    if (bands == 1) return band_components(bits, w, 0, h).pts;
    std::vector<BandComps> B(static_cast<size_t>(bands));
    parallel_for(bands, bands, [&](int b) {
        B[size_t(b)] = band_components(bits, w, int(long(h) * b / bands), int(long(h) * (b + 1) / bands));
    });
    std::vector<int> off(static_cast<size_t>(bands) + 1, 0);
    for (int b = 0; b < bands; b++) off[size_t(b) + 1] = off[size_t(b)] + int(B[size_t(b)].pts.size());
    std::vector<int> parent(static_cast<size_t>(off[size_t(bands)]));
    std::iota(parent.begin(), parent.end(), 0);
    for (int b = 0; b + 1 < bands; b++) {
        const BandComps &A = B[size_t(b)], &C = B[size_t(b) + 1];
        size_t i = 0, j = 0;
        while (i < A.last.size() && j < C.first.size()) {
            const Run &a = A.last[i], &c = C.first[j];
            if (a.x1 + 1 >= c.x0 && c.x1 + 1 >= a.x0) {
                int ra = find(parent, off[size_t(b)] + A.last_c[i]), rc = find(parent, off[size_t(b) + 1] + C.first_c[j]);
                if (ra != rc) parent[size_t(std::max(ra, rc))] = std::min(ra, rc);
            }
            if (a.x1 < c.x1) i++;
            else j++;
        }
    }
    std::vector<int> gid(parent.size(), -1);
    std::vector<std::vector<int>> members;
    for (int k = 0; k < int(parent.size()); k++) {
        const int root = find(parent, k);
        if (gid[size_t(root)] < 0) {
            gid[size_t(root)] = int(members.size());
            members.emplace_back();
        }
        members[size_t(gid[size_t(root)])].push_back(k);
    }
    std::vector<std::vector<Pt>> out(members.size());
    auto local = [&](int k) -> std::vector<Pt> & {
        const int b = int(std::upper_bound(off.begin(), off.end(), k) - off.begin()) - 1;
        return B[size_t(b)].pts[size_t(k - off[size_t(b)])];
    };
    for (size_t m = 0; m < members.size(); m++) {
        if (members[m].size() == 1) {
            out[m] = std::move(local(members[m][0]));
            continue;
        }
        std::vector<Pt> all;
        for (int k : members[m]) all.insert(all.end(), local(k).begin(), local(k).end());
        out[m] = merge_rows(std::move(all));
    }
    return out;
}

namespace {

// A component to trace: its raster-first pixel (the leftmost of its top row) and bounding box.
struct Seed {
    int fx, fy, x0, y0, x1, y1;
};

Seed seed_of_rows(const std::vector<Pt> &v) {
    Seed s{int(v[0].x), int(v[0].y), int(v[0].x), int(v[0].y), int(v[0].x), int(v[0].y)};
    for (const Pt &p : v) {
        s.x0 = std::min(s.x0, int(p.x)), s.x1 = std::max(s.x1, int(p.x));
        s.y0 = std::min(s.y0, int(p.y)), s.y1 = std::max(s.y1, int(p.y));
    }
    return s;
}

// Whether the outer border xy (a closed chain of 8-neighbours) winds around the pixel (qx, qy) an
// odd number of times: the chain's steps across rows qy..qy+1 whose end on row qy lies left of qx.
bool encloses(const std::vector<int32_t> &xy, int qx, int qy) {
    const size_t n = xy.size() / 2;
    bool odd = false;
    for (size_t k = 0; k < n; k++) {
        const size_t j = k + 1 == n ? 0 : k + 1;
        const int ay = xy[2 * k + 1], by = xy[2 * j + 1];
        if ((ay > qy) != (by > qy)) {
            const int x = ay <= qy ? xy[2 * k] : xy[2 * j];
            if (x < qx) odd = !odd;
        }
    }
    return odd;
}

// The rectangles of the external components (ocr-bench.rs:47-55: find_contours External,
// simplify_polygon(2), min_area_rect), given every 8-connected component of the mask by its seed
// in raster order of first pixels; ok[i] is false for a component inside a hole of another one
// and for one without a rectangle (a single pixel).
//
// A component is external when the background pixel west of its first pixel belongs to the
// background reaching the frame. That pixel lies in a hole of some component exactly when an
// outer border winds around it (a 4-connected background path cannot cross an outer border
// through 8-neighbouring pixel centres), and the component whose hole it is spans it strictly in
// both axes and comes earlier in raster order: only those are tested.
void external_rects(const uint32_t *bits, int w, int h, const std::vector<Seed> &seeds, int threads,
                    std::vector<RRect> &rects, std::vector<char> &ok) {
    PaddedMask m;  // read by the worker threads too
    m.build(bits, w, h);
    const int n = int(seeds.size());
    // Components that could enclose the pixel west of a component's first pixel: earlier ones
    // (in raster order) whose bounding box holds it strictly. Rare on text pages.
    std::vector<std::pair<int, int>> cand;  // (component, possible encloser)
    std::vector<char> encloser(size_t(n), 0);
    std::vector<int> active;  // earlier components whose rows reach below the current row
    for (int i = 0; i < n; i++) {
        const Seed &c = seeds[size_t(i)];
        const int qx = c.fx - 1, qy = c.fy;
        size_t keep = 0;
        for (int j : active)
            if (seeds[size_t(j)].y1 > qy) active[keep++] = j;
        active.resize(keep);
        if (qx >= 0)
            for (int j : active) {
                const Seed &d = seeds[size_t(j)];
                if (d.y0 < qy && d.x0 < qx && qx < d.x1) cand.push_back({i, j}), encloser[size_t(j)] = 1;
            }
        active.push_back(i);
    }
    // Every component's border, simplification and rectangle in one pass; the borders of
    // possible enclosers are kept for the winding test.
    std::vector<std::vector<int32_t>> chains(static_cast<size_t>(n));
    rects.assign(size_t(n), RRect{});
    ok.assign(size_t(n), 1);
    parallel_ranges(n, threads, [&](int lo, int hi) {
        thread_local std::vector<int32_t> buf[TRACE_LANES];
        thread_local std::vector<Pt> simp, hull;
        thread_local SimplifyScratch scratch;
        trace_outer_many(m, seeds, lo, hi, buf, [&](int i, const std::vector<int32_t> &xy) {
            if (encloser[size_t(i)]) chains[size_t(i)] = xy;
            simplify_closed(xy, 2.f, simp, scratch);
            if (!min_area_rect(simp, hull, rects[size_t(i)])) ok[size_t(i)] = 0;
        });
    });
    // A component inside a hole of another one is left out (an outer border winds around the
    // background pixel west of its first pixel).
    for (const auto &[i, j] : cand)
        if (ok[size_t(i)] && encloses(chains[size_t(j)], seeds[size_t(i)].fx - 1, seeds[size_t(i)].fy)) ok[size_t(i)] = 0;
}

std::vector<RRect> grown_rects(const uint32_t *bits, int w, int h, const std::vector<Seed> &seeds, float expand,
                               float min_area, int threads) {
    std::vector<RRect> rects;
    std::vector<char> ok;
    external_rects(bits, w, h, seeds, threads, rects, ok);
    std::vector<RRect> out;
    for (size_t i = 0; i < rects.size(); i++) {
        if (!ok[i]) continue;
        RRect r = rects[i];
        r.resize(r.w + 2 * expand, r.h + 2 * expand);
        if (r.area() >= min_area) out.push_back(r);
    }
    return out;
}

}  // namespace

std::vector<RRect> word_rects(const uint32_t *bits, int w, int h, float expand, float min_area, int threads) {
    const auto comps = component_points(bits, w, h, threads);
    std::vector<Seed> seeds;
    seeds.reserve(comps.size());
    for (const auto &v : comps) seeds.push_back(seed_of_rows(v));
    return grown_rects(bits, w, h, seeds, expand, min_area, threads);
}

std::vector<RRect> word_rects_from_rows(const uint32_t *bits, int w, int h, const int32_t *comps, int ncomps,
                                        const uint32_t *xmin, const uint32_t *xmax, int nslots, float expand,
                                        float min_area, int threads) {
    // Components in order of first run (row-major): the order of their first pixels.
    std::vector<int> order(size_t(std::max(ncomps, 0)));
    for (int c = 0; c < ncomps; c++) order[size_t(c)] = c;
    std::sort(order.begin(), order.end(), [&](int a, int b) { return comps[4 * a] < comps[4 * b]; });
    std::vector<Seed> seeds(order.size());
    for (size_t k = 0; k < order.size(); k++) {
        const int32_t *rec = comps + 4 * order[k];
        const int top = rec[1], rows = rec[2], b = rec[3];
        if (rows < 1 || b < 0 || b + rows > nslots || top < 0 || top + rows > h)
            fail("word_rects_from_rows: a component's row slots");
        Seed &s = seeds[k];
        s.fx = int(xmin[b]), s.fy = top, s.y0 = top, s.y1 = top + rows - 1;
        s.x0 = INT32_MAX, s.x1 = -1;
        for (int r = 0; r < rows; r++) {
            const uint32_t x0 = xmin[b + r], x1 = xmax[b + r];
            if (x0 > x1 || x1 >= uint32_t(w)) fail("word_rects_from_rows: a component row without pixels");
            s.x0 = std::min(s.x0, int(x0)), s.x1 = std::max(s.x1, int(x1));
        }
        // The border following starts at a set pixel whose west neighbour is clear (a walk from
        // anywhere else need not come back to its start).
        const int words = (w + 31) / 32;
        auto bit = [&](int x, int y) { return (bits[size_t(y) * size_t(words) + size_t(x >> 5)] >> (x & 31)) & 1u; };
        if (!bit(s.fx, s.fy) || (s.fx > 0 && bit(s.fx - 1, s.fy)))
            fail("word_rects_from_rows: a component's first pixel is not the start of a run");
    }
    return grown_rects(bits, w, h, seeds, expand, min_area, threads);
}

// ppdet.rs:65-85: the mean probability (an f32 sum in row-major order) of the map's pixels whose
// position lies inside r (its height along the up axis, its width across it), scanning r's
// bounding box.
static float db_score(const float *prob, int w, int h, const RRect &r) {
    float l, t, rr, b;
    r.bbox(l, t, rr, b);
    const int x0 = int(std::max(std::floor(l), 0.f)), y0 = int(std::max(std::floor(t), 0.f));
    const int x1 = std::min(std::max(int(std::ceil(rr)), 0), w - 1), y1 = std::min(std::max(int(std::ceil(b)), 0), h - 1);
    const float hw = r.w / 2, hh = r.h / 2;
    float sum = 0;
    long n = 0;
    for (int y = y0; y <= y1; y++)
        for (int x = x0; x <= x1; x++) {
            const float dx = float(x) - r.cx, dy = float(y) - r.cy;
            const float along_up = dx * r.ux + dy * r.uy, across = dx * -r.uy + dy * r.ux;
            if (std::fabs(along_up) <= hh && std::fabs(across) <= hw) {
                sum += prob[size_t(y) * w + x];
                n++;
            }
        }
    return n ? sum / float(n) : 0.f;
}

std::vector<RRect> db_boxes(const uint32_t *bits, const float *prob, int w, int h, float to_page_x, float to_page_y,
                            const DbParams &db) {
    const auto comps = component_points(bits, w, h);
    std::vector<Seed> seeds;
    seeds.reserve(comps.size());
    for (const auto &v : comps) seeds.push_back(seed_of_rows(v));
    std::vector<RRect> rects;
    std::vector<char> ok;
    external_rects(bits, w, h, seeds, 1, rects, ok);
    std::vector<RRect> out;
    for (size_t i = 0; i < rects.size(); i++) {
        if (!ok[i]) continue;
        const RRect &r = rects[i];
        if (std::min(r.w, r.h) < db.min_size || db_score(prob, w, h, r) < db.box_thresh) continue;
        // Unclip: grown by area * ratio / perimeter on every side (ppdet.rs:104-109).
        const float d = r.w * r.h * db.unclip_ratio / std::max(2.f * (r.w + r.h), 1e-6f);
        const float nw = r.w + 2 * d, nh = r.h + 2 * d;
        if (std::min(nw, nh) < db.min_size + 2) continue;
        const float s = (to_page_x + to_page_y) / 2;
        RRect p = r;
        p.cx = r.cx * to_page_x, p.cy = r.cy * to_page_y;
        p.w = nw * s, p.h = nh * s;
        out.push_back(p);
    }
    // Reading order (ppdet.rs:118-131): by the top edge; a box within 10 px of the previous one's
    // top moves before it when it starts further left.
    auto top = [](const RRect &r) {
        float l, t, rr, b;
        r.bbox(l, t, rr, b);
        return t;
    };
    auto left = [](const RRect &r) {
        float l, t, rr, b;
        r.bbox(l, t, rr, b);
        return l;
    };
    std::stable_sort(out.begin(), out.end(), [&](const RRect &a, const RRect &b) { return top(a) < top(b); });
    for (size_t i = 0; i < out.size(); i++)
        for (size_t j = i; j > 0; j--) {
            if (std::fabs(top(out[j]) - top(out[j - 1])) < 10.f && left(out[j]) < left(out[j - 1]))
                std::swap(out[j - 1], out[j]);
            else
                break;
        }
    return out;
}

PpLine pp_line_box(const RRect &box, float relv, int page_w, int page_h) {
    // ocr-bench.rs:538-555 with one box a line: grown by relv * its height across.
    std::vector<std::vector<RRect>> line{{box}};
    pad_lines(line, relv, 0.f);
    float l, t, r, b;
    line[0][0].bbox(l, t, r, b);
    // ppocr.rs:42-53: the clamped box, at least 1 x 1, resized to 48 rows keeping its aspect.
    auto clampf = [](float v, int hi) { return int(std::min(std::max(v, 0.f), float(hi))); };
    PpLine p;
    p.left = clampf(l, page_w), p.top = clampf(t, page_h);
    const int rr = clampf(r, page_w), bb = clampf(b, page_h);
    p.cw = std::max(rr - p.left, 1), p.ch = std::max(bb - p.top, 1);
    p.out_w = std::min(std::max(int(std::ceil(float(PP_LINE_H) * float(p.cw) / float(p.ch))), 8), 3200);
    return p;
}

BatchPlan plan_pp_batches(const std::vector<int> &out_w, int per_batch) {
    // ocr-bench.rs:330-345 (PPGROUP = 0): sorted by width, cut into batches of per_batch, each as
    // wide as its widest line rounded up to a multiple of 8.
    std::vector<int> order(out_w.size());
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return out_w[size_t(a)] < out_w[size_t(b)]; });
    BatchPlan plan;
    for (size_t c = 0; c < order.size(); c += size_t(per_batch)) {
        std::vector<int> members(order.begin() + long(c), order.begin() + long(std::min(order.size(), c + size_t(per_batch))));
        int wmax = 8;
        for (int i : members) wmax = std::max(wmax, out_w[size_t(i)]);
        plan.lines.push_back(std::move(members));
        plan.width.push_back((wmax + 7) / 8 * 8);
    }
    return plan;
}

std::string pp_ctc_decode(const uint32_t *best, int steps) {
    // ppocr.rs:23-33: repeats merged, blanks dropped; class k >= 1 is dictionary entry k - 1,
    // here the synthetic dictionary (code point U+4E00 + k - 1), the last class a space.
    std::string s;
    uint32_t prev = 0;
    for (int t = 0; t < steps; t++) {
        const uint32_t c = best[t];
        if (c != 0 && c != prev) {
            if (c + 1 == PP_CLASSES) {
                s.push_back(' ');
            } else {
                const uint32_t cp = 0x4E00u + c - 1;  // 3-byte UTF-8
                s.push_back(char(0xE0 | (cp >> 12)));
                s.push_back(char(0x80 | ((cp >> 6) & 0x3F)));
                s.push_back(char(0x80 | (cp & 0x3F)));
            }
        }
        prev = c;
    }
    return s;
}

std::vector<std::vector<RRect>> find_text_lines(const std::vector<RRect> &words) {
    struct Box {
        float l, t, r, b;
        int i;
    };
    std::vector<Box> boxes;
    for (size_t i = 0; i < words.size(); i++) {
        Box b;
        words[i].bbox(b.l, b.t, b.r, b.b);
        b.i = int(i);
        boxes.push_back(b);
    }
    std::stable_sort(boxes.begin(), boxes.end(), [](const Box &a, const Box &b) { return a.l < b.l; });
    // A word joins the line whose last word ends nearest before it, when the two overlap
    // vertically by at least half the smaller height and the gap is at most twice the taller.
    std::vector<std::vector<int>> lines;
    std::vector<Box> last;
    for (const Box &b : boxes) {
        int best = -1;
        float best_gap = INFINITY;
        const float hb = b.b - b.t;
        for (size_t k = 0; k < lines.size(); k++) {
            const Box &a = last[k];
            const float ha = a.b - a.t;
            const float overlap = std::min(a.b, b.b) - std::max(a.t, b.t);
            const float gap = b.l - a.r;
            if (overlap < 0.5f * std::min(ha, hb) || gap > 2.f * std::max(ha, hb) || gap < -0.5f * std::min(ha, hb))
                continue;
            if (gap < best_gap) best_gap = gap, best = int(k);
        }
        if (best < 0) {
            lines.push_back({b.i});
            last.push_back(b);
        } else {
            lines[size_t(best)].push_back(b.i);
            last[size_t(best)] = b;
        }
    }
    // Reading order: lines by the top of their first word, then left.
    std::vector<size_t> order(lines.size());
    std::iota(order.begin(), order.end(), 0);
    auto top_left = [&](size_t k) {
        float l, t, r, b;
        words[size_t(lines[k][0])].bbox(l, t, r, b);
        return std::make_pair(t, l);
    };
    std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) { return top_left(a) < top_left(b); });
    std::vector<std::vector<RRect>> out;
    for (size_t k : order) {
        std::vector<RRect> line;
        for (int i : lines[k]) line.push_back(words[size_t(i)]);
        out.push_back(std::move(line));
    }
    return out;
}

void pad_lines(std::vector<std::vector<RRect>> &lines, float relv, float relend) {
    if (relv <= 0 && relend <= 0) return;
    for (auto &line : lines) {
        std::vector<float> hs;
        for (const RRect &r : line) hs.push_back(r.upright() ? r.h : r.w);
        std::sort(hs.begin(), hs.end());
        const float h = hs.empty() ? 0.f : hs[hs.size() / 2];
        const size_t n = line.size();
        for (size_t i = 0; i < n; i++) {
            RRect &r = line[i];
            const float along = (i == 0 || i + 1 == n) ? relend * h : 0.f, across = relv * h;
            if (r.upright()) r.resize(r.w + 2 * along, r.h + 2 * across);
            else r.resize(r.w + 2 * across, r.h + 2 * along);
        }
    }
}

LineGeom line_geometry(const std::vector<RRect> &words) {
    // Polygon: top edges left to right, then bottom edges right to left, floored.
    std::vector<Pt> poly;
    for (const RRect &r : words) {
        float xs[4], ys[4];
        r.corners(xs, ys);
        poly.push_back({std::floor(xs[0]), std::floor(ys[0])});
        poly.push_back({std::floor(xs[1]), std::floor(ys[1])});
    }
    for (size_t i = words.size(); i-- > 0;) {
        float xs[4], ys[4];
        words[i].corners(xs, ys);
        poly.push_back({std::floor(xs[2]), std::floor(ys[2])});
        poly.push_back({std::floor(xs[3]), std::floor(ys[3])});
    }
    LineGeom g;
    if (poly.empty()) return g;
    float l = INFINITY, t = INFINITY, r = -INFINITY, b = -INFINITY;
    for (const Pt &p : poly) l = std::min(l, p.x), r = std::max(r, p.x), t = std::min(t, p.y), b = std::max(b, p.y);
    g.left = int(l), g.top = int(t);
    g.bw = std::max(1, int(r - l)), g.bh = std::max(1, int(b - t));
    const float aspect = float(g.bw) / float(g.bh);
    g.out_w = int(std::min(std::max(float(LINE_H) * aspect, float(LINE_MIN_W)), float(LINE_MAX_W)));
    // Row spans: crossings of the line y + 0.5 with the polygon's edges (even-odd rule).
    g.row_off.assign(size_t(g.bh) + 1, 0);
    std::vector<float> xs;
    for (int cy = 0; cy < g.bh; cy++) {
        g.row_off[size_t(cy)] = int(g.spans.size());
        const float Y = float(g.top + cy) + 0.5f;
        xs.clear();
        for (size_t i = 0; i < poly.size(); i++) {
            const Pt &a = poly[i], &c = poly[(i + 1) % poly.size()];
            if ((a.y <= Y && c.y > Y) || (c.y <= Y && a.y > Y))
                xs.push_back(a.x + (Y - a.y) * (c.x - a.x) / (c.y - a.y));
        }
        std::sort(xs.begin(), xs.end());
        for (size_t k = 0; k + 1 < xs.size(); k += 2) {
            // pixels whose centre x + 0.5 lies in [xs[k], xs[k+1])
            const int x0 = std::max(0, int(std::ceil(xs[k] - 0.5f)) - g.left);
            const int x1 = std::min(g.bw, int(std::ceil(xs[k + 1] - 0.5f)) - g.left);
            if (x1 > x0) {
                g.spans.push_back(x0);
                g.spans.push_back(x1);
            }
        }
    }
    g.row_off[size_t(g.bh)] = int(g.spans.size());
    return g;
}

BatchPlan plan_batches(const std::vector<int> &out_w, int round_to, int per_batch) {
    std::vector<std::pair<int, int>> keyed;  // (rounded width, line)
    for (size_t i = 0; i < out_w.size(); i++)
        keyed.push_back({(out_w[i] + round_to - 1) / round_to * round_to, int(i)});
    std::stable_sort(keyed.begin(), keyed.end(),
                     [](const std::pair<int, int> &a, const std::pair<int, int> &b) { return a.first < b.first; });
    BatchPlan plan;
    size_t i = 0;
    while (i < keyed.size()) {
        size_t j = i;
        while (j < keyed.size() && keyed[j].first == keyed[i].first) j++;
        for (size_t c = i; c < j; c += size_t(per_batch)) {
            std::vector<int> members;
            for (size_t k = c; k < std::min(j, c + size_t(per_batch)); k++) members.push_back(keyed[k].second);
            plan.lines.push_back(std::move(members));
            plan.width.push_back(keyed[i].first);
        }
        i = j;
    }
    return plan;
}

std::string ctc_decode(const uint32_t *best, int steps, int stride, int width) {
    std::string s;
    uint32_t prev = 0;
    const int nalpha = int(std::strlen(OCRS_ALPHABET));
    for (int t = 0; t < steps; t++) {
        const uint32_t b = best[size_t(t) * stride];
        if (b != 0 && b != prev && t * 4 < width && int(b) <= nalpha) s.push_back(OCRS_ALPHABET[b - 1]);
        prev = b;
    }
    return s;
}

}  // namespace ocr
