/*
 * ORACLE - test infrastructure only. The word boxes of a binary mask as the reference finds them
 * (src/bin/ocr-bench.rs:40-60, ocrs' find_connected_component_rects; DB boxes, src/ppdet.rs:87-101):
 *   find_contours(mask, RetrievalMode::External) -> simplify_polygon(points, 2) -> min_area_rect
 *   -> grown by 3 px -> kept when the area is at least 100.
 * Those three routines live in rten-imageproc 0.26.0 (Cargo.lock), which is not vendored; this
 * file restates the published algorithms they implement:
 *   - S. Suzuki and K. Abe, "Topological structural analysis of digitized binary images by border
 *     following", CVGIP 30 (1985), Appendix I (Algorithm 1: every border with its type and
 *     parent; 8-connected 1-pixels, 4-connected 0-pixels). The mask is padded with one row and
 *     column of zeros on every side, so the frame is the outermost hole border. External
 *     retrieval keeps the outer borders whose parent is the frame. A border's points are the
 *     pixels (i3, j3) of step (3.4) in the order visited, starting at its start pixel.
 *   - Ramer-Douglas-Peucker on the closed polygon (the polyline with the first point appended,
 *     the appended point dropped again): the farthest inner point from the segment between the
 *     ends (distance to the segment, a zero-length segment measuring from its point; the last of
 *     equally far points) splits the run when it is farther than epsilon.
 *   - Minimum-area rectangle: the best of the rectangles with a side on an edge of the convex
 *     hull (Freeman and Shapira 1975), edges in hull order, the first of equal areas; the hull by
 *     Jarvis's march (gift wrapping) from the smallest (x, y) point, counter-clockwise in the sense
 *     cross > 0, collinear points dropped. Then turned by a multiple of 90 degrees so its up axis
 *     points most towards -y (the last of equally good turns: up, +90, +180, +270).
 * Nothing in the product links or calls this file. Pinned by tests/test_oracle_layout.py (border
 * sets and external selection against scipy labelling, hand-built chains and polylines, an angle
 * sweep for the rectangles).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Directions: 0 E, 1 NE, 2 N, 3 NW, 4 W, 5 SW, 6 S, 7 SE (y down); increasing index turns
 * counter-clockwise on the page. */
static const int CDX[8] = {1, 1, 0, -1, -1, -1, 0, 1};
static const int CDY[8] = {0, -1, -1, -1, 0, 1, 1, 1};

typedef struct {
    int n;          /* borders found (the frame is not listed) */
    int *type;      /* 1 outer, 2 hole */
    int *parent;    /* index of the parent border in this list, -1 for the frame */
    int *off;       /* n + 1 offsets into xy (in points) */
    int *xy;        /* x, y pairs */
    int cap_b, cap_p, npts;
} orc_contours;

static void push_pt(orc_contours *c, int x, int y) {
    if (c->npts == c->cap_p) {
        c->cap_p = c->cap_p ? 2 * c->cap_p : 4096;
        c->xy = (int *)realloc(c->xy, sizeof(int) * 2 * (size_t)c->cap_p);
    }
    c->xy[2 * c->npts] = x;
    c->xy[2 * c->npts + 1] = y;
    c->npts++;
}

void orc_contours_free(orc_contours *c) {
    if (!c) return;
    free(c->type);
    free(c->parent);
    free(c->off);
    free(c->xy);
    free(c);
}

/* Every border of the mask (h rows of ceil(w / 32) words, bit x % 32 of word x / 32). */
orc_contours *orc_find_contours(const uint32_t *bits, int w, int h) {
    const int W = w + 2, H = h + 2, words = (w + 31) / 32;
    int *f = (int *)calloc((size_t)W * H, sizeof(int));
    for (int y = 0; y < h; y++)
        for (int x = 0; x < w; x++) f[(size_t)(y + 1) * W + x + 1] = (bits[(size_t)y * words + x / 32] >> (x % 32)) & 1u;
    orc_contours *c = (orc_contours *)calloc(1, sizeof(orc_contours));
    /* Border numbers: NBD 1 is the frame (a hole border); border NBD >= 2 is list entry NBD - 2. */
    int nbd = 1;
    int cap = 1024;
    int *btype = (int *)malloc(sizeof(int) * cap), *bparent = (int *)malloc(sizeof(int) * cap);
    btype[1] = 2;
    bparent[1] = 0;
    c->off = (int *)malloc(sizeof(int));
    c->off[0] = 0;
    for (int i = 1; i <= h; i++) {
        int lnbd = 1;
        for (int j = 1; j <= w; j++) {
            const int v = f[(size_t)i * W + j];
            int start = 0, type = 0, i2 = 0, j2 = 0;
            if (v == 1 && f[(size_t)i * W + j - 1] == 0) {
                start = 1, type = 1, i2 = i, j2 = j - 1; /* (1)(a) outer border */
            } else if (v >= 1 && f[(size_t)i * W + j + 1] == 0) {
                start = 1, type = 2, i2 = i, j2 = j + 1; /* (1)(b) hole border */
                if (v > 1) lnbd = v;
            }
            if (start) {
                nbd++;
                if (nbd + 1 >= cap) {
                    cap *= 2;
                    btype = (int *)realloc(btype, sizeof(int) * cap);
                    bparent = (int *)realloc(bparent, sizeof(int) * cap);
                }
                /* (2) the parent from the border met last (Table 1 of the paper). */
                btype[nbd] = type;
                bparent[nbd] = (type == btype[lnbd]) ? bparent[lnbd] : lnbd;
                /* (3) follow the border. */
                int d0 = (j2 > j) ? 0 : 4, d1 = -1;
                for (int k = 0; k < 8; k++) { /* (3.1) clockwise from (i2, j2) */
                    const int d = (d0 - k) & 7;
                    if (f[(size_t)(i + CDY[d]) * W + j + CDX[d]] != 0) {
                        d1 = d;
                        break;
                    }
                }
                if (d1 < 0) {
                    f[(size_t)i * W + j] = -nbd;
                    push_pt(c, j - 1, i - 1);
                } else {
                    const int i1 = i + CDY[d1], j1 = j + CDX[d1];
                    int i3 = i, j3 = j, dprev = d1; /* (3.2) (i2, j2) = (i1, j1) */
                    for (;;) {
                        int d4 = -1, east_zero = 0;
                        for (int k = 1; k <= 8; k++) { /* (3.3) counter-clockwise after (i2, j2) */
                            const int d = (dprev + k) & 7;
                            if (f[(size_t)(i3 + CDY[d]) * W + j3 + CDX[d]] != 0) {
                                d4 = d;
                                break;
                            }
                            if (d == 0) east_zero = 1;
                        }
                        const int i4 = i3 + CDY[d4], j4 = j3 + CDX[d4];
                        int *p3 = &f[(size_t)i3 * W + j3]; /* (3.4) */
                        if (east_zero) *p3 = -nbd;
                        else if (*p3 == 1) *p3 = nbd;
                        push_pt(c, j3 - 1, i3 - 1);
                        if (i4 == i && j4 == j && i3 == i1 && j3 == j1) break; /* (3.5) */
                        dprev = (d4 + 4) & 7;
                        i3 = i4, j3 = j4;
                    }
                }
                c->n++;
                c->off = (int *)realloc(c->off, sizeof(int) * (size_t)(c->n + 1));
                c->off[c->n] = c->npts;
            }
            { /* (4): LNBD is the number of the last border pixel passed (0-pixels leave it) */
                const int u = f[(size_t)i * W + j];
                if (u != 0 && u != 1) lnbd = u < 0 ? -u : u;
            }
        }
    }
    c->type = (int *)malloc(sizeof(int) * (size_t)(c->n ? c->n : 1));
    c->parent = (int *)malloc(sizeof(int) * (size_t)(c->n ? c->n : 1));
    for (int k = 0; k < c->n; k++) {
        c->type[k] = btype[k + 2];
        c->parent[k] = bparent[k + 2] >= 2 ? bparent[k + 2] - 2 : -1;
    }
    free(btype);
    free(bparent);
    free(f);
    return c;
}

int orc_contours_count(const orc_contours *c) { return c->n; }
int orc_contours_points(const orc_contours *c) { return c->npts; }
/* Copies type, parent and offsets (n, n, n + 1 ints) and the points (2 * npts ints). */
void orc_contours_get(const orc_contours *c, int *type, int *parent, int *off, int *xy) {
    memcpy(type, c->type, sizeof(int) * (size_t)c->n);
    memcpy(parent, c->parent, sizeof(int) * (size_t)c->n);
    memcpy(off, c->off, sizeof(int) * (size_t)(c->n + 1));
    memcpy(xy, c->xy, sizeof(int) * 2 * (size_t)c->npts);
}

/* ---- Ramer-Douglas-Peucker ------------------------------------------------------------- */

static float seg_dist(float ax, float ay, float bx, float by, float px, float py) {
    if (ax == bx && ay == by) {
        const float dx = px - ax, dy = py - ay;
        return sqrtf(dx * dx + dy * dy);
    }
    const float abx = bx - ax, aby = by - ay, acx = px - ax, acy = py - ay;
    const float t = (acx * abx + acy * aby) / (abx * abx + aby * aby);
    float qx, qy;
    if (t <= 0.f) {
        qx = ax, qy = ay;
    } else if (t >= 1.f) {
        qx = bx, qy = by;
    } else {
        qx = ax + abx * t, qy = ay + aby * t;
    }
    const float dx = px - qx, dy = py - qy;
    return sqrtf(dx * dx + dy * dy);
}

static void rdp(const float *p, int s, int e, float eps, unsigned char *keep) {
    keep[s] = keep[e] = 1;
    if (e - s < 2) return;
    int best = s;
    float dmax = 0.f;
    for (int k = s + 1; k < e; k++) {
        const float d = seg_dist(p[2 * s], p[2 * s + 1], p[2 * e], p[2 * e + 1], p[2 * k], p[2 * k + 1]);
        if (d >= dmax) dmax = d, best = k;
    }
    if (dmax > eps) {
        rdp(p, s, best, eps, keep);
        rdp(p, best, e, eps, keep);
    }
}

/* simplify_polygon: n points (x, y) -> the kept ones into out (at most n); returns their count. */
int orc_simplify_polygon(const float *pts, int n, float eps, float *out) {
    if (n <= 0) return 0;
    float *p = (float *)malloc(sizeof(float) * 2 * (size_t)(n + 1));
    memcpy(p, pts, sizeof(float) * 2 * (size_t)n);
    p[2 * n] = pts[0], p[2 * n + 1] = pts[1];
    unsigned char *keep = (unsigned char *)calloc((size_t)n + 1, 1);
    rdp(p, 0, n, eps, keep);
    int m = 0;
    for (int k = 0; k < n; k++) /* the appended copy of the first point is dropped */
        if (keep[k]) out[2 * m] = p[2 * k], out[2 * m + 1] = p[2 * k + 1], m++;
    free(p);
    free(keep);
    return m;
}

/* ---- Convex hull (Jarvis's march) and minimum-area rectangle ---------------------------- */

/* In double: exact for integer coordinates of any page size. */
static double crossf(float ox, float oy, float ax, float ay, float bx, float by) {
    return ((double)ax - ox) * ((double)by - oy) - ((double)ay - oy) * ((double)bx - ox);
}

/* Hull vertices of n points into hull (2 * n floats); returns their count. */
int orc_convex_hull(const float *pts, int n, float *hull) {
    if (n <= 0) return 0;
    int start = 0;
    for (int k = 1; k < n; k++)
        if (pts[2 * k] < pts[2 * start] || (pts[2 * k] == pts[2 * start] && pts[2 * k + 1] < pts[2 * start + 1]))
            start = k;
    int m = 0, cur = start;
    for (;;) {
        hull[2 * m] = pts[2 * cur], hull[2 * m + 1] = pts[2 * cur + 1];
        m++;
        /* The next vertex: every other point is left of cur -> next (cross >= 0), the farthest
         * of collinear candidates. */
        int next = -1;
        for (int k = 0; k < n; k++) {
            if (pts[2 * k] == pts[2 * cur] && pts[2 * k + 1] == pts[2 * cur + 1]) continue;
            if (next < 0) {
                next = k;
                continue;
            }
            const double cr = crossf(pts[2 * cur], pts[2 * cur + 1], pts[2 * next], pts[2 * next + 1], pts[2 * k],
                                    pts[2 * k + 1]);
            if (cr < 0.0) {
                next = k;
            } else if (cr == 0.0) {
                const float dn = (pts[2 * next] - pts[2 * cur]) * (pts[2 * next] - pts[2 * cur]) +
                                 (pts[2 * next + 1] - pts[2 * cur + 1]) * (pts[2 * next + 1] - pts[2 * cur + 1]);
                const float dk = (pts[2 * k] - pts[2 * cur]) * (pts[2 * k] - pts[2 * cur]) +
                                 (pts[2 * k + 1] - pts[2 * cur + 1]) * (pts[2 * k + 1] - pts[2 * cur + 1]);
                if (dk > dn) next = k;
            }
        }
        if (next < 0) break; /* a single distinct point */
        if (pts[2 * next] == pts[2 * start] && pts[2 * next + 1] == pts[2 * start + 1]) break;
        cur = next;
        if (m >= n) break;
    }
    return m;
}

/* min_area_rect of n points -> rect {cx, cy, ux, uy, w, h}; returns 0 when there is none (no
 * points, or all the same point). */
int orc_min_area_rect(const float *pts, int n, float *rect) {
    if (n <= 0) return 0;
    float *hull = (float *)malloc(sizeof(float) * 2 * (size_t)n);
    const int m = orc_convex_hull(pts, n, hull);
    int found = 0;
    float best = INFINITY;
    for (int i = 0; i < m && m >= 2; i++) {
        const float ax = hull[2 * i], ay = hull[2 * i + 1];
        const float bx = hull[2 * ((i + 1) % m)], by = hull[2 * ((i + 1) % m) + 1];
        float ex = bx - ax, ey = by - ay;
        const float len = sqrtf(ex * ex + ey * ey);
        if (len == 0.f) continue;
        ex /= len, ey /= len;
        const float nx = -ey, ny = ex; /* into the hull (counter-clockwise in the cross > 0 sense) */
        float pmin = INFINITY, pmax = -INFINITY, qmax = -INFINITY;
        for (int k = 0; k < m; k++) {
            const float dx = hull[2 * k] - ax, dy = hull[2 * k + 1] - ay;
            const float par = dx * ex + dy * ey, perp = dx * nx + dy * ny;
            if (par < pmin) pmin = par;
            if (par > pmax) pmax = par;
            if (perp > qmax) qmax = perp;
        }
        const float width = pmax - pmin, height = qmax, area = width * height;
        if (area < best) {
            best = area;
            found = 1;
            const float mid = (pmin + pmax) / 2.f, half = height / 2.f;
            rect[0] = ax + ex * mid + nx * half;
            rect[1] = ay + ey * mid + ny * half;
            rect[2] = nx, rect[3] = ny, rect[4] = width, rect[5] = height;
        }
    }
    free(hull);
    if (!found) return 0;
    /* Turned so the up axis points most towards -y: candidates up, +90 (uy, -ux), +180, +270. */
    const float ux = rect[2], uy = rect[3], w = rect[4], h = rect[5];
    const float cand[4][2] = {{ux, uy}, {uy, -ux}, {-ux, -uy}, {-uy, ux}};
    int k = 0;
    for (int c = 1; c < 4; c++)
        if (-cand[c][1] >= -cand[k][1]) k = c;
    rect[2] = cand[k][0], rect[3] = cand[k][1];
    rect[4] = (k & 1) ? h : w;
    rect[5] = (k & 1) ? w : h;
    return 1;
}

/* word_rects: external contours, simplified by eps, minimum-area rectangles grown by expand on
 * every side, kept when their area is at least min_area; at most cap rects into out (6 floats
 * each). Returns the number found. */
int orc_word_rects(const uint32_t *bits, int w, int h, float eps, float expand, float min_area, float *out, int cap) {
    orc_contours *c = orc_find_contours(bits, w, h);
    int found = 0;
    for (int b = 0; b < c->n; b++) {
        if (c->type[b] != 1 || c->parent[b] != -1) continue;
        const int n = c->off[b + 1] - c->off[b];
        float *pts = (float *)malloc(sizeof(float) * 2 * (size_t)n), *simp = (float *)malloc(sizeof(float) * 2 * (size_t)n);
        for (int k = 0; k < n; k++) pts[2 * k] = (float)c->xy[2 * (c->off[b] + k)], pts[2 * k + 1] = (float)c->xy[2 * (c->off[b] + k) + 1];
        const int m = orc_simplify_polygon(pts, n, eps, simp);
        float r[6];
        if (orc_min_area_rect(simp, m, r)) {
            r[4] += 2.f * expand, r[5] += 2.f * expand;
            if (r[4] * r[5] >= min_area) {
                if (found < cap) memcpy(out + 6 * found, r, sizeof(r));
                found++;
            }
        }
        free(pts);
        free(simp);
    }
    orc_contours_free(c);
    return found;
}
