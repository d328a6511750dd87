// Word boxes from GPU component records (word_rects_from_rows, wgpu-ocr_amd/csrc/geometry.cpp) fed
// records that a faulty labelling could hand over: a component's row slots past the slot count,
// rows past the page, a row whose leftmost pixel lies right of its rightmost, a pixel past the
// width, a first pixel that does not start a run (a run whose parent is not its component's
// final root), and one component split over two records. Each is refused with an error or gives
// rectangles, never a read outside the buffers. Built and run by tests/test_geometry_records.py
// under AddressSanitizer + UndefinedBehaviorSanitizer.
#include "common.h"
#include "geometry.h"

#include <array>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace ocr {
[[noreturn]] void fail(const std::string &msg) { throw Error(msg); }
}  // namespace ocr

using namespace ocr;

namespace {

int failures = 0;
#define CHECK(c, what)                                                          \
    do {                                                                        \
        if (!(c)) {                                                             \
            failures++;                                                         \
            std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, what); \
        }                                                                       \
    } while (0)

struct Mask {
    int w, h, words;
    std::vector<uint32_t> bits;
    Mask(int w_, int h_) : w(w_), h(h_), words((w_ + 31) / 32), bits(size_t(words) * h_, 0u) {}
    void set(int x, int y) { bits[size_t(y) * words + x / 32] |= 1u << (x % 32); }
    void box(int x0, int y0, int x1, int y1) {
        for (int y = y0; y <= y1; y++)
            for (int x = x0; x <= x1; x++) set(x, y);
    }
};

// The records of a correct labelling of m's rectangles (given as boxes, one component each, in
// raster order): {first run, top, rows, first slot} and per row the extremes.
struct Records {
    std::vector<int32_t> comps;
    std::vector<uint32_t> xmin, xmax;
};

Records records_of(const std::vector<std::array<int, 4>> &boxes) {
    Records r;
    int run = 0;
    for (const auto &b : boxes) {
        const int rows = b[3] - b[1] + 1;
        r.comps.insert(r.comps.end(), {run, b[1], rows, int(r.xmin.size())});
        for (int y = 0; y < rows; y++) r.xmin.push_back(uint32_t(b[0])), r.xmax.push_back(uint32_t(b[2]));
        run += rows;
    }
    return r;
}

bool refused(const Mask &m, const Records &r, int nslots = -1) {
    try {
        word_rects_from_rows(m.bits.data(), m.w, m.h, r.comps.data(), int(r.comps.size() / 4), r.xmin.data(),
                             r.xmax.data(), nslots < 0 ? int(r.xmin.size()) : nslots);
    } catch (const Error &) {
        return true;
    }
    return false;
}

}  // namespace

int main() {
    Mask m(100, 60);
    const std::vector<std::array<int, 4>> boxes = {{5, 3, 40, 12}, {50, 20, 95, 30}, {10, 40, 30, 58}};
    for (const auto &b : boxes) m.box(b[0], b[1], b[2], b[3]);
    Records good = records_of(boxes);
    {
        auto want = word_rects(m.bits.data(), m.w, m.h);
        auto got = word_rects_from_rows(m.bits.data(), m.w, m.h, good.comps.data(), 3, good.xmin.data(),
                                        good.xmax.data(), int(good.xmin.size()));
        CHECK(got.size() == want.size() && got.size() == 3, "valid records give the host's rectangles");
        for (size_t i = 0; i < got.size() && i < want.size(); i++)
            CHECK(std::memcmp(&got[i], &want[i], sizeof(RRect)) == 0, "same rectangle");
    }
    {  // slots past the slot count (a block handed out past the capacity)
        Records r = good;
        CHECK(refused(m, r, int(r.xmin.size()) - 1), "slots past nslots");
        r.comps[3 + 4] = int(r.xmin.size()) - 2;
        CHECK(refused(m, r), "a block running past the last slot");
        r = good;
        r.comps[3] = -1;
        CHECK(refused(m, r), "negative first slot");
    }
    {  // rows past the page, and no rows
        Records r = good;
        r.comps[1 + 8] = 50, r.comps[2 + 8] = 11;
        r.xmin.resize(r.xmin.size() + 2, 10), r.xmax.resize(r.xmax.size() + 2, 30);
        CHECK(refused(m, r), "rows past the page");
        r = good;
        r.comps[2] = 0;
        CHECK(refused(m, r), "a component with no rows");
    }
    {  // a row slot never written (leftmost > rightmost), and a pixel past the width
        Records r = good;
        r.xmin[2] = 0xffffu, r.xmax[2] = 0u;
        CHECK(refused(m, r), "an empty row slot");
        r = good;
        r.xmax[r.comps[3 + 4]] = 100;
        CHECK(refused(m, r), "a pixel past the width");
    }
    {  // a first pixel that does not start a run: clear, or with its west neighbour set
        Records r = good;
        r.xmin[0] = 6;
        CHECK(refused(m, r), "first pixel inside a run");
        r = good;
        r.comps[1] = 2, r.comps[2] = 11;  // one row too high: row 2 is clear
        r.xmin.insert(r.xmin.begin(), 5), r.xmax.insert(r.xmax.begin(), 40);
        for (size_t k = 1; k < 3; k++) r.comps[4 * k + 3] += 1;
        CHECK(refused(m, r), "first pixel clear");
    }
    {  // one component split over two records (a run left under a non-final root): both
        // records are well formed, the border of each is the whole component's
        Records r = good;
        r.comps = {0, 3, 5, 0, 5, 8, 5, 5, 10, 20, 11, 10, 21, 40, 19, 21};
        auto got = word_rects_from_rows(m.bits.data(), m.w, m.h, r.comps.data(), 4, r.xmin.data(), r.xmax.data(),
                                        int(r.xmin.size()));
        CHECK(got.size() >= 3, "split records still give rectangles");
    }
    if (failures) {
        std::printf("%d checks failed\n", failures);
        return 1;
    }
    std::printf("all checks passed\n");
    return 0;
}
