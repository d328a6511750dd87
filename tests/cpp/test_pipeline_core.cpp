// The page pipeline's schedule (wgpu-ocr_amd/csrc/pipeline_core.h) with hooks that record the
// order of the steps and fail on purpose: a failing step fails exactly the pages it covers and
// every other page finishes (the reference reports errors per page, src/bin/ocr-bench.rs:277-281,
// 303-307), the ordering rules hold, and nothing deadlocks with few workers. Built and run by
// tests/test_pipeline_core.py under AddressSanitizer + UndefinedBehaviorSanitizer and under
// ThreadSanitizer.
#include <algorithm>
#include "pipeline_core.h"
#include "wait.h"

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <deque>
#include <random>
#include <stdexcept>
#include <string>

using namespace ocr;

namespace {

int failures = 0;
#define CHECK(c, ...)                                     \
    do {                                                  \
        if (!(c)) {                                       \
            failures++;                                   \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);            \
            std::fprintf(stderr, "\n");                   \
        }                                                 \
    } while (0)

// A small FIFO thread pool (the pipeline's Workers without HIP).
class Pool {
  public:
    explicit Pool(int n) {
        for (int i = 0; i < n; i++) t_.emplace_back([this] { loop(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : t_) t.join();
    }
    void submit(std::function<void()> f) {
        {
            std::lock_guard<std::mutex> lk(mu_);
            q_.push_back(std::move(f));
        }
        cv_.notify_one();
    }

  private:
    void loop() {
        for (;;) {
            std::function<void()> f;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [this] { return stop_ || !q_.empty(); });
                if (q_.empty()) return;
                f = std::move(q_.front());
                q_.pop_front();
            }
            f();
        }
    }
    std::vector<std::thread> t_;
    std::deque<std::function<void()>> q_;
    std::mutex mu_;
    std::condition_variable cv_;
    bool stop_ = false;
};

struct Faults {
    int stage = -1, detect = -1, detect_wait = -1, layout = -1, recognize = -1, decode = -1;
    int detect_stall = -1;  // this group's wait never sees its event: the bounded wait gives up
};

// Records what ran and checks the ordering rules as it goes.
struct Hooks final : PipelineHooks {
    const PipelinePlan &P;
    Faults f;
    std::mt19937 rng;
    std::mutex mu;
    std::vector<int> staged_at, detected_at, waited_at, laid_at, rec_at, dec_at;
    std::vector<std::vector<char>> rec_ok;
    int clock = 0;
    bool jitter, lookahead = false, interleave = false;
    int polled_groups = 0;  // groups a recognition pass queued between its stages
    // Copies in flight: landed(g) holds land_us after stage(g) returned (at once when negative),
    // never for group never_lands.
    int land_us = -1, never_lands = -1;
    int early_groups = 0;  // groups detected before their copy landed, needed by the next pass
    int late_queued = 0;   // groups queued on the 100 ms fallback
    int slow_layout = -1;  // this page's layout takes 150 ms
    std::vector<std::chrono::steady_clock::time_point> staged_time;
    Hooks(const PipelinePlan &plan, Faults faults, unsigned seed, bool jit)
        : P(plan), f(faults), rng(seed), jitter(jit) {
        staged_time.resize(size_t(P.groups()));
        staged_at.assign(size_t(P.groups()), -1);
        detected_at = waited_at = staged_at;
        laid_at.assign(size_t(P.npages), -1);
        rec_at.assign(size_t(P.passes()), -1);
        dec_at = rec_at;
        rec_ok.resize(size_t(P.passes()));
    }
    void nap() {
        if (!jitter) return;
        int us;
        {
            std::lock_guard<std::mutex> lk(mu);
            us = int(rng() % 300);
        }
        std::this_thread::sleep_for(std::chrono::microseconds(us));
    }
    int tick() {
        std::lock_guard<std::mutex> lk(mu);
        return clock++;
    }
    void stage(int g) override {
        nap();
        if (g == f.stage) throw std::runtime_error("stage fault");
        staged_time[size_t(g)] = std::chrono::steady_clock::now();
        staged_at[size_t(g)] = tick();
    }
    bool landed(int g) override {
        if (g == never_lands) return false;
        return land_us < 0 ||
               std::chrono::steady_clock::now() - staged_time[size_t(g)] >= std::chrono::microseconds(land_us);
    }
    void detect(int g) override {
        CHECK(staged_at[size_t(g)] >= 0, "detect(%d) before its stage", g);
        // Before its copy lands only when the next pass to be recognised needs the group, or
        // (a copy that never lands) 100 ms after it was staged.
        int r = 0;
        while (r < P.passes() && rec_at[size_t(r)] >= 0) r++;
        const int need = r + 1 < P.passes() ? P.group_of[size_t(P.pass_p0[size_t(r) + 1])] : P.groups();
        if (!landed(g) && g >= need) {
            const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() -
                                                                        staged_time[size_t(g)]).count();
            CHECK(g == never_lands && ms >= 100.0, "detect(%d) %.1f ms after its stage, before its copy landed", g, ms);
            late_queued++;
        } else if (!landed(g)) {
            early_groups++;
        }
        nap();
        if (g == f.detect) throw std::runtime_error("detect fault");
        detected_at[size_t(g)] = tick();
    }
    void detect_wait(int g) override {
        CHECK(detected_at[size_t(g)] >= 0, "detect_wait(%d) before detect", g);
        nap();
        if (g == f.detect_wait) throw std::runtime_error("detect_wait fault");
        if (g == f.detect_stall)
            wait_until([] { return false; }, [&] { return "detection group " + std::to_string(g) + " (stall fault)"; },
                       false, 20.0);
        waited_at[size_t(g)] = tick();
    }
    void layout(int p) override {
        const int g = P.group_of[size_t(p)];
        CHECK(waited_at[size_t(g)] >= 0, "layout(%d) before its detection finished", p);
        {
            std::lock_guard<std::mutex> lk(mu);
            for (int q = 0; q < P.pass_p0[size_t(P.pass_of[size_t(p)])]; q++)
                CHECK(laid_at[size_t(q)] >= 0 || q == f.layout || P.group_of[size_t(q)] == f.stage ||
                          P.group_of[size_t(q)] == f.detect || P.group_of[size_t(q)] == f.detect_wait ||
                          P.group_of[size_t(q)] == f.detect_stall,
                      "layout(%d) before page %d of an earlier pass", p, q);
        }
        nap();
        if (p == slow_layout) std::this_thread::sleep_for(std::chrono::milliseconds(150));
        if (p == f.layout) throw std::runtime_error("layout fault");
        const int t = tick();
        std::lock_guard<std::mutex> lk(mu);
        laid_at[size_t(p)] = t;
    }
    void recognize(int r, const std::vector<char> &ok) override {
        const int p0 = P.pass_p0[size_t(r)], p1 = P.pass_p0[size_t(r) + 1];
        CHECK(int(ok.size()) == p1 - p0, "recognize(%d): ok has %zu entries", r, ok.size());
        for (int p = p0; p < p1; p++) {
            std::lock_guard<std::mutex> lk(mu);
            CHECK((laid_at[size_t(p)] >= 0) == (ok[size_t(p - p0)] != 0), "recognize(%d): page %d ok flag", r, p);
        }
        if (lookahead && r + 1 < P.passes())
            for (int q = P.pass_p0[size_t(r) + 1]; q < P.pass_p0[size_t(r) + 2]; q++) {
                const int g = P.group_of[size_t(q)];
                CHECK(detected_at[size_t(g)] >= 0 || g == f.stage || g == f.detect,
                      "recognize(%d) before group %d of the next pass was queued", r, g);
            }
        nap();
        if (r == f.recognize) throw std::runtime_error("recognize fault");
        if (interleave) {
            // Three stages, the groups staged meanwhile queued between them.
            CHECK(bool(poll_detections), "recognize(%d): no poll_detections", r);
            for (int k = 0; k < 3 && poll_detections; k++) {
                const int before = int(std::count_if(detected_at.begin(), detected_at.end(), [](int t) { return t >= 0; }));
                const bool any = poll_detections();
                const int after = int(std::count_if(detected_at.begin(), detected_at.end(), [](int t) { return t >= 0; }));
                if (f.detect < 0) CHECK(any == (after > before), "recognize(%d): poll result %d, %d -> %d groups", r, int(any), before, after);
                polled_groups += after - before;
                CHECK(bool(detections_pending), "recognize(%d): no detections_pending", r);
                if (!detections_pending())
                    for (int g = 0; g < P.groups(); g++)
                        CHECK(detected_at[size_t(g)] >= 0 || g == f.stage || g == f.detect,
                              "recognize(%d): nothing pending but group %d not queued", r, g);
                nap();
            }
        }
        rec_ok[size_t(r)] = ok;
        rec_at[size_t(r)] = tick();
    }
    void decode(int r, bool last) override {
        CHECK(rec_at[size_t(r)] >= 0, "decode(%d) before recognize", r);
        CHECK(last == (r == P.passes() - 1), "decode(%d): last flag", r);
        nap();
        if (r == f.decode) throw std::runtime_error("decode fault");
        dec_at[size_t(r)] = tick();
    }
};

// Which pages a fault must fail.
std::vector<char> expected_failed(const PipelinePlan &P, const Faults &f) {
    std::vector<char> bad(size_t(P.npages), 0);
    for (int p = 0; p < P.npages; p++) {
        const int g = P.group_of[size_t(p)], r = P.pass_of[size_t(p)];
        bad[size_t(p)] = g == f.stage || g == f.detect || g == f.detect_wait || g == f.detect_stall ||
                         p == f.layout || r == f.recognize || r == f.decode;
    }
    return bad;
}

int run_case(const char *name, int npages, int merge, int det_batch, int workers, Faults f, unsigned seed,
             bool jitter, bool lookahead = false, bool interleave = false, int land_us = -1,
             int never_lands = -1, int slow_layout = -1, int *fallbacks = nullptr, int *early = nullptr) {
    // The interleaved cases stand for pages from host memory, and take their plan.
    const PipelinePlan P = plan_pipeline(npages, merge, det_batch, interleave);
    Hooks H(P, f, seed, jitter);
    H.land_us = land_us, H.never_lands = never_lands, H.slow_layout = slow_layout;
    H.lookahead = lookahead;
    H.interleave = interleave;
    std::vector<std::string> err;
    {
        Pool pool(workers);
        double busy = -1;
        err = run_schedule(P, H, [&](std::function<void()> fn) { pool.submit(std::move(fn)); }, &busy, lookahead);
        CHECK(busy >= 0, "%s: busy time not reported", name);
    }
    const std::vector<char> bad = expected_failed(P, f);
    CHECK(int(err.size()) == npages, "%s: %zu page results", name, err.size());
    for (int p = 0; p < npages && p < int(err.size()); p++) {
        CHECK(bad[size_t(p)] == !err[size_t(p)].empty(), "%s: page %d error '%s', expected %s", name, p,
              err[size_t(p)].c_str(), bad[size_t(p)] ? "a failure" : "success");
        if (bad[size_t(p)] && !err[size_t(p)].empty())
            CHECK(err[size_t(p)].find("fault") != std::string::npos, "%s: page %d message '%s'", name, p,
                  err[size_t(p)].c_str());
        if (P.group_of[size_t(p)] == f.detect_stall && p < int(err.size()))
            CHECK(err[size_t(p)].find("did not finish within 20 ms") != std::string::npos &&
                      err[size_t(p)].find("detection group") != std::string::npos,
                  "%s: page %d stall message '%s'", name, p, err[size_t(p)].c_str());
    }
    // Every pass with a page that reached recognition was recognised and (unless it failed
    // there) decoded; every page without a failure was laid out.
    for (int r = 0; r < P.passes(); r++) {
        bool any_ok = false;
        for (int p = P.pass_p0[size_t(r)]; p < P.pass_p0[size_t(r) + 1]; p++) {
            const int g = P.group_of[size_t(p)];
            any_ok |= !(g == f.stage || g == f.detect || g == f.detect_wait || g == f.detect_stall || p == f.layout);
        }
        if (any_ok && r != f.recognize) CHECK(H.rec_at[size_t(r)] >= 0, "%s: pass %d not recognised", name, r);
        if (any_ok && r != f.recognize && r != f.decode) CHECK(H.dec_at[size_t(r)] >= 0, "%s: pass %d not decoded", name, r);
        if (!any_ok) CHECK(H.rec_at[size_t(r)] < 0, "%s: pass %d recognised without pages", name, r);
    }
    for (int p = 0; p < npages; p++)
        if (!bad[size_t(p)]) CHECK(H.laid_at[size_t(p)] >= 0, "%s: page %d not laid out", name, p);
    if (fallbacks) *fallbacks = H.late_queued;
    if (early) *early += H.early_groups;
    CHECK(!H.poll_detections, "%s: poll_detections left set after the run", name);
    CHECK(!H.detections_pending, "%s: detections_pending left set after the run", name);
    return H.polled_groups;
}

}  // namespace

int main() {
    // The plan itself: passes of at most `merge` pages, the first of ceil(merge / 2) when there
    // are more, groups inside passes, the first group smaller and the last pass's last group half
    // of det_batch rounded up.
    {
        const PipelinePlan P = plan_pipeline(12, 6, 6);
        CHECK(P.passes() == 3 && P.pass_p0[1] == 3 && P.pass_p0[2] == 7 && P.pass_p0[3] == 12, "plan: passes");
        CHECK(P.groups() == 5 && P.group_p0[0] == 0 && P.group_p0[1] == 2 && P.group_p0[2] == 3 &&
                  P.group_p0[3] == 7 && P.group_p0[4] == 9 && P.group_p0[5] == 12,
              "plan: groups");
        // The bench's plan (merge 6, det_batch 3): passes [0, 3), [3, 7), [7, 12); groups [0],
        // [1, 2], [3, 4], [5, 6], [7 .. 9], [10, 11].
        const PipelinePlan B = plan_pipeline(12, 6, 3);
        const int bg[] = {0, 1, 3, 5, 7, 10, 12};
        CHECK(B.groups() == 6, "plan: bench groups %d", B.groups());
        for (int g = 0; g <= 6 && g <= B.groups(); g++) CHECK(B.group_p0[size_t(g)] == bg[g], "plan: bench group %d", g);
        // Pages from host memory: the first pass's pages one group each, the rest as above.
        const PipelinePlan H = plan_pipeline(12, 6, 3, true);
        const int hg[] = {0, 1, 2, 3, 5, 7, 10, 12};
        CHECK(H.groups() == 7 && H.passes() == 3, "plan: host groups %d", H.groups());
        for (int g = 0; g <= 7 && g <= H.groups(); g++) CHECK(H.group_p0[size_t(g)] == hg[g], "plan: host group %d", g);
        // One pass: the option changes nothing (the first and last rules apply).
        const PipelinePlan H1 = plan_pipeline(6, 6, 4, true);
        CHECK(H1.groups() == 3 && H1.group_p0[1] == 1 && H1.group_p0[2] == 4, "plan: host, one pass");
        // Passes share the pages after the first evenly: 3, then 5, 5, 5, 6 for 24 pages.
        const PipelinePlan L = plan_pipeline(24, 6, 3);
        const int lp[] = {0, 3, 8, 13, 18, 24};
        CHECK(L.passes() == 5, "plan: 24 pages, %d passes", L.passes());
        for (int r = 0; r <= 5 && r <= L.passes(); r++) CHECK(L.pass_p0[size_t(r)] == lp[r], "plan: 24 pages, pass %d", r);
        // One pass (no more pages than merge): the first and the last rules both apply; two pages
        // split one and one.
        const PipelinePlan O = plan_pipeline(6, 6, 4);
        CHECK(O.passes() == 1 && O.groups() == 3 && O.group_p0[1] == 1 && O.group_p0[2] == 4, "plan: one pass");
        CHECK(plan_pipeline(2, 6, 4).groups() == 2 && plan_pipeline(1, 6, 4).groups() == 1, "plan: small runs");
        CHECK(plan_pipeline(5, 1, 4).passes() == 5, "plan: merge 1");
        for (int n = 1; n <= 40; n++)
            for (int merge = 1; merge <= 8; merge++)
                for (int db = 1; db <= 12; db++) {
                    const PipelinePlan Q = plan_pipeline(n, merge, db > 6 ? db - 6 : db, db > 6);
                    const int dbq = db > 6 ? db - 6 : db;
                    CHECK(Q.pass_p0.front() == 0 && Q.pass_p0.back() == n && Q.group_p0.front() == 0 &&
                              Q.group_p0.back() == n,
                          "plan (%d, %d, %d): ends", n, merge, db);
                    for (int r = 0; r < Q.passes(); r++) {
                        const int len = Q.pass_p0[size_t(r) + 1] - Q.pass_p0[size_t(r)];
                        CHECK(len >= 1 && len <= merge, "plan (%d, %d, %d): pass %d of %d pages", n, merge, db, r, len);
                    }
                    for (int g = 0; g < Q.groups(); g++) {
                        const int a = Q.group_p0[size_t(g)], b = Q.group_p0[size_t(g) + 1];
                        CHECK(b > a && b - a <= dbq, "plan (%d, %d, %d): group %d of %d pages", n, merge, db, g, b - a);
                        CHECK(Q.pass_of[size_t(a)] == Q.pass_of[size_t(b - 1)], "plan (%d, %d, %d): group %d straddles a pass",
                              n, merge, db, g);
                    }
                }
        CHECK(plan_pipeline(0, 2, 4).passes() == 0, "plan: no pages");
    }
    // The bounded wait itself: it returns once ready() holds, passes ready()'s own errors through,
    // and gives up past its deadline with the description of what it waited for.
    {
        int polls = 0;
        wait_until([&] { return ++polls == 5; }, [] { return std::string("five polls"); }, false, 1000.0);
        CHECK(polls == 5, "wait_until: %d polls", polls);
        bool passed = false;
        try {
            wait_until([]() -> bool { throw std::runtime_error("gpu error"); }, [] { return std::string("x"); });
        } catch (const WaitTimeout &) {
        } catch (const std::runtime_error &e) {
            passed = std::string(e.what()) == "gpu error";
        }
        CHECK(passed, "wait_until: ready()'s error not passed through");
        const auto t0 = std::chrono::steady_clock::now();
        std::string msg;
        try {
            wait_until([] { return false; }, [] { return std::string("stage 2 of recognition pass 1"); }, false, 30.0);
        } catch (const WaitTimeout &e) {
            msg = e.what();
        }
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        CHECK(msg.find("within 30 ms") != std::string::npos && msg.find("stage 2 of recognition pass 1") != std::string::npos,
              "wait_until: timeout message '%s'", msg.c_str());
        CHECK(ms >= 30.0 && ms < 5000.0, "wait_until: gave up after %.1f ms", ms);
        CHECK(wait_timeout_ms() == 25.0, "wait_timeout_ms: %.1f (OCR_WAIT_TIMEOUT_MS=25 expected)", wait_timeout_ms());
    }
    const Faults none;
    run_case("clean", 12, 6, 6, 4, none, 1, true);
    run_case("one worker", 9, 2, 3, 1, none, 2, true);
    run_case("many pages few workers", 50, 4, 4, 2, none, 3, true);
    for (int page : {0, 5, 11}) {
        Faults f;
        f.layout = page;
        run_case("layout fault", 12, 6, 6, 4, f, 10u + unsigned(page), true);
    }
    for (int g : {0, 1, 2}) {
        Faults f;
        f.stage = g;
        run_case("stage fault", 12, 6, 6, 3, f, 20u + unsigned(g), true);
        Faults d;
        d.detect = g;
        run_case("detect fault", 12, 6, 6, 3, d, 30u + unsigned(g), true);
        Faults w;
        w.detect_wait = g;
        run_case("detect_wait fault", 12, 6, 6, 3, w, 40u + unsigned(g), true);
        Faults sl;
        sl.detect_stall = g;
        run_case("detect stall", 12, 6, 6, 3, sl, 45u + unsigned(g), true);
    }
    for (int r : {0, 1}) {
        Faults f;
        f.recognize = r;
        run_case("recognize fault", 12, 6, 6, 4, f, 50u + unsigned(r), true);
        Faults d;
        d.decode = r;
        run_case("decode fault", 12, 6, 6, 4, d, 60u + unsigned(r), true);
    }
    {
        // Every page of pass 0 fails before recognition: pass 0 is never recognised.
        Faults f;
        f.stage = 0;
        run_case("whole first group", 2, 2, 6, 2, f, 70, false);
    }
    for (unsigned seed = 100; seed < 120; seed++) run_case("jitter", 17, 3, 4, 1 + int(seed % 4), none, seed, true);
    // Lookahead: a pass waits for the next pass's detections to be queued.
    for (unsigned seed = 200; seed < 210; seed++)
        run_case("lookahead", 13, 3, 2, 1 + int(seed % 3), none, seed, true, true);
    {
        Faults f;
        f.stage = 3;
        run_case("lookahead stage fault", 12, 4, 2, 2, f, 220, true, true);
        Faults g;
        g.layout = 7;
        run_case("lookahead layout fault", 12, 4, 2, 2, g, 221, true, true);
    }
    // Interleaved: recognition passes queue the groups staged meanwhile between their stages.
    {
        int polled = 0;
        for (unsigned seed = 300; seed < 320; seed++)
            polled += run_case("interleave", 12 + int(seed % 6), 3, 2, 1 + int(seed % 3), none, seed, true, false, true);
        for (unsigned seed = 320; seed < 330; seed++)
            polled += run_case("interleave merge 6", 12 + int(seed % 7), 6, 2, 1 + int(seed % 3), none, seed, true,
                               false, true);
        CHECK(polled > 0, "interleave: no group was ever queued from inside a pass");
        Faults d;
        d.detect = 4;
        run_case("interleave detect fault", 12, 3, 2, 2, d, 330, true, false, true);
        Faults st;
        st.stage = 5;
        run_case("interleave stage fault", 12, 3, 2, 2, st, 331, true, false, true);
    }
    // Copies still in flight after stage() returns: a group is detected only once it has landed,
    // and one that never lands is queued after 100 ms anyway (its bounded waits then report it).
    int early = 0;
    for (unsigned seed = 400; seed < 410; seed++)
        run_case("in flight", 12, 6, 4, 1 + int(seed % 3), none, seed, true, false, seed % 2 == 0, 400, -1, -1,
                 nullptr, &early);
    CHECK(early > 0, "in flight: no group needed by the next pass was queued before it landed");
    // Group 3 (pages 3 and 4, the second pass) never lands while the first pass waits 150 ms for
    // page 2's layout: it is queued on the fallback. Without the slow layout the second pass
    // needs it as soon as the first has gone, and it is queued then.
    int fb = 0;
    run_case("never lands", 12, 6, 4, 2, none, 410, true, false, true, 200, 3, 2, &fb);
    CHECK(fb == 1, "never lands: %d groups queued on the fallback", fb);
    run_case("never lands, needed", 12, 6, 4, 2, none, 411, true, false, true, 200, 3);
    if (failures) {
        std::fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    std::printf("pipeline schedule: all checks passed\n");
    return 0;
}
