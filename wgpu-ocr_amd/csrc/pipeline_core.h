// The page pipeline's schedule, without the device: which step of which page runs when, on which
// host thread, and what a failure stops. The reference runs it as a GPU thread with a job queue
// and the main thread doing the host work of page k while page k + 1 is detected
// (src/bin/ocr-bench.rs:133-310, 458-585); errors travel per page as Done::Part(page, Err)
// (ocr-bench.rs:277-281, 303-307). Here:
//
//   stager thread:  stage(g)        groups in order (the pages' bytes onto the device)
//   main thread:    detect(g)       once g is staged; recognize(r) once pass r's pages are laid
//                                   out (a staged detection goes first); a pass may call
//                                   poll_detections() between its stages to queue the groups
//                                   staged meanwhile
//   watcher thread: detect_wait(g)  groups in order, once queued
//   worker threads: layout(p)       once p's group is detected and every page of the earlier
//                                   passes is laid out; decode(r) once pass r is queued
//
// A step that throws fails the pages it covers (a group's pages, one page, a pass's pages);
// their later steps are skipped and every other page goes on. Header-only and HIP-free, so the
// schedule is tested on the CPU with hooks that fail on purpose.
#pragma once

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <exception>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace ocr {

// Recognition passes of at most `merge` pages, and detection groups of at most det_batch pages
// that never straddle a pass. With more than `merge` pages the first pass holds ceil(merge / 2)
// and the others share the rest evenly: the first pass is laid out and recognised while later
// pages still upload, where a full one would leave the GPU idle until more pages had arrived.
// The first group is a third of det_batch (at least one page), so the host starts on layouts
// while the GPU detects the rest of the first pass; the last pass's last group is half of
// det_batch rounded up, so that its other pages are detected and laid out while those last pages
// still upload, and less detection and layout follows the last upload. With first_singles (pages
// that arrive from host memory one upload at a time) every page of the first pass is a group of
// its own instead: each is detected as soon as it has landed, and the first pass is ready sooner.
struct PipelinePlan {
    int npages = 0;
    std::vector<int> pass_p0;   // pass r covers pages [pass_p0[r], pass_p0[r + 1])
    std::vector<int> group_p0;  // group g covers pages [group_p0[g], group_p0[g + 1])
    std::vector<int> group_of, pass_of;
    int passes() const { return int(pass_p0.size()) - 1; }
    int groups() const { return int(group_p0.size()) - 1; }
};

inline PipelinePlan plan_pipeline(int npages, int merge, int det_batch, bool first_singles = false) {
    PipelinePlan P;
    P.npages = std::max(npages, 0);
    merge = std::max(merge, 1), det_batch = std::max(det_batch, 1);
    if (P.npages > 0) P.pass_p0.push_back(0);
    if (P.npages > merge) {
        const int first = (merge + 1) / 2, rest = P.npages - first, nr = (rest + merge - 1) / merge;
        for (int k = 0; k < nr; k++) P.pass_p0.push_back(first + int(long(rest) * k / nr));
    }
    P.pass_p0.push_back(P.npages);
    P.group_of.assign(size_t(P.npages), 0);
    P.pass_of.assign(size_t(P.npages), 0);
    for (int r = 0; r < P.passes(); r++) {
        int q0 = P.pass_p0[size_t(r)];
        const int r1 = P.pass_p0[size_t(r) + 1];
        for (int p = q0; p < r1; p++) P.pass_of[size_t(p)] = r;
        if (r == 0 && first_singles && P.passes() > 1) {
            for (int p = q0; p < r1; p++) P.group_p0.push_back(p);
            continue;
        }
        if (r == 0 && r1 - q0 > 1) {
            const int first = std::min(r1 - q0, std::max(1, det_batch / 3));
            P.group_p0.push_back(q0);
            q0 += first;
        }
        const int last = std::max(1, (det_batch + 1) / 2);
        const int tail = (r + 1 == P.passes() && r1 - q0 > last) ? last : 0;
        const int b1 = r1 - tail;
        const int ng = (b1 - q0 + det_batch - 1) / det_batch;
        for (int k = 0; k < ng; k++) P.group_p0.push_back(q0 + int(long(b1 - q0) * k / ng));
        if (tail) P.group_p0.push_back(b1);
    }
    P.group_p0.push_back(P.npages);
    for (int g = 0; g < P.groups(); g++)
        for (int p = P.group_p0[size_t(g)]; p < P.group_p0[size_t(g) + 1]; p++) P.group_of[size_t(p)] = g;
    return P;
}

class PipelineHooks {
  public:
    virtual ~PipelineHooks() = default;
    virtual void stage(int g) = 0;
    // Whether staged group g's pages have reached the device (stage() may return with the copy
    // still in flight). A recognition pass that is ready goes ahead of a group that has not: the
    // group would only hold the stream until it lands.
    virtual bool landed(int) { return true; }
    virtual void detect(int g) = 0;
    virtual void detect_wait(int g) = 0;
    virtual void layout(int p) = 0;
    // ok[p - first page of r]: page p has a layout (pages without one are left out).
    virtual void recognize(int r, const std::vector<char> &ok) = 0;
    virtual void decode(int r, bool last) = 0;
    // Set by run_schedule while it runs (main thread only): queues, in order, the detection groups
    // that are staged, landed and not yet queued, returns whether it queued any. A recognition pass may call it
    // between its stages, so that pages which reach the device meanwhile are detected after the
    // stage in flight rather than after the whole pass.
    std::function<bool()> poll_detections;
    // Set with poll_detections: whether some detection group is not queued yet (staged or not).
    // A pass that knows one is still to come can wait on its stage in flight, polling, so the
    // group goes right behind that stage.
    std::function<bool()> detections_pending;
};

// Runs fn on a worker thread (the caller's pool); must not block the calling thread.
using SubmitFn = std::function<void(std::function<void()>)>;

// Runs the plan. Returns every page's error ("" for a page that finished). Never throws: a
// failure of a step fails its pages. cpu_busy_ms (if given) receives the worker time spent in
// layout and decode. lookahead: pass r is queued only once every detection group of pass r + 1
// is queued too (on one in-order stream a recognition pass would otherwise hold back the next
// pages' detection, and with it their host layouts, for its whole length).
inline std::vector<std::string> run_schedule(const PipelinePlan &P, PipelineHooks &H, const SubmitFn &submit,
                                             double *cpu_busy_ms = nullptr, bool lookahead = false) {
    using clk = std::chrono::steady_clock;
    const int np = P.npages, ng = P.groups(), nr = P.passes();
    std::vector<std::string> err(static_cast<size_t>(np));
    if (np == 0) return err;
    std::mutex mu;
    std::condition_variable cv;
    // Progress, all under mu.
    int staged = 0, queued = 0, detected = 0, pending = 0;
    std::vector<char> group_failed(size_t(ng), 0), laid(size_t(np), 0), ok(size_t(np), 0);
    double busy = 0;
    auto what = [](const std::exception_ptr &e) -> std::string {
        try {
            std::rethrow_exception(e);
        } catch (const std::exception &x) {
            return x.what();
        } catch (...) {
            return "unknown error";
        }
    };
    // Fails pages [p0, p1) that have not failed yet (mu held).
    auto fail_pages = [&](int p0, int p1, const std::string &m) {
        for (int p = p0; p < p1; p++)
            if (err[size_t(p)].empty()) err[size_t(p)] = m.empty() ? "failed" : m;
    };
    auto group_pages = [&](int g, int &p0, int &p1) { p0 = P.group_p0[size_t(g)], p1 = P.group_p0[size_t(g) + 1]; };

    std::thread stager([&] {
        for (int g = 0; g < ng; g++) {
            std::string m;
            try {
                H.stage(g);
            } catch (...) {
                m = what(std::current_exception());
            }
            std::lock_guard<std::mutex> lk(mu);
            if (!m.empty()) {
                int p0, p1;
                group_pages(g, p0, p1);
                fail_pages(p0, p1, m);
                group_failed[size_t(g)] = 1;
            }
            staged = g + 1;
            cv.notify_all();
        }
    });
    std::thread watcher([&] {
        for (int g = 0; g < ng; g++) {
            bool skip;
            {
                std::unique_lock<std::mutex> lk(mu);
                cv.wait(lk, [&] { return queued > g; });
                skip = group_failed[size_t(g)] != 0;
            }
            std::string m;
            if (!skip) {
                try {
                    H.detect_wait(g);
                } catch (...) {
                    m = what(std::current_exception());
                }
            }
            std::lock_guard<std::mutex> lk(mu);
            if (!m.empty()) {
                int p0, p1;
                group_pages(g, p0, p1);
                fail_pages(p0, p1, m);
                group_failed[size_t(g)] = 1;
            }
            detected = g + 1;
            cv.notify_all();
        }
    });
    // Layout tasks: every page, waiting for its group and the earlier passes.
    for (int p = 0; p < np; p++) {
        {
            std::lock_guard<std::mutex> lk(mu);
            pending++;
        }
        submit([&, p] {
            const int g = P.group_of[size_t(p)], before = P.pass_p0[size_t(P.pass_of[size_t(p)])];
            bool run_it;
            {
                std::unique_lock<std::mutex> lk(mu);
                cv.wait(lk, [&] {
                    if (detected <= g) return false;
                    for (int q = 0; q < before; q++)
                        if (!laid[size_t(q)]) return false;
                    return true;
                });
                run_it = err[size_t(p)].empty();
            }
            std::string m;
            double t = 0;
            if (run_it) {
                const auto t0 = clk::now();
                try {
                    H.layout(p);
                } catch (...) {
                    m = what(std::current_exception());
                }
                t = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
            }
            std::lock_guard<std::mutex> lk(mu);
            if (!m.empty()) fail_pages(p, p + 1, m);
            ok[size_t(p)] = err[size_t(p)].empty();
            laid[size_t(p)] = 1;
            busy += t;
            pending--;
            cv.notify_all();
        });
    }
    // Main thread: detections as soon as staged, recognition passes as soon as laid out.
    int next_det = 0, next_rec = 0;
    // Queues detection group g (next_det already moved past it, mu not held).
    auto queue_group = [&](int g) {
        std::string m;
        try {
            H.detect(g);
        } catch (...) {
            m = what(std::current_exception());
        }
        std::lock_guard<std::mutex> lk(mu);
        if (!m.empty()) {
            int p0, p1;
            group_pages(g, p0, p1);
            fail_pages(p0, p1, m);
            group_failed[size_t(g)] = 1;
        }
        queued = next_det;
        cv.notify_all();
    };
    H.poll_detections = [&]() -> bool {
        bool any = false;
        for (;;) {
            int g;
            {
                std::lock_guard<std::mutex> lk(mu);
                if (next_det >= ng || staged <= next_det || !H.landed(next_det)) return any;
                g = next_det++;
                if (group_failed[size_t(g)]) {
                    queued = next_det;
                    cv.notify_all();
                    continue;
                }
            }
            queue_group(g);
            any = true;
        }
    };
    H.detections_pending = [&]() -> bool {
        std::lock_guard<std::mutex> lk(mu);
        return next_det < ng;
    };
    while (next_rec < nr) {
        int do_det = -1, do_rec = -1;
        std::vector<char> pass_ok;
        {
            std::unique_lock<std::mutex> lk(mu);
            auto pass_ready = [&](int r) {
                for (int p = P.pass_p0[size_t(r)]; p < P.pass_p0[size_t(r) + 1]; p++)
                    if (!laid[size_t(p)]) return false;
                return true;
            };
            // Groups that must be queued before pass r: those of passes r and r + 1.
            auto groups_before = [&](int r) {
                const int q = P.pass_p0[size_t(std::min(r + (lookahead ? 2 : 1), nr))];
                return q >= np ? ng : P.group_of[size_t(q)];
            };
            // A staged group goes first once it has landed; a ready pass goes ahead of a group
            // still in flight (one the next pass does not need). While such a group is in flight
            // and no pass is ready, look again every 20 us, for at most 100 ms (then the group is
            // queued anyway, and the stream's own bounded waits report a copy that never ends).
            auto staged_next = [&] { return next_det < ng && staged > next_det; };
            auto rec_now = [&] { return pass_ready(next_rec) && next_det >= groups_before(next_rec); };
            // A group the next pass still needs goes at once, landed or not: no pass can run
            // before it, and the stream's own wait for its copy starts it the moment it lands.
            auto needed = [&] { return next_rec >= nr || next_det < groups_before(next_rec); };
            bool take_det = false;
            const auto t_in = clk::now();
            for (;;) {
                if (staged_next() && (needed() || H.landed(next_det) ||
                                      clk::now() - t_in > std::chrono::milliseconds(100))) {
                    take_det = true;
                    break;
                }
                if (rec_now()) break;
                if (staged_next()) {
                    // A plain sleep (a timed condition wait on the steady clock is a call that
                    // thread checkers do not follow).
                    lk.unlock();
                    std::this_thread::sleep_for(std::chrono::microseconds(20));
                    lk.lock();
                } else {
                    cv.wait(lk, [&] { return staged_next() || rec_now(); });
                }
            }
            if (take_det) {
                do_det = next_det++;
                if (group_failed[size_t(do_det)]) {
                    queued = next_det;  // nothing to queue, nothing to wait for
                    cv.notify_all();
                    continue;
                }
            } else {
                do_rec = next_rec++;
                const int p0 = P.pass_p0[size_t(do_rec)], p1 = P.pass_p0[size_t(do_rec) + 1];
                pass_ok.assign(ok.begin() + p0, ok.begin() + p1);
            }
        }
        if (do_det >= 0) {
            queue_group(do_det);
            continue;
        }
        const int r = do_rec, p0 = P.pass_p0[size_t(r)], p1 = P.pass_p0[size_t(r) + 1];
        if (std::none_of(pass_ok.begin(), pass_ok.end(), [](char c) { return c != 0; })) continue;
        std::string m;
        try {
            H.recognize(r, pass_ok);
        } catch (...) {
            m = what(std::current_exception());
        }
        if (!m.empty()) {
            std::lock_guard<std::mutex> lk(mu);
            fail_pages(p0, p1, m);
            continue;
        }
        {
            std::lock_guard<std::mutex> lk(mu);
            pending++;
        }
        const bool last = r == nr - 1;
        submit([&, r, p0, p1, last] {
            std::string m2;
            const auto t0 = clk::now();
            try {
                H.decode(r, last);
            } catch (...) {
                m2 = what(std::current_exception());
            }
            const double t = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
            std::lock_guard<std::mutex> lk(mu);
            if (!m2.empty()) fail_pages(p0, p1, m2);
            busy += t;
            pending--;
            cv.notify_all();
        });
    }
    H.poll_detections = nullptr;
    H.detections_pending = nullptr;
    // Detections queued after the last pass (none in a valid plan), then every task and thread.
    {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] { return staged == ng; });
        queued = ng;
        cv.notify_all();
        cv.wait(lk, [&] { return pending == 0 && detected == ng; });
    }
    stager.join();
    watcher.join();
    if (cpu_busy_ms) *cpu_busy_ms = busy;
    return err;
}

}  // namespace ocr
