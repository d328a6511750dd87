// Bounded host waits. Every place where a host thread of the library waits for GPU work polls
// through wait_until: it gives up after a deadline and throws WaitTimeout with a description of
// what it waited for (which stream, event, pass or stage), so a stalled queue reports instead of
// leaving the caller silent. The deadline is OCR_WAIT_TIMEOUT_MS milliseconds (default 120000),
// read once per process. Header-only and free of HIP, so the CPU tests can force a deadline.
#pragma once

#include <chrono>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <thread>

namespace ocr {

struct WaitTimeout : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline double wait_timeout_ms() {
    static const double ms = [] {
        const char *v = std::getenv("OCR_WAIT_TIMEOUT_MS");
        const double t = v ? std::atof(v) : 0.0;
        return t > 0 ? t : 120000.0;
    }();
    return ms;
}

// Polls ready() until it returns true. The first 200 microseconds only yield between polls (a
// short wait stays short); after that a poll is followed by a 20-microsecond sleep, which leaves
// the cores to other host work, unless `spin` asks to keep yielding (a wait on the critical
// path, where a sleep's wake-up would add to the run). Past timeout_ms it throws WaitTimeout
// with describe()'s text. ready() may throw (a GPU error), which passes through.
template <class Ready, class Describe>
void wait_until(Ready &&ready, Describe &&describe, bool spin = false, double timeout_ms = wait_timeout_ms()) {
    using Clock = std::chrono::steady_clock;
    if (ready()) return;
    const auto t0 = Clock::now();
    for (;;) {
        const double ms = std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
        if (ms > timeout_ms)
            throw WaitTimeout("GPU work did not finish within " + std::to_string(long(timeout_ms)) +
                              " ms (OCR_WAIT_TIMEOUT_MS): waiting for " + std::string(describe()));
        if (spin || ms < 0.2) std::this_thread::yield();
        else std::this_thread::sleep_for(std::chrono::microseconds(20));
        if (ready()) return;
    }
}

}  // namespace ocr
