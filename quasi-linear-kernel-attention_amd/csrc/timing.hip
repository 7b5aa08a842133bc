// Opt-in per-stage timing. When enabled (qlka_timing_enable(1)), every kernel launch of the library is bracketed by
// two hipEvents recorded on the launch's own stream; qlka_timing_read() synchronises the recorded events and returns
// the accumulated milliseconds and launch count of one stage. Off by default: then no event is created or recorded.
// The pseudo-stage "busy" is the union of all bracketed intervals: the time in which at least one library kernel
// ran, which differs from the sum over stages when launches on two streams overlap.
#include "qlka.h"
#include "qlka_internal.h"

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace qlka {

namespace {
struct Pending { std::string name; hipEvent_t a, b; };
struct Totals { double ms = 0; long long count = 0; };
std::atomic<int> g_on{0};
std::mutex g_mu;
std::vector<Pending> g_pending;
std::map<std::string, Totals> g_totals;

void drain_locked() {
    std::vector<std::pair<float, float>> spans;     // [start, end] relative to the first launch's start
    for (auto& p : g_pending) {
        float ms = 0.f, t0 = 0.f, t1 = 0.f;
        if (hipEventSynchronize(p.b) == hipSuccess && hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            auto& t = g_totals[p.name];
            t.ms += ms;
            t.count += 1;
            if (hipEventElapsedTime(&t0, g_pending[0].a, p.a) == hipSuccess &&
                hipEventElapsedTime(&t1, g_pending[0].a, p.b) == hipSuccess)
                spans.emplace_back(t0, t1);
        }
    }
    std::sort(spans.begin(), spans.end());
    double busy = 0.0;
    float lo = 0.f, hi = 0.f;
    for (size_t i = 0; i < spans.size(); ++i) {
        if (i == 0 || spans[i].first > hi) {
            busy += hi - lo;
            lo = spans[i].first;
            hi = spans[i].second;
        } else {
            hi = std::max(hi, spans[i].second);
        }
    }
    busy += hi - lo;
    if (!spans.empty()) g_totals["busy"].ms += busy;
    for (auto& p : g_pending) {
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    g_pending.clear();
}
}  // namespace

StageTimer::StageTimer(const char* name, hipStream_t st) : name_(name), st_(st) {
    if (!g_on.load(std::memory_order_relaxed)) return;
    if (hipEventCreate(&a_) != hipSuccess) { a_ = nullptr; return; }
    if (hipEventCreate(&b_) != hipSuccess) { (void)hipEventDestroy(a_); a_ = nullptr; b_ = nullptr; return; }
    (void)hipEventRecord(a_, st_);
}

StageTimer::~StageTimer() {
    if (!a_) return;
    (void)hipEventRecord(b_, st_);
    std::lock_guard<std::mutex> lk(g_mu);
    g_pending.push_back({name_, a_, b_});
}

}  // namespace qlka

extern "C" {

int qlka_timing_enable(int on) {
    qlka::g_on.store(on ? 1 : 0);
    return QLKA_OK;
}

int qlka_timing_reset(void) {
    std::lock_guard<std::mutex> lk(qlka::g_mu);
    qlka::drain_locked();
    qlka::g_totals.clear();
    return QLKA_OK;
}

int qlka_timing_read(const char* stage, double* total_ms, long long* count) {
    std::lock_guard<std::mutex> lk(qlka::g_mu);
    qlka::drain_locked();
    auto it = qlka::g_totals.find(stage ? stage : "");
    if (total_ms) *total_ms = (it == qlka::g_totals.end()) ? 0.0 : it->second.ms;
    if (count) *count = (it == qlka::g_totals.end()) ? 0 : it->second.count;
    return QLKA_OK;
}

}  // extern "C"
