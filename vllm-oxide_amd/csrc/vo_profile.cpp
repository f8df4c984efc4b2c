// vo_profile.cpp -- opt-in per-kernel timing with HIP events.
//
// GPU counterpart of the reference's opt-in per-op timing
// (crates/engine/src/arena.rs:82-87 OpStat, :129-136 enable_profiling,
// :243-255 op()).  When enabled, every kernel launch is bracketed by a pair
// of events recorded on the launch stream; nothing waits for them until
// vo_profile_read, so timing never adds a sync to the hot loop (ADR 0003:
// "Per-op timing is opt-in and never adds a sync").
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "kernels/vo_kernels.hpp"
#include "vo_paged.hpp"

namespace vo {
namespace kernels {

namespace {

struct Pending {
    const char *name;
    hipEvent_t start;
    hipEvent_t stop;
};

struct Stat {
    uint64_t calls = 0;
    double total_ms = 0.0;
    double min_ms = 1e30;
    double max_ms = 0.0;
};

struct Profiler {
    std::mutex mu;
    bool enabled = false;
    std::vector<Pending> pending;
    std::vector<hipEvent_t> free_events;
    std::map<std::string, Stat> stats;

    hipEvent_t get_event() {
        if (!free_events.empty()) {
            hipEvent_t e = free_events.back();
            free_events.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        return e;
    }
};

Profiler &profiler() {
    static Profiler p;
    return p;
}

}  // namespace

KernelTimer::KernelTimer(const char *name, hipStream_t stream) : name_(name), stream_(stream) {
    Profiler &p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    if (!p.enabled) return;
    start_ = p.get_event();
    if (start_ && hipEventRecord(start_, stream_) != hipSuccess) {
        p.free_events.push_back(start_);
        start_ = nullptr;
    }
}

KernelTimer::~KernelTimer() {
    if (!start_) return;
    Profiler &p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    hipEvent_t stop = p.get_event();
    if (stop && hipEventRecord(stop, stream_) == hipSuccess) {
        p.pending.push_back({name_, start_, stop});
    } else {
        p.free_events.push_back(start_);
        if (stop) p.free_events.push_back(stop);
    }
}

}  // namespace kernels
}  // namespace vo

using vo::kernels::profiler;

extern "C" int32_t vo_profiling_enable(int32_t on) {
    auto &p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    p.enabled = on != 0;
    vo::clear_error();
    return VO_OK;
}

extern "C" int32_t vo_profile_read(vo_kernel_stat *out, uint64_t capacity, uint64_t *count) {
    auto &p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    for (const auto &e : p.pending) {
        float ms = 0.0f;
        if (hipEventSynchronize(e.stop) == hipSuccess &&
            hipEventElapsedTime(&ms, e.start, e.stop) == hipSuccess) {
            auto &s = p.stats[e.name];
            s.calls += 1;
            s.total_ms += ms;
            if (ms < s.min_ms) s.min_ms = ms;
            if (ms > s.max_ms) s.max_ms = ms;
        }
        p.free_events.push_back(e.start);
        p.free_events.push_back(e.stop);
    }
    p.pending.clear();
    uint64_t n = 0;
    for (const auto &kv : p.stats) {
        if (out && n < capacity) {
            vo_kernel_stat &o = out[n];
            std::memset(&o, 0, sizeof(o));
            std::snprintf(o.name, sizeof(o.name), "%s", kv.first.c_str());
            o.calls = kv.second.calls;
            o.total_ms = kv.second.total_ms;
            o.min_ms = kv.second.calls ? kv.second.min_ms : 0.0;
            o.max_ms = kv.second.max_ms;
        }
        ++n;
    }
    if (count) *count = n;
    vo::clear_error();
    return VO_OK;
}

extern "C" void vo_profile_reset(void) {
    auto &p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    for (const auto &e : p.pending) {
        (void)hipEventSynchronize(e.stop);
        p.free_events.push_back(e.start);
        p.free_events.push_back(e.stop);
    }
    p.pending.clear();
    p.stats.clear();
}
