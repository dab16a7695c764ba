// Optional per-launch timing with HIP events recorded on the launch stream.
// Off by default (one relaxed atomic load per launch).  When on, every kernel
// launch of the library is bracketed by two events; natten_hip_profile_read
// waits for them and folds the elapsed times into per-kernel totals.
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "na_launch.h"

namespace na {
namespace {

struct Pending {
    const char* name;
    hipEvent_t start, stop;
};

struct Stat {
    std::string name;
    long long launches = 0;
    double total_ms = 0.0;
    double min_ms = 1e30, max_ms = 0.0;
};

std::atomic<int> g_on{0};
std::mutex g_mu;
std::vector<Pending> g_pending;
std::vector<Stat> g_stats;
std::vector<hipEvent_t> g_free;  // recycled events (creating one per launch is slow)
thread_local Pending t_open{nullptr, nullptr, nullptr};

hipEvent_t take_event() {
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!g_free.empty()) {
            hipEvent_t e = g_free.back();
            g_free.pop_back();
            return e;
        }
    }
    // timing-only events: no system-scope fence (cache write-back and
    // invalidate) on record, which would slow the bracketed kernel and
    // stretch the interval
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
    return e;
}

void give_back(const Pending& p) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (p.start) g_free.push_back(p.start);
    if (p.stop) g_free.push_back(p.stop);
}

}  // namespace

void prof_begin(const char* name, hipStream_t s) {
    if (!g_on.load(std::memory_order_relaxed)) return;
    Pending p{name, take_event(), take_event()};
    // a failed record leaves the launch untimed; the launch itself proceeds
    if (!p.start || !p.stop || hipEventRecord(p.start, s) != hipSuccess) {
        give_back(p);
        return;
    }
    t_open = p;
}

void prof_end(hipStream_t s) {
    if (!t_open.name) return;
    if (hipEventRecord(t_open.stop, s) != hipSuccess) {
        give_back(t_open);
        t_open = Pending{nullptr, nullptr, nullptr};
        return;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    g_pending.push_back(t_open);
    t_open = Pending{nullptr, nullptr, nullptr};
}

}  // namespace na

extern "C" {

int natten_hip_profile_enable(int on) {
    na::g_on.store(on ? 1 : 0);
    return NATTEN_OK;
}

int natten_hip_profile_read(natten_kernel_stat_t* out, int max_entries, int reset) {
    std::lock_guard<std::mutex> lk(na::g_mu);
    for (auto& p : na::g_pending) {
        float ms = 0.f;
        if (hipEventSynchronize(p.stop) == hipSuccess && hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
            na::Stat* st = nullptr;
            for (auto& s : na::g_stats)
                if (s.name == p.name) st = &s;
            if (!st) {
                na::g_stats.push_back(na::Stat{});
                st = &na::g_stats.back();
                st->name = p.name;
            }
            st->launches += 1;
            st->total_ms += ms;
            if (ms < st->min_ms) st->min_ms = ms;
            if (ms > st->max_ms) st->max_ms = ms;
        }
        na::g_free.push_back(p.start);
        na::g_free.push_back(p.stop);
    }
    na::g_pending.clear();
    const int n = static_cast<int>(na::g_stats.size());
    for (int i = 0; i < n && i < max_entries && out; ++i) {
        std::memset(&out[i], 0, sizeof(out[i]));
        std::strncpy(out[i].name, na::g_stats[i].name.c_str(), sizeof(out[i].name) - 1);
        out[i].launches = na::g_stats[i].launches;
        out[i].total_ms = na::g_stats[i].total_ms;
        out[i].min_ms = na::g_stats[i].min_ms;
        out[i].max_ms = na::g_stats[i].max_ms;
    }
    if (reset) na::g_stats.clear();
    return n;
}

}  // extern "C"
