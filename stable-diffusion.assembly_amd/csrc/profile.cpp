// The profile of the library's kernels: with sdhip_profile_enable(1), the
// kernels of every KernelScope stamp two HIP events from their own dispatch
// packets (profile.h), and sdhip_profile_collect() adds the elapsed times up
// per scope name.  The reference's profile (profile.cc, sdasm_profile_*)
// times each node and each phase of it on the CPU; here the phases are the
// kernels.

#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "host.h"
#include "profile.h"

namespace sdhip {

namespace {

struct Pending {
    std::string name;
    hipEvent_t start, stop;
};

struct Totals {
    double ms = 0.0;
    int64_t launches = 0;
};

struct Profile {
    std::mutex lock;
    bool enabled = false;
    std::vector<Pending> pending;
    std::vector<hipEvent_t> spare;
    std::map<std::string, Totals> totals;
    std::vector<std::string> names;  // stable storage for sdhip_profile_entry
};

Profile &profile() {
    static Profile p;
    return p;
}

hipEvent_t take_event(Profile &p) {
    if (!p.spare.empty()) {
        hipEvent_t e = p.spare.back();
        p.spare.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    return hipEventCreate(&e) == hipSuccess ? e : nullptr;
}

}  // namespace

bool profiling() { return profile().enabled; }

namespace {
thread_local ScopeEvents *innermost = nullptr;
}

ScopeEvents *active_scope() { return innermost; }

KernelScope::KernelScope(const char *name, hipStream_t) : name_(name) {
    Profile &p = profile();
    if (!p.enabled) return;
    {
        std::lock_guard<std::mutex> g(p.lock);
        events_.start = take_event(p);
        events_.stop = take_event(p);
    }
    if (events_.start == nullptr || events_.stop == nullptr) {
        std::lock_guard<std::mutex> g(p.lock);
        if (events_.start != nullptr) p.spare.push_back(events_.start);
        if (events_.stop != nullptr) p.spare.push_back(events_.stop);
        return;
    }
    outer_ = innermost;
    innermost = &events_;
    open_ = true;
}

KernelScope::~KernelScope() {
    if (!open_) return;
    innermost = outer_;
    Profile &p = profile();
    std::lock_guard<std::mutex> g(p.lock);
    if (events_.launches > 0) {
        p.pending.push_back({name_, events_.start, events_.stop});
    } else {
        p.spare.push_back(events_.start);
        p.spare.push_back(events_.stop);
    }
}

}  // namespace sdhip

using namespace sdhip;

extern "C" {

void sdhip_profile_enable(int on) { profile().enabled = on != 0; }

void sdhip_profile_reset(void) {
    Profile &p = profile();
    std::lock_guard<std::mutex> g(p.lock);
    p.totals.clear();
}

int sdhip_profile_collect(void) {
    Profile &p = profile();
    std::lock_guard<std::mutex> g(p.lock);
    for (Pending &e : p.pending) {
        float ms = 0.0f;
        if (hipEventSynchronize(e.stop) != hipSuccess || hipEventElapsedTime(&ms, e.start, e.stop) != hipSuccess)
            ms = 0.0f;
        Totals &t = p.totals[e.name];
        t.ms += ms;
        t.launches += 1;
        p.spare.push_back(e.start);
        p.spare.push_back(e.stop);
    }
    p.pending.clear();
    p.names.clear();
    for (auto &kv : p.totals) p.names.push_back(kv.first);
    return static_cast<int>(p.names.size());
}

int sdhip_profile_entry(int i, const char **name, double *total_ms, int64_t *launches) {
    Profile &p = profile();
    std::lock_guard<std::mutex> g(p.lock);
    if (i < 0 || i >= static_cast<int>(p.names.size())) return 0;
    const Totals &t = p.totals[p.names[i]];
    *name = p.names[i].c_str();
    *total_ms = t.ms;
    *launches = t.launches;
    return 1;
}

}  // extern "C"
