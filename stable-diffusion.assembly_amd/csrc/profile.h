// Kernel timing for the profile (profile.cpp).  A KernelScope names the
// kernels launched inside it; with profiling on, every launch goes through
// hipExtLaunchKernel with the scope's events, so that the dispatch packet
// itself stamps them: the elapsed time is the kernels' own execution, from
// the first one's start to the last one's end, without the dispatch latency
// that events recorded around a launch would add.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

namespace sdhip {

bool profiling();

// The events of the innermost open KernelScope of this thread (null when
// profiling is off or no scope is open) and how many kernels it launched.
struct ScopeEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
    int launches = 0;
};
ScopeEvents *active_scope();

class KernelScope {
public:
    KernelScope(const char *name, hipStream_t stream);
    ~KernelScope();
    KernelScope(const KernelScope &) = delete;
    KernelScope &operator=(const KernelScope &) = delete;

private:
    const char *name_;
    ScopeEvents events_;
    ScopeEvents *outer_ = nullptr;
    bool open_ = false;
};

}  // namespace sdhip

// Every kernel of the library is launched by this: a plain launch, or under
// an open scope the same launch with the scope's events (the first kernel
// stamps the start, each one the stop).
#define SDHIP_LAUNCH(kernel, grid, block, shared, stream, ...)                                                     \
    do {                                                                                                           \
        ::sdhip::ScopeEvents *scope_events_ = ::sdhip::active_scope();                                             \
        if (scope_events_ == nullptr) {                                                                            \
            hipLaunchKernelGGL(kernel, grid, block, shared, stream, __VA_ARGS__);                                  \
        } else {                                                                                                   \
            hipExtLaunchKernelGGL(kernel, grid, block, shared, stream,                                             \
                                  scope_events_->launches++ == 0 ? scope_events_->start : nullptr,                 \
                                  scope_events_->stop, 0, __VA_ARGS__);                                            \
        }                                                                                                          \
    } while (0)
