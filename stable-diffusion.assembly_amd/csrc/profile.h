// Kernel timing for the profile (profile.cpp): a KernelScope around a launch
// records HIP events on the launch's stream when profiling is on.
#pragma once

#include <hip/hip_runtime.h>

namespace sdhip {

bool profiling();

class KernelScope {
public:
    KernelScope(const char *name, hipStream_t stream);
    ~KernelScope();
    KernelScope(const KernelScope &) = delete;
    KernelScope &operator=(const KernelScope &) = delete;

private:
    const char *name_;
    hipStream_t stream_;
    hipEvent_t start_ = nullptr;
    hipEvent_t stop_ = nullptr;
};

}  // namespace sdhip
