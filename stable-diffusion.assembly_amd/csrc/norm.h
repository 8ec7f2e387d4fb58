// GROUP_NORM and NORM (norm.cc) on the device.  Strides in elements.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device.h"

namespace sdhip {

struct GroupNormArgs {
    const float *x;
    float *y;
    int64_t ne0, ne1, ne2, ne3;
    int64_t xnb2, xnb3, ynb2, ynb3;
    int64_t groups, per_group;
    float eps;
    DevChain chain;
};

struct NormArgs {
    const float *x;
    float *y;
    int64_t ne0, ne1, ne2, rows;
    int64_t xnb1, xnb2, xnb3, ynb1, ynb2, ynb3;
    float eps;
    DevChain chain;
};

hipError_t launch_group_norm(const GroupNormArgs &a, hipStream_t stream);
hipError_t launch_norm(const NormArgs &a, hipStream_t stream);

}  // namespace sdhip
