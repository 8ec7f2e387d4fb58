// GROUP_NORM and NORM (norm.cc) on the device.  Strides in elements.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sdhip.h"
#include "device.h"

namespace sdhip {

struct GroupNormArgs {
    const float *x;
    float *y;
    int64_t ne0, ne1, ne2, ne3;
    int64_t xnb2, xnb3, ynb2, ynb3;
    int64_t groups, per_group;
    int64_t chunk, slices;  // numbers of a slice; slices of a group
    double *partials;       // [2][ne3 * groups][slices]: sums of x, then of (x - mean)^2
    float eps;
    DevChain chain;
};

// How a group norm of these extents splits, and its work buffer's bytes.
struct GroupNormShape {
    int64_t chunk, slices;
    size_t work;
};

GroupNormShape group_norm_shape(int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, int64_t groups);

struct NormArgs {
    const float *x;
    float *y;
    int64_t ne0, ne1, ne2, rows;
    int64_t xnb1, xnb2, xnb3, ynb1, ynb2, ynb3;
    float eps;
    DevChain chain;
};

hipError_t launch_group_norm(const GroupNormArgs &a, hipStream_t stream);

// The static scratch of sdhip_group_norm_static (norm.hip): its bytes, and
// its address on `device`, which must be current (looked up once per device).
constexpr size_t kStaticScratchBytes = size_t(1) << 20;
sdhip_status static_scratch(int device, double *&ptr);
hipError_t launch_norm(const NormArgs &a, hipStream_t stream);

}  // namespace sdhip
