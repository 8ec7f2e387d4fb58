// GROUP_NORM and NORM with the chain after them (norm.cc), on the device.
// The statistics are the reference's: the mean as float(sum(x) / n) with the
// sum in double precision; the variance as float(sum((x - mean)^2) / n), each
// difference and square in single precision and the sum in double; the scale
// 1 / sqrt(variance + eps) in single precision, correctly rounded; the output
// (x - mean) * scale and then the chain (norm.cc:44-175).  Only the order of
// the double-precision sums differs from the reference's eight lanes.

#include "host.h"
#include "norm.h"

namespace sdhip {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// The sum of a block's values, every thread receiving it.
__device__ double block_sum(double v, double *scratch) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scratch[wave] = v;
    __syncthreads();
    double s = 0.0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) s += scratch[w];
    return s;
}

// One block per (image, group): the group's channels are consecutive planes,
// ne0 * ne1 * channels numbers one after another.
__global__ __launch_bounds__(kThreads) void group_norm_kernel(GroupNormArgs a) {
    __shared__ double scratch[kThreads / 64];
    const int64_t item = blockIdx.x;
    const int64_t i3 = item / a.groups;
    const int64_t g = item % a.groups;
    const int64_t c0 = g * a.per_group;
    const int64_t c1 = c0 + a.per_group < a.ne2 ? c0 + a.per_group : a.ne2;
    if (c0 >= c1) return;
    const int64_t plane = a.ne0 * a.ne1;
    const int64_t count = plane * (c1 - c0);
    const float *x = a.x + i3 * a.xnb3 + c0 * a.xnb2;
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < count; i += kThreads) s += static_cast<double>(x[i]);
    const float mean = static_cast<float>(block_sum(s, scratch) / static_cast<double>(count));
    double q = 0.0;
    for (int64_t i = threadIdx.x; i < count; i += kThreads) {
        const float d = x[i] - mean;
        q += static_cast<double>(__fmul_rn(d, d));
    }
    const float variance = static_cast<float>(block_sum(q, scratch) / static_cast<double>(count));
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(variance + a.eps));
    float *y = a.y + i3 * a.ynb3 + c0 * a.ynb2;
    for (int64_t i = threadIdx.x; i < count; i += kThreads) {
        const int64_t c = i / plane;
        const int64_t r = (i - c * plane) / a.ne0;
        const int64_t i0 = i - c * plane - r * a.ne0;
        const float v = __fmul_rn(x[i] - mean, scale);
        y[i] = apply_chain(a.chain, v, i0, r, c0 + c, i3);
    }
}

// One wave per row of ne0.
__global__ __launch_bounds__(kThreads) void norm_kernel(NormArgs a) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const int lane = threadIdx.x & 63;
    const int64_t i1 = row % a.ne1;
    const int64_t i2 = (row / a.ne1) % a.ne2;
    const int64_t i3 = row / (a.ne1 * a.ne2);
    const float *x = a.x + i1 * a.xnb1 + i2 * a.xnb2 + i3 * a.xnb3;
    float *y = a.y + i1 * a.ynb1 + i2 * a.ynb2 + i3 * a.ynb3;
    double s = 0.0;
    for (int64_t i = lane; i < a.ne0; i += 64) s += static_cast<double>(x[i]);
    const float mean = static_cast<float>(wave_sum(s) / static_cast<double>(a.ne0));
    double q = 0.0;
    for (int64_t i = lane; i < a.ne0; i += 64) {
        const float d = x[i] - mean;
        q += static_cast<double>(__fmul_rn(d, d));
    }
    const float variance = static_cast<float>(wave_sum(q) / static_cast<double>(a.ne0));
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(variance + a.eps));
    for (int64_t i = lane; i < a.ne0; i += 64) {
        const float v = __fmul_rn(x[i] - mean, scale);
        y[i] = apply_chain(a.chain, v, i, i1, i2, i3);
    }
}

}  // namespace

hipError_t launch_group_norm(const GroupNormArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(group_norm_kernel, dim3(a.groups * a.ne3), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_norm(const NormArgs &a, hipStream_t stream) {
    hipLaunchKernelGGL(norm_kernel, dim3(ceil_div(a.rows, kThreads / 64)), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace sdhip
