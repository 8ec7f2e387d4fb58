// GROUP_NORM and NORM with the chain after them (norm.cc), on the device.
// The statistics are the reference's: the mean as float(sum(x) / n) with the
// sum in double precision; the variance as float(sum((x - mean)^2) / n), each
// difference and square in single precision and the sum in double; the scale
// 1 / sqrt(variance + eps) in single precision, correctly rounded; the output
// (x - mean) * scale and then the chain (norm.cc:44-175).  Only the order of
// the double-precision sums differs from the reference's eight lanes.

#include "host.h"
#include "norm.h"
#include "profile.h"

namespace sdhip {

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

constexpr int kGroupThreads = 1024;

// The sum of a block of kGroupThreads' values, every thread receiving it.
__device__ double group_block_sum(double v, double *scratch) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scratch[wave] = v;
    __syncthreads();
    double s = 0.0;
#pragma unroll
    for (int w = 0; w < kGroupThreads / 64; ++w) s += scratch[w];
    return s;
}

// One block of 16 waves per (image, group): the group's channels are
// consecutive planes, ne0 * ne1 * channels numbers one after another, read
// four at a time where they are aligned.  The output goes channel by channel,
// so that a position's coordinates need no division unless the chain reads
// operands along the rows.
__global__ __launch_bounds__(kGroupThreads) void group_norm_kernel(GroupNormArgs a) {
    __shared__ double scratch[kGroupThreads / 64];
    const int64_t item = blockIdx.x;
    const int64_t i3 = item / a.groups;
    const int64_t g = item % a.groups;
    const int64_t c0 = g * a.per_group;
    const int64_t c1 = c0 + a.per_group < a.ne2 ? c0 + a.per_group : a.ne2;
    if (c0 >= c1) return;
    const int64_t plane = a.ne0 * a.ne1;
    const int64_t count = plane * (c1 - c0);
    const float *x = a.x + i3 * a.xnb3 + c0 * a.xnb2;
    const bool vec = count % 4 == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0;
    const int tid = threadIdx.x;
    double s = 0.0;
    if (vec) {
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        for (int64_t i = tid; i < count / 4; i += kGroupThreads) {
            const float4 v = x4[i];
            s += static_cast<double>(v.x);
            s += static_cast<double>(v.y);
            s += static_cast<double>(v.z);
            s += static_cast<double>(v.w);
        }
    } else {
        for (int64_t i = tid; i < count; i += kGroupThreads) s += static_cast<double>(x[i]);
    }
    const float mean = static_cast<float>(group_block_sum(s, scratch) / static_cast<double>(count));
    double q = 0.0;
    if (vec) {
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        for (int64_t i = tid; i < count / 4; i += kGroupThreads) {
            const float4 v = x4[i];
            const float d0 = v.x - mean, d1 = v.y - mean, d2 = v.z - mean, d3 = v.w - mean;
            q += static_cast<double>(__fmul_rn(d0, d0));
            q += static_cast<double>(__fmul_rn(d1, d1));
            q += static_cast<double>(__fmul_rn(d2, d2));
            q += static_cast<double>(__fmul_rn(d3, d3));
        }
    } else {
        for (int64_t i = tid; i < count; i += kGroupThreads) {
            const float d = x[i] - mean;
            q += static_cast<double>(__fmul_rn(d, d));
        }
    }
    const float variance = static_cast<float>(group_block_sum(q, scratch) / static_cast<double>(count));
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(variance + a.eps));
    float *y = a.y + i3 * a.ynb3 + c0 * a.ynb2;
    // Four numbers of a thread at a time, their chain's loads before their
    // stores; those past the plane read its last and are not stored.
    constexpr int kU = 4;
    for (int64_t c = c0; c < c1; ++c) {
        const float *xc = x + (c - c0) * plane;
        float *yc = y + (c - c0) * plane;
        for (int64_t i = tid; i < plane; i += kGroupThreads * kU) {
            const auto at = [&](int u) -> int64_t {
                const int64_t j = i + static_cast<int64_t>(u) * kGroupThreads;
                return j < plane ? j : plane - 1;
            };
            float v[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) v[u] = __fmul_rn(xc[at(u)] - mean, scale);
            apply_chain_block(a.chain, v, [&](int s, int u) {
                const DevStep &st = a.chain.steps[s];
                int64_t xy = at(u) * st.nb[0];
                if (!st.flat01) {
                    const uint32_t r = static_cast<uint32_t>(at(u)) / static_cast<uint32_t>(a.ne0);
                    xy = (at(u) - static_cast<int64_t>(r) * a.ne0) * st.nb[0] + static_cast<int64_t>(r) * st.nb[1];
                }
                return xy + c * st.nb[2] + i3 * st.nb[3];
            });
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const int64_t j = i + static_cast<int64_t>(u) * kGroupThreads;
                if (j < plane) yc[j] = v[u];
            }
        }
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
    constexpr int kU = 4;
    for (int64_t i = lane; i < a.ne0; i += 64 * kU) {
        const auto at = [&](int u) -> int64_t {
            const int64_t j = i + 64 * u;
            return j < a.ne0 ? j : a.ne0 - 1;
        };
        float v[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) v[u] = __fmul_rn(x[at(u)] - mean, scale);
        apply_chain_block(a.chain, v, [&](int s, int u) {
            const DevStep &st = a.chain.steps[s];
            return at(u) * st.nb[0] + i1 * st.nb[1] + i2 * st.nb[2] + i3 * st.nb[3];
        });
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            if (i + 64 * u < a.ne0) y[i + 64 * u] = v[u];
        }
    }
}

}  // namespace

hipError_t launch_group_norm(const GroupNormArgs &a, hipStream_t stream) {
    KernelScope scope("group_norm", stream);
    hipLaunchKernelGGL(group_norm_kernel, dim3(a.groups * a.ne3), dim3(kGroupThreads), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_norm(const NormArgs &a, hipStream_t stream) {
    KernelScope scope("norm", stream);
    hipLaunchKernelGGL(norm_kernel, dim3(ceil_div(a.rows, kThreads / 64)), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace sdhip
