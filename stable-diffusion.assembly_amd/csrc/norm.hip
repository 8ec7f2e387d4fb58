// GROUP_NORM and NORM with the chain after them (norm.cc), on the device.
// The statistics are the reference's: the mean as float(sum(x) / n) with the
// sum in double precision; the variance as float(sum((x - mean)^2) / n), each
// difference and square in single precision and the sum in double; the scale
// 1 / sqrt(variance + eps) in single precision, correctly rounded; the output
// (x - mean) * scale and then the chain (norm.cc:44-175).  Only the order of
// the double-precision sums differs from the reference's eight lanes.

#include <mutex>

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

// GROUP_NORM in three launches over blocks of (image, group, slice), the
// slices `chunk` consecutive numbers of the group's channels (consecutive
// planes, ne0 * ne1 numbers each): the partial sums of x; from their total
// the mean, and the partial sums of (x - mean)^2; from both totals the scale,
// and the output with its chain.  Each sum of a slice goes to the work buffer
// and is added up, in the order of the slices, by each block that needs the
// total.

struct GroupView {
    int64_t item, slice, i3, c0, count, e0, e1;
};

__device__ __forceinline__ GroupView group_view(const GroupNormArgs &a) {
    GroupView v;
    v.item = blockIdx.x / a.slices;
    v.slice = blockIdx.x - v.item * a.slices;
    v.i3 = v.item / a.groups;
    const int64_t g = v.item - v.i3 * a.groups;
    v.c0 = g * a.per_group;
    const int64_t c1 = v.c0 + a.per_group < a.ne2 ? v.c0 + a.per_group : a.ne2;
    v.count = v.c0 < c1 ? (c1 - v.c0) * a.ne0 * a.ne1 : 0;
    v.e0 = v.slice * a.chunk;
    v.e1 = v.e0 + a.chunk < v.count ? v.e0 + a.chunk : v.count;
    return v;
}

__device__ __forceinline__ double block_sum(double v, double *lds_sums) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds_sums[threadIdx.x >> 6] = v;
    __syncthreads();
    double s = 0.0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) s += lds_sums[w];
    return s;
}

// The total over the slices of an item, in their order.
__device__ __forceinline__ double total(const double *partials, int64_t item, int64_t slices) {
    double t = 0.0;
    for (int64_t q = 0; q < slices; ++q) t += partials[item * slices + q];
    return t;
}

// PASS 0: the sum of x over the block's slice; PASS 1: of (x - mean)^2, each
// difference and square in single precision (norm.cc:44-90).
template <int PASS>
__device__ __forceinline__ double term(float x, float mean) {
    if (PASS == 0) return static_cast<double>(x);
    const float d = x - mean;
    return static_cast<double>(__fmul_rn(d, d));
}

template <int PASS>
__global__ __launch_bounds__(kThreads) void group_sums_kernel(GroupNormArgs a) {
    __shared__ double lds_sums[kThreads / 64];
    __shared__ float shared_mean;
    const GroupView g = group_view(a);
    const int tid = threadIdx.x;
    float mean = 0.0f;
    if (PASS == 1) {
        if (tid == 0 && g.count > 0) {
            shared_mean = static_cast<float>(total(a.partials, g.item, a.slices) / static_cast<double>(g.count));
        }
        __syncthreads();
        mean = shared_mean;
    }
    const float *x = a.x + g.i3 * a.xnb3 + g.c0 * a.xnb2;
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        // a.chunk is a multiple of 4: the slice's quads start at e0 / 4.
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        const int64_t q1 = g.e1 / 4;
        int64_t i = g.e0 / 4 + tid;
        for (; i + 3 * kThreads < q1; i += 4 * kThreads) {
            const float4 v0 = x4[i], v1 = x4[i + kThreads], v2 = x4[i + 2 * kThreads], v3 = x4[i + 3 * kThreads];
            s0 += term<PASS>(v0.x, mean) + term<PASS>(v0.y, mean) + term<PASS>(v0.z, mean) + term<PASS>(v0.w, mean);
            s1 += term<PASS>(v1.x, mean) + term<PASS>(v1.y, mean) + term<PASS>(v1.z, mean) + term<PASS>(v1.w, mean);
            s2 += term<PASS>(v2.x, mean) + term<PASS>(v2.y, mean) + term<PASS>(v2.z, mean) + term<PASS>(v2.w, mean);
            s3 += term<PASS>(v3.x, mean) + term<PASS>(v3.y, mean) + term<PASS>(v3.z, mean) + term<PASS>(v3.w, mean);
        }
        for (; i < q1; i += kThreads) {
            const float4 v0 = x4[i];
            s0 += term<PASS>(v0.x, mean) + term<PASS>(v0.y, mean) + term<PASS>(v0.z, mean) + term<PASS>(v0.w, mean);
        }
        for (int64_t e = q1 * 4 + tid; e < g.e1; e += kThreads) s1 += term<PASS>(x[e], mean);
    } else {
        for (int64_t e = g.e0 + tid; e < g.e1; e += kThreads) s0 += term<PASS>(x[e], mean);
    }
    const double sum = block_sum((s0 + s1) + (s2 + s3), lds_sums);
    if (tid == 0) a.partials[(PASS * a.ne3 * a.groups + g.item) * a.slices + g.slice] = sum;
}

// The most channels a slice's operands of one number a channel are held
// for in LDS.
constexpr int kApplyChannels = 256;

// The output of the block's slice, (x - mean) * scale and the chain, four
// consecutive numbers of a thread at a time where the planes allow (the four
// then share their channel); all loads of a step before its stores.
__global__ __launch_bounds__(kThreads) void group_apply_kernel(GroupNormArgs a) {
    __shared__ float shared[2];
    const GroupView g = group_view(a);
    const int tid = threadIdx.x;
    if (tid == 0 && g.count > 0) {
        const double n = static_cast<double>(g.count);
        const float mean = static_cast<float>(total(a.partials, g.item, a.slices) / n);
        const float variance =
            static_cast<float>(total(a.partials + a.ne3 * a.groups * a.slices, g.item, a.slices) / n);
        shared[0] = mean;
        shared[1] = __fdiv_rn(1.0f, __fsqrt_rn(variance + a.eps));
    }
    __syncthreads();
    const float mean = shared[0], scale = shared[1];
    const int64_t plane = a.ne0 * a.ne1;
    const float *x = a.x + g.i3 * a.xnb3 + g.c0 * a.xnb2;
    float *y = a.y + g.i3 * a.ynb3 + g.c0 * a.ynb2;
    // A step whose operand is one number per channel (and image) reads one.
    bool per_channel = true;
    for (int s = 0; s < a.chain.count; ++s) {
        const DevStep &st = a.chain.steps[s];
        if (st.kind != 2 && (st.nb[0] != 0 || st.nb[1] != 0)) per_channel = false;
    }
    const auto offset = [&](const DevStep &st, int64_t c, int64_t p) -> int64_t {
        const int64_t c_part = (g.c0 + c) * st.nb[2] + g.i3 * st.nb[3];
        if (per_channel) return c_part;
        const uint32_t r = static_cast<uint32_t>(p) / static_cast<uint32_t>(a.ne0);
        return (p - static_cast<int64_t>(r) * a.ne0) * st.nb[0] + static_cast<int64_t>(r) * st.nb[1] + c_part;
    };
    const bool quads = plane % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                       (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    // Operands of one number a channel, for the channels of the slice (few
    // enough): loaded once into LDS, and the slice's quads four a thread at a
    // time, all four loads issued before any is used -- no global load waits
    // on another inside the loop.
    __shared__ float chan_ops[kMaxSteps][kApplyChannels];
    const int64_t c_first = g.e0 / plane;
    const int64_t nch = g.e1 > g.e0 ? (g.e1 - 1) / plane - c_first + 1 : 0;
    if (quads && per_channel && nch <= kApplyChannels) {
        for (int s = 0; s < a.chain.count; ++s) {
            const DevStep &st = a.chain.steps[s];
            if (st.kind == 2) continue;
            for (int64_t ch = tid; ch < nch; ch += kThreads) chan_ops[s][ch] = st.operand[offset(st, c_first + ch, 0)];
        }
        __syncthreads();
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        float4 *y4 = reinterpret_cast<float4 *>(y);
        const int64_t q_end = g.e1 / 4;
        constexpr int kBatch = 4;
        for (int64_t q0 = g.e0 / 4 + tid; q0 < q_end; q0 += kBatch * kThreads) {
            float4 q[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int64_t i = q0 + u * kThreads;
                q[u] = x4[i < q_end ? i : q0];
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int64_t i = q0 + u * kThreads;
                if (i >= q_end) continue;
                const int64_t ch = static_cast<int64_t>(static_cast<uint32_t>(4 * i) / static_cast<uint32_t>(plane)) -
                                   c_first;
                float v[4] = {__fmul_rn(q[u].x - mean, scale), __fmul_rn(q[u].y - mean, scale),
                              __fmul_rn(q[u].z - mean, scale), __fmul_rn(q[u].w - mean, scale)};
#pragma unroll 1
                for (int s = 0; s < a.chain.count; ++s) {
                    const int kind = a.chain.steps[s].kind;
                    if (kind == 2) {
#pragma unroll
                        for (int k = 0; k < 4; ++k) v[k] = silu(v[k]);
                        continue;
                    }
                    const float b = chan_ops[s][ch];
#pragma unroll
                    for (int k = 0; k < 4; ++k) v[k] = kind == 0 ? __fadd_rn(v[k], b) : __fmul_rn(v[k], b);
                }
                y4[i] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
        return;
    }
    if (quads) {
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        float4 *y4 = reinterpret_cast<float4 *>(y);
        for (int64_t i = g.e0 / 4 + tid; i < g.e1 / 4; i += kThreads) {
            const float4 q = x4[i];
            const int64_t e = i * 4;
            const uint32_t c = static_cast<uint32_t>(e) / static_cast<uint32_t>(plane);
            const int64_t p = e - static_cast<int64_t>(c) * plane;
            float v[4] = {__fmul_rn(q.x - mean, scale), __fmul_rn(q.y - mean, scale), __fmul_rn(q.z - mean, scale),
                          __fmul_rn(q.w - mean, scale)};
#pragma unroll 1
            for (int s = 0; s < a.chain.count; ++s) {
                const DevStep &st = a.chain.steps[s];
                if (st.kind == 2) {
#pragma unroll
                    for (int u = 0; u < 4; ++u) v[u] = silu(v[u]);
                    continue;
                }
                float o[4];
                if (per_channel) {
                    const float b = st.operand[offset(st, c, p)];
#pragma unroll
                    for (int u = 0; u < 4; ++u) o[u] = b;
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u) o[u] = st.operand[offset(st, c, p + u)];
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = st.kind == 0 ? __fadd_rn(v[u], o[u]) : __fmul_rn(v[u], o[u]);
            }
            y4[i] = make_float4(v[0], v[1], v[2], v[3]);
        }
        return;
    }
    for (int64_t e = g.e0 + tid; e < g.e1; e += kThreads) {
        const uint32_t c = static_cast<uint32_t>(e) / static_cast<uint32_t>(plane);
        const int64_t p = e - static_cast<int64_t>(c) * plane;
        float v = __fmul_rn(x[e] - mean, scale);
#pragma unroll 1
        for (int s = 0; s < a.chain.count; ++s) {
            const DevStep &st = a.chain.steps[s];
            if (st.kind == 2) {
                v = silu(v);
                continue;
            }
            const float o = st.operand[offset(st, c, p)];
            v = st.kind == 0 ? __fadd_rn(v, o) : __fmul_rn(v, o);
        }
        y[e] = v;
    }
}

// GROUP_NORM of small groups in one launch: a block of 1024 threads per
// (image, group) holds the group's count <= kResident numbers in registers,
// four consecutive numbers of one channel a thread at a time (planes of a
// multiple of 4), and takes the same statistics as the three launches above
// -- float(sum / n) with the sum in double, then float(sum of the single-
// precision squares of x - mean / n) -- with x read once.
constexpr int kResidentThreads = 1024;
constexpr int kResidentQuads = 4;  // float4 a thread
constexpr int64_t kResident = int64_t(kResidentThreads) * 4 * kResidentQuads;

__device__ __forceinline__ double block_sum_wide(double v, double *lds_sums) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds_sums[threadIdx.x >> 6] = v;
    __syncthreads();
    double s = 0.0;
#pragma unroll
    for (int w = 0; w < kResidentThreads / 64; ++w) s += lds_sums[w];
    return s;
}

__global__ __launch_bounds__(kResidentThreads) void group_norm_resident_kernel(GroupNormArgs a) {
    __shared__ double lds_sums[kResidentThreads / 64];
    const int tid = threadIdx.x;
    const int64_t item = blockIdx.x;
    const int64_t i3 = item / a.groups;
    const int64_t g = item - i3 * a.groups;
    const int64_t c0 = g * a.per_group;
    const int64_t c1 = c0 + a.per_group < a.ne2 ? c0 + a.per_group : a.ne2;
    const int64_t count = c0 < c1 ? (c1 - c0) * a.ne0 * a.ne1 : 0;
    const int64_t plane = a.ne0 * a.ne1;
    const float4v *x4 = reinterpret_cast<const float4v *>(a.x + i3 * a.xnb3 + c0 * a.xnb2);
    float4v v[kResidentQuads];
    double s = 0.0;
#pragma unroll
    for (int u = 0; u < kResidentQuads; ++u) {
        const int64_t q = tid + kResidentThreads * u;
        v[u] = 4 * q < count ? x4[q] : float4v{};
        s += (static_cast<double>(v[u][0]) + static_cast<double>(v[u][1])) +
             (static_cast<double>(v[u][2]) + static_cast<double>(v[u][3]));
    }
    const double n = static_cast<double>(count);
    const float mean = static_cast<float>(block_sum_wide(s, lds_sums) / n);
    double t = 0.0;
#pragma unroll
    for (int u = 0; u < kResidentQuads; ++u) {
        if (4 * (tid + kResidentThreads * u) >= count) continue;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float d = v[u][k] - mean;
            t += static_cast<double>(__fmul_rn(d, d));
        }
    }
    const float variance = static_cast<float>(block_sum_wide(t, lds_sums) / n);
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(variance + a.eps));
    float4v *y4 = reinterpret_cast<float4v *>(a.y + i3 * a.ynb3 + c0 * a.ynb2);
#pragma unroll
    for (int u = 0; u < kResidentQuads; ++u) {
        const int64_t q = tid + kResidentThreads * u;
        if (4 * q >= count) continue;
        const int64_t e = 4 * q;
        const uint32_t c = static_cast<uint32_t>(e) / static_cast<uint32_t>(plane);
        const int64_t p = e - static_cast<int64_t>(c) * plane;
        float w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = __fmul_rn(v[u][k] - mean, scale);
        apply_chain_block(a.chain, w, [&](int st_i, int k) {
            const DevStep &st = a.chain.steps[st_i];
            const int64_t pk = p + k;
            const uint32_t r = static_cast<uint32_t>(pk) / static_cast<uint32_t>(a.ne0);
            return (pk - static_cast<int64_t>(r) * a.ne0) * st.nb[0] + static_cast<int64_t>(r) * st.nb[1] +
                   (c0 + c) * st.nb[2] + i3 * st.nb[3];
        });
        y4[q] = float4v{w[0], w[1], w[2], w[3]};
    }
}

// NORM with the row in registers: one wave per row of ne0 <= 64 E, E numbers
// a lane (lane + 64 u), x read once; the same statistics as norm_kernel.
template <int E>
__global__ __launch_bounds__(kThreads) void norm_resident_kernel(NormArgs a) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const int lane = threadIdx.x & 63;
    const int64_t i1 = row % a.ne1;
    const int64_t i2 = (row / a.ne1) % a.ne2;
    const int64_t i3 = row / (a.ne1 * a.ne2);
    const float *x = a.x + i1 * a.xnb1 + i2 * a.xnb2 + i3 * a.xnb3;
    float *y = a.y + i1 * a.ynb1 + i2 * a.ynb2 + i3 * a.ynb3;
    const auto at = [&](int u) -> int64_t {
        const int64_t j = lane + 64 * u;
        return j < a.ne0 ? j : a.ne0 - 1;
    };
    float v[E];
#pragma unroll
    for (int u = 0; u < E; ++u) v[u] = x[at(u)];
    double s = 0.0;
#pragma unroll
    for (int u = 0; u < E; ++u)
        if (lane + 64 * u < a.ne0) s += static_cast<double>(v[u]);
    const float mean = static_cast<float>(wave_sum(s) / static_cast<double>(a.ne0));
    double q = 0.0;
#pragma unroll
    for (int u = 0; u < E; ++u) {
        if (lane + 64 * u >= a.ne0) continue;
        const float d = v[u] - mean;
        q += static_cast<double>(__fmul_rn(d, d));
    }
    const float variance = static_cast<float>(wave_sum(q) / static_cast<double>(a.ne0));
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(variance + a.eps));
#pragma unroll
    for (int u = 0; u < E; ++u) v[u] = __fmul_rn(v[u] - mean, scale);
    apply_chain_block(a.chain, v, [&](int s, int u) {
        const DevStep &st = a.chain.steps[s];
        return at(u) * st.nb[0] + i1 * st.nb[1] + i2 * st.nb[2] + i3 * st.nb[3];
    });
#pragma unroll
    for (int u = 0; u < E; ++u) {
        if (lane + 64 * u < a.ne0) y[lane + 64 * u] = v[u];
    }
}

// The sum of v over each group of L lanes (L a power of two up to 64).
template <int L>
__device__ __forceinline__ double group_sum(double v) {
#pragma unroll
    for (int off = L / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// NORM of rows of ne0 <= 4 L Q, a multiple of 4, rows 16-byte aligned: L
// lanes per row (64, a wave; or 16, four rows a wave, for short rows, whose
// lanes would idle and whose reductions would weigh on a wave to each), Q
// float4 a lane (lane + L u), x read once; the same statistics as
// norm_kernel (sums in double, whose order moves no float result).  A chain
// step whose operand runs along the row with stride 1 and 16-byte aligned
// rows loads it a float4 at a time.  A row's L lanes return together, so no
// reduction reads a lane that has left.
template <int Q, int L>
__global__ __launch_bounds__(kThreads) void norm_rows4_kernel(NormArgs a) {
    const int64_t row =
        (static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6)) * (64 / L) + ((threadIdx.x & 63) / L);
    if (row >= a.rows) return;
    const int lane = threadIdx.x & (L - 1);
    const int64_t i1 = row % a.ne1;
    const int64_t i2 = (row / a.ne1) % a.ne2;
    const int64_t i3 = row / (a.ne1 * a.ne2);
    const float4v *x = reinterpret_cast<const float4v *>(a.x + i1 * a.xnb1 + i2 * a.xnb2 + i3 * a.xnb3);
    float4v *y = reinterpret_cast<float4v *>(a.y + i1 * a.ynb1 + i2 * a.ynb2 + i3 * a.ynb3);
    const int n4 = static_cast<int>(a.ne0 / 4);
    float v[Q][4];
#pragma unroll
    for (int u = 0; u < Q; ++u) {
        const int j = lane + L * u;
        const float4v q4 = x[j < n4 ? j : n4 - 1];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[u][k] = q4[k];
    }
    // Step st_i's operand where it lies along the row (the first two steps'
    // loaded with x's, before the statistics wait for it).
    const auto operand = [&](int st_i, float (&o)[Q][4]) {
        const DevStep &st = a.chain.steps[st_i];
        const float *base = st.operand + i1 * st.nb[1] + i2 * st.nb[2] + i3 * st.nb[3];
        const bool vec = st.nb[0] == 1 && (reinterpret_cast<uintptr_t>(base) & 15) == 0;
#pragma unroll
        for (int u = 0; u < Q; ++u) {
            const int j = lane + L * u;
            const int64_t e = 4 * static_cast<int64_t>(j < n4 ? j : n4 - 1);
            if (vec) {
                const float4v o4 = *reinterpret_cast<const float4v *>(base + e);
#pragma unroll
                for (int k = 0; k < 4; ++k) o[u][k] = o4[k];
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) o[u][k] = base[(e + k) * st.nb[0]];
            }
        }
    };
    constexpr int kEarly = 2;
    float early[kEarly][Q][4];
#pragma unroll
    for (int st_i = 0; st_i < kEarly; ++st_i)
        if (st_i < a.chain.count && a.chain.steps[st_i].kind != 2) operand(st_i, early[st_i]);
    double s = 0.0;
#pragma unroll
    for (int u = 0; u < Q; ++u)
        if (lane + L * u < n4)
#pragma unroll
            for (int k = 0; k < 4; ++k) s += static_cast<double>(v[u][k]);
    const float mean = static_cast<float>(group_sum<L>(s) / static_cast<double>(a.ne0));
    double q = 0.0;
#pragma unroll
    for (int u = 0; u < Q; ++u) {
        if (lane + L * u >= n4) continue;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float d = v[u][k] - mean;
            q += static_cast<double>(__fmul_rn(d, d));
        }
    }
    const float variance = static_cast<float>(group_sum<L>(q) / static_cast<double>(a.ne0));
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(variance + a.eps));
#pragma unroll
    for (int u = 0; u < Q; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k) v[u][k] = __fmul_rn(v[u][k] - mean, scale);
#pragma unroll 1
    for (int st_i = 0; st_i < a.chain.count; ++st_i) {
        const DevStep &st = a.chain.steps[st_i];
        if (st.kind == 2) {
#pragma unroll
            for (int u = 0; u < Q; ++u)
#pragma unroll
                for (int k = 0; k < 4; ++k) v[u][k] = silu(v[u][k]);
            continue;
        }
        float o[Q][4];
        if (st_i == 0) {
#pragma unroll
            for (int u = 0; u < Q; ++u)
#pragma unroll
                for (int k = 0; k < 4; ++k) o[u][k] = early[0][u][k];
        } else if (st_i == 1) {
#pragma unroll
            for (int u = 0; u < Q; ++u)
#pragma unroll
                for (int k = 0; k < 4; ++k) o[u][k] = early[1][u][k];
        } else {
            operand(st_i, o);
        }
#pragma unroll
        for (int u = 0; u < Q; ++u)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                v[u][k] = st.kind == 0 ? __fadd_rn(v[u][k], o[u][k]) : __fmul_rn(v[u][k], o[u][k]);
    }
#pragma unroll
    for (int u = 0; u < Q; ++u) {
        const int j = lane + L * u;
        if (j < n4) y[j] = float4v{v[u][0], v[u][1], v[u][2], v[u][3]};
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

GroupNormShape group_norm_shape(int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, int64_t groups) {
    GroupNormShape g{};
    const int64_t per_group = ceil_div(ne2, groups);
    const int64_t count = per_group * ne0 * ne1;
    const int64_t items = ne3 * groups;
    // About 1024 blocks in all, each of 4096 numbers or more, a slice a
    // multiple of 4 numbers so that every slice's quads start aligned.
    const int64_t want = ceil_div(1024, items);
    g.chunk = round_up(ceil_div(count, want), 4);
    if (g.chunk < 4096) g.chunk = round_up(count < 4096 ? count : 4096, 4);
    if (g.chunk < 4) g.chunk = 4;
    g.slices = ceil_div(count, g.chunk);
    if (g.slices < 1) g.slices = 1;
    g.work = static_cast<size_t>(2 * items * g.slices) * sizeof(double);
    return g;
}

hipError_t launch_group_norm(const GroupNormArgs &a, hipStream_t stream) {
    const int64_t plane = a.ne0 * a.ne1;
    const bool resident = a.per_group * plane <= kResident && plane % 4 == 0 && a.xnb2 == plane &&
                          a.ynb2 == plane && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
                          (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 && a.xnb3 % 4 == 0 && a.ynb3 % 4 == 0;
    if (resident) {
        KernelScope scope("group_norm", stream);
        SDHIP_LAUNCH(group_norm_resident_kernel, dim3(static_cast<uint32_t>(a.ne3 * a.groups)),
                     dim3(kResidentThreads), 0, stream, a);
        return hipGetLastError();
    }
    const dim3 grid(static_cast<uint32_t>(a.ne3 * a.groups * a.slices));
    {
        KernelScope scope("group_norm.sums", stream);
        SDHIP_LAUNCH(group_sums_kernel<0>, grid, dim3(kThreads), 0, stream, a);
    }
    {
        KernelScope scope("group_norm.squares", stream);
        SDHIP_LAUNCH(group_sums_kernel<1>, grid, dim3(kThreads), 0, stream, a);
    }
    KernelScope scope("group_norm.apply", stream);
    SDHIP_LAUNCH(group_apply_kernel, grid, dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

// ------------------------------------------------------------------ the entry point that allocates nothing

// The partial sums of sdhip_group_norm_static: a file-scope array of the
// device code, one copy on each GPU the library runs on, held until the
// process ends.  Host code never names it as a device address: its address
// on each device comes from hipGetSymbolAddress, once per device, with that
// device current (static_scratch below), and only that address goes to the
// kernels.  The sums are written before they are read, so nothing needs
// clearing; every call on one GPU shares it, so calls that overlap on one
// GPU race.
static __device__ __align__(256) double scratch[kStaticScratchBytes / sizeof(double)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
double *g_scratch[kMaxDevices] = {};

}  // namespace

sdhip_status static_scratch(int device, double *&ptr) {
    ptr = nullptr;
    if (device < 0 || device >= kMaxDevices) {
        return fail(SDHIP_ERROR, "device %d: at most %d devices hold the static scratch", device, kMaxDevices);
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch[device] == nullptr) {
        int current = -1;
        if (hipGetDevice(&current) != hipSuccess || current != device) {
            return fail(SDHIP_ERROR, "static scratch of device %d looked up with device %d current", device, current);
        }
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            return fail(SDHIP_ERROR, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
        }
        g_scratch[device] = static_cast<double *>(p);
    }
    ptr = g_scratch[device];
    return SDHIP_OK;
}

hipError_t launch_norm(const NormArgs &a, hipStream_t stream) {
    KernelScope scope("norm", stream);
    const dim3 grid(static_cast<uint32_t>(ceil_div(a.rows, kThreads / 64)));
    const bool rows4 = a.ne0 >= 4 && a.ne0 % 4 == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
                       (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 && a.xnb1 % 4 == 0 && a.xnb2 % 4 == 0 &&
                       a.xnb3 % 4 == 0 && a.ynb1 % 4 == 0 && a.ynb2 % 4 == 0 && a.ynb3 % 4 == 0;
    const int64_t quads = ceil_div(a.ne0, 256);
    // Rows of up to 320 numbers: 16 lanes a row, four rows a wave (8192 rows
    // of 320: 8.7 -> 6.7 us; rows of 640 by 32 lanes, two a wave, measured
    // slower than a wave each: 5.5 -> 5.8 us).
    const dim3 grid16(static_cast<uint32_t>(ceil_div(a.rows, 4 * (kThreads / 64))));
    if (rows4 && a.ne0 <= 128) {
        SDHIP_LAUNCH((norm_rows4_kernel<2, 16>), grid16, dim3(kThreads), 0, stream, a);
    } else if (rows4 && a.ne0 <= 320) {
        SDHIP_LAUNCH((norm_rows4_kernel<5, 16>), grid16, dim3(kThreads), 0, stream, a);
    } else if (rows4 && quads <= 2) {
        SDHIP_LAUNCH((norm_rows4_kernel<2, 64>), grid, dim3(kThreads), 0, stream, a);
    } else if (rows4 && quads <= 3) {
        SDHIP_LAUNCH((norm_rows4_kernel<3, 64>), grid, dim3(kThreads), 0, stream, a);
    } else if (rows4 && quads <= 5) {
        SDHIP_LAUNCH((norm_rows4_kernel<5, 64>), grid, dim3(kThreads), 0, stream, a);
    } else if (rows4 && quads <= 8) {
        SDHIP_LAUNCH((norm_rows4_kernel<8, 64>), grid, dim3(kThreads), 0, stream, a);
    } else if (a.ne0 <= 64 * 8) {
        SDHIP_LAUNCH(norm_resident_kernel<8>, grid, dim3(kThreads), 0, stream, a);
    } else if (a.ne0 <= 64 * 16) {
        SDHIP_LAUNCH(norm_resident_kernel<16>, grid, dim3(kThreads), 0, stream, a);
    } else if (a.ne0 <= 64 * 32) {
        SDHIP_LAUNCH(norm_resident_kernel<32>, grid, dim3(kThreads), 0, stream, a);
    } else {
        SDHIP_LAUNCH(norm_kernel, grid, dim3(kThreads), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace sdhip
