// FLASH_ATTN_EXT without a mask (attention.cc) on gfx950's single-precision
// MFMA, v_mfma_f32_16x16x4_f32, so that the products are those of single
// precision, as the reference's.
//
// A workgroup of 4 waves takes 64 queries of one head, 16 a wave, and goes
// through the keys in blocks of 32, which all four waves read from LDS.  A
// wave computes the scores transposed, keys by queries (S^T = K Q^T), so
// that its lane l holds the scores of query l % 16 for keys 4 (l / 16) + r of
// each tile of 16 keys: those are exactly the operand B of the product by the
// values, O^T = V^T P^T, when the MFMA's k index 4 (l / 16) + r is taken
// four times, r = 0..3.  The probabilities never leave the registers.
//
// The softmax is the online one of flash attention: per block of keys the
// running maximum of each query (a max over the lane's scores and across the
// four lanes of a query), the exponentials exp(s - max) by Cephes' method as
// the reference's exponential() computes them (scalar_math.h:34-51), the
// running output and sum rescaled by exp(old max - new max).  The reference's
// softmax takes two passes instead (attention.cc:9-27); the rescaling adds a
// rounding of no consequence at single precision.  The sum of the
// exponentials is kept in double precision, as the reference keeps it
// (attention.cc:287-301), and the output is multiplied at the end by the
// reciprocal of the sum rounded to single precision (attention.cc:1055-1062).

#include "attention.h"
#include "host.h"
#include "profile.h"

namespace sdhip {

namespace {

constexpr int kQueries = 64;  // a workgroup's queries, 16 a wave
constexpr int kKeys = 32;     // keys of a block

template <bool HALF>
__device__ __forceinline__ float load_kv(const void *p, int64_t at) {
    if (HALF) return static_cast<float>(static_cast<const _Float16 *>(p)[at]);
    return static_cast<const float *>(p)[at];
}

// NDV tiles of 16 of the values' dimensions.
template <int NDV, bool KHALF, bool VHALF>
__global__ __launch_bounds__(256) void attention_kernel(AttentionArgs a) {
    extern __shared__ float lds[];
    float *qs = lds;                          // [64][ldq]
    float *ks = qs + kQueries * a.ldq;        // [32][ldk]
    float *vs = ks + kKeys * a.ldk;           // [32][ldv]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 15;  // the query of the lane, or the row of an operand
    const int lg = lane >> 4;  // the lane's group of four

    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint32_t qb = b % static_cast<uint32_t>(a.qblocks);
    const uint32_t bh = b / static_cast<uint32_t>(a.qblocks);
    const int64_t hi = bh % a.h;
    const int64_t bi = bh / a.h;
    const int64_t kh = hi / (a.h / a.hk);
    const int64_t q0 = static_cast<int64_t>(qb) * kQueries;

    // The block's queries into LDS, zeros past d and past lq.
    for (int idx = tid; idx < kQueries * a.dp; idx += 256) {
        const int qi = idx / a.dp, e = idx - qi * a.dp;
        const int64_t i = q0 + qi;
        float x = 0.0f;
        if (e < a.d && i < a.lq) x = a.q[bi * a.qnb3 + hi * a.qnb2 + i * a.qnb1 + e];
        qs[qi * a.ldq + e] = x;
    }

    const int64_t kbase = bi * a.knb3 + kh * a.knb2;
    const int64_t vbase = bi * a.vnb3 + kh * a.vnb2;
    float4v o[NDV];
#pragma unroll
    for (int t = 0; t < NDV; ++t) o[t] = float4v{};
    float m = -INFINITY;
    double l = 0.0;
    const float *qw = qs + (wave * 16 + lr) * a.ldq + lg;

    for (int64_t k0 = 0; k0 < a.lk; k0 += kKeys) {
        __syncthreads();  // the last block's keys and values are read
        for (int idx = tid; idx < kKeys * a.dp; idx += 256) {
            const int j = idx / a.dp, e = idx - j * a.dp;
            const int64_t key = k0 + j;
            ks[j * a.ldk + e] = (e < a.d && key < a.lk) ? load_kv<KHALF>(a.k, kbase + key * a.knb1 + e) : 0.0f;
        }
        for (int idx = tid; idx < kKeys * 16 * NDV; idx += 256) {
            const int j = idx / (16 * NDV), e = idx - j * (16 * NDV);
            const int64_t key = k0 + j;
            vs[j * a.ldv + e] = (e < a.dv && key < a.lk) ? load_kv<VHALF>(a.v, vbase + key * a.vnb1 + e) : 0.0f;
        }
        __syncthreads();

        // S^T = K Q^T for two tiles of 16 keys: the lane's scores of its
        // query lr, keys 16 t + 4 lg + r.
        float4v s[2] = {float4v{}, float4v{}};
        for (int e = 0; e < a.dp; e += 4) {
            const float qv = qw[e];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const float kv = ks[(16 * t + lr) * a.ldk + e + lg];
                s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv, qv, s[t], 0, 0, 0);
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t key = k0 + 16 * t + 4 * lg + r;
                const float x = key < a.lk ? s[t][r] * a.scale : -INFINITY;
                s[t][r] = x;
                mx = fmaxf(mx, x);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(m, mx);
        const float alpha = m == -INFINITY ? 0.0f : cephes_exp(m - mnew);
        m = mnew;
        double part = 0.0;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = s[t][r] == -INFINITY ? 0.0f : cephes_exp(s[t][r] - mnew);
                s[t][r] = p;
                part += static_cast<double>(p);
            }
        l = l * static_cast<double>(alpha) + part;
#pragma unroll
        for (int t = 0; t < NDV; ++t) o[t] *= alpha;

        // O^T += V^T P^T: k index 4 lg + r of each tile of 16 keys.
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float *vrow = vs + (16 * t + 4 * lg + r) * a.ldv + lr;
#pragma unroll
                for (int c = 0; c < NDV; ++c) {
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[16 * c], s[t][r], o[c], 0, 0, 0);
                }
            }
    }

    // The sum of the query's exponentials over its four lanes, and the
    // output: lane holds O^T[16 c + 4 lg + r][query lr].
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const float reciprocal = static_cast<float>(1.0 / l);
    const int64_t i = q0 + wave * 16 + lr;
    if (i >= a.lq) return;
    float *out = a.y + bi * a.ynb3 + i * a.ynb2 + hi * a.ynb1;
#pragma unroll
    for (int c = 0; c < NDV; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int e = 16 * c + 4 * lg + r;
            if (e < a.dv) out[e] = o[c][r] * reciprocal;
        }
}

template <int NDV>
hipError_t launch_ndv(AttentionArgs a, hipStream_t stream) {
    a.ldv = 16 * NDV + 4;
    const size_t lds = sizeof(float) * (kQueries * a.ldq + kKeys * a.ldk + kKeys * a.ldv);
    dim3 grid(static_cast<uint32_t>(a.qblocks * a.h * a.b)), block(256);
    if (a.khalf && a.vhalf) {
        hipLaunchKernelGGL((attention_kernel<NDV, true, true>), grid, block, lds, stream, a);
    } else if (a.khalf) {
        hipLaunchKernelGGL((attention_kernel<NDV, true, false>), grid, block, lds, stream, a);
    } else if (a.vhalf) {
        hipLaunchKernelGGL((attention_kernel<NDV, false, true>), grid, block, lds, stream, a);
    } else {
        hipLaunchKernelGGL((attention_kernel<NDV, false, false>), grid, block, lds, stream, a);
    }
    return hipGetLastError();
}

}  // namespace

size_t attention_lds_bytes(int64_t d, int64_t dv) {
    const int64_t dp = round_up(d, 4);
    return sizeof(float) * static_cast<size_t>(kQueries * (dp + 1) + kKeys * (dp + 1) + kKeys * (16 * 16 + 4));
}

hipError_t launch_attention(AttentionArgs a, hipStream_t stream) {
    a.dp = static_cast<int>(round_up(a.d, 4));
    a.ldq = a.dp + 1;
    a.ldk = a.dp + 1;
    const int ndv = static_cast<int>(ceil_div(a.dv, 16));
    a.qblocks = ceil_div(a.lq, kQueries);
    KernelScope scope("attention", stream);
    switch (ndv) {
    case 1: return launch_ndv<1>(a, stream);
    case 2: return launch_ndv<2>(a, stream);
    case 3: return launch_ndv<3>(a, stream);
    case 4: return launch_ndv<4>(a, stream);
    case 5: return launch_ndv<5>(a, stream);
    case 6:
    case 7:
    case 8: return launch_ndv<8>(a, stream);
    case 9:
    case 10: return launch_ndv<10>(a, stream);
    default: return launch_ndv<16>(a, stream);
    }
}

}  // namespace sdhip
