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
// Two forms: a generic one (any head size up to 256, FP16 keys and values,
// any strides), described first, and a fast one for single-precision keys and
// values of the head sizes SD takes, described further down.
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
//
// With bits=16 and half_format=1 (AttentionArgs::bf16) the generic and wide
// forms take every head: they round the queries, keys and values, and the
// exponentials the second product takes, to bfloat16 before their products --
// which are exact in single precision and summed there, the products of
// bfloat16 first parts of the reference's vector units (attention.cc:309-323,
// 466-467).  Each query's largest score is found over all its keys before any
// exponential, so that each is rounded from exp(s - max) of the whole row, as
// the reference's two passes round them; the sum of the exponentials takes
// them unrounded, as the reference's does.

#include <type_traits>

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
        qs[qi * a.ldq + e] = bf16_operand(x, a.bf16);
    }

    const int64_t kbase = bi * a.knb3 + kh * a.knb2;
    const int64_t vbase = bi * a.vnb3 + kh * a.vnb2;
    float4v o[NDV];
#pragma unroll
    for (int t = 0; t < NDV; ++t) o[t] = float4v{};
    float m = -INFINITY;
    double l = 0.0;
    const float *qw = qs + (wave * 16 + lr) * a.ldq + lg;

    // The block of keys from k0 into LDS, zeros past d and past lk.
    const auto stage_keys = [&](int64_t k0) {
        for (int idx = tid; idx < kKeys * a.dp; idx += 256) {
            const int j = idx / a.dp, e = idx - j * a.dp;
            const int64_t key = k0 + j;
            ks[j * a.ldk + e] =
                (e < a.d && key < a.lk) ? bf16_operand(load_kv<KHALF>(a.k, kbase + key * a.knb1 + e), a.bf16) : 0.0f;
        }
    };
    // S^T = K Q^T for two tiles of 16 keys, scaled, -inf past lk: the lane's
    // scores of its query lr, keys 16 t + 4 lg + r; and the largest of the
    // query's over its four lanes.
    const auto block_scores = [&](int64_t k0, float4v(&s)[2]) {
        s[0] = float4v{};
        s[1] = float4v{};
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
        return fmaxf(mx, __shfl_xor(mx, 32, 64));
    };

    // Products in bfloat16: each query's largest score over all the keys
    // first, a pass of the first product alone, so that every exponential is
    // exp(s - max) of the whole row rounded to bfloat16 from that, as the
    // reference's two passes round them (attention.cc:519-545); the running
    // rescaling below then multiplies by exp(0) = 1.
    if (a.bf16) {
        for (int64_t k0 = 0; k0 < a.lk; k0 += kKeys) {
            __syncthreads();
            stage_keys(k0);
            __syncthreads();
            float4v s[2];
            m = fmaxf(m, block_scores(k0, s));
        }
    }

    for (int64_t k0 = 0; k0 < a.lk; k0 += kKeys) {
        __syncthreads();  // the last block's keys and values are read
        stage_keys(k0);
        for (int idx = tid; idx < kKeys * 16 * NDV; idx += 256) {
            const int j = idx / (16 * NDV), e = idx - j * (16 * NDV);
            const int64_t key = k0 + j;
            vs[j * a.ldv + e] =
                (e < a.dv && key < a.lk) ? bf16_operand(load_kv<VHALF>(a.v, vbase + key * a.vnb1 + e), a.bf16) : 0.0f;
        }
        __syncthreads();

        float4v s[2];
        const float mx = block_scores(k0, s);
        const float mnew = fmaxf(m, mx);
        const float alpha = m == -INFINITY ? 0.0f : cephes_exp(m - mnew);
        m = mnew;
        double part = 0.0;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = s[t][r] == -INFINITY ? 0.0f : cephes_exp(s[t][r] - mnew);
                s[t][r] = bf16_operand(p, a.bf16);  // the sum takes p as it is
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

// ------------------------------------------------------------------ wide heads
//
// Heads of more than 256 dimensions (the VAE's, 512): the generic form's
// products, softmax and sums, with the queries and keys staged 128 dimensions
// at a time -- the scores of a block of 32 keys summed over the chunks -- so
// that LDS holds 64 queries and 32 keys of one chunk and the block's values
// of NDV tiles of 16 dimensions (dv <= 16 NDV).
constexpr int kWideChunk = 128;
constexpr int kWideLd = kWideChunk + 1;

// Whether the wide form takes the head: more than 256 dimensions of the
// queries and keys or of the values.
inline bool wide_form(const AttentionArgs &a) { return a.d > 256 || a.dv > 256; }

// The splits of the keys: enough for about 512 blocks with the query blocks
// of 64, of 256 keys or more each (a multiple of 32).
struct WideSplits {
    int64_t splits, key_len;
};

inline WideSplits wide_splits(const AttentionArgs &a) {
    const int64_t blocks = ceil_div(a.lq, kQueries) * a.h * a.b;
    int64_t sp = ceil_div(512, blocks);
    // Products in bfloat16 take all the keys in one split: each exponential
    // is rounded from exp(s - max) of the whole row.
    const int64_t most = a.lk / 256 > 1 && !a.bf16 ? a.lk / 256 : 1;
    sp = sp < most ? sp : most;
    WideSplits w;
    w.key_len = round_up(ceil_div(a.lk, sp), kKeys);
    w.splits = ceil_div(a.lk, w.key_len);
    return w;
}

// With `part`, a block takes the keys of one split of key_len (a multiple
// of 32) and writes its queries' running maximum, sum and unnormalised output
// there (WidePartial) for attention_combine_kernel.
struct WidePartial {
    float *m;    // [b h][split][lq]
    double *l;   // [b h][split][lq]
    float *o;    // [b h][split][lq][dv]
};

__host__ __device__ inline WidePartial wide_partial(void *work, const AttentionArgs &a, int64_t splits) {
    const int64_t n = a.b * a.h * splits * a.lq;
    char *p = static_cast<char *>(work);
    WidePartial w;
    w.l = reinterpret_cast<double *>(p);
    w.m = reinterpret_cast<float *>(p + n * 8);
    w.o = reinterpret_cast<float *>(p + n * 12);
    return w;
}

template <int NDV, bool KHALF, bool VHALF>
__global__ __launch_bounds__(256) void attention_wide_kernel(AttentionArgs a, int64_t splits, int64_t key_len,
                                                             WidePartial part) {
    extern __shared__ float lds[];
    float *qs = lds;                       // [64][kWideLd]
    float *ks = qs + kQueries * kWideLd;   // [32][kWideLd]
    float *vs = ks + kKeys * kWideLd;      // [32][ldv]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 15;
    const int lg = lane >> 4;

    // Neighbouring blocks share a split's keys and values.  Values of more
    // than 16 NDV dimensions go in slices of 16 NDV, a block each, every
    // slice with the same scores, maxima and sums.
    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint32_t qb = b % static_cast<uint32_t>(a.qblocks);
    const uint32_t rest = b / static_cast<uint32_t>(a.qblocks);
    const int64_t sp = rest % splits;
    const uint32_t rest2 = static_cast<uint32_t>(rest / splits);
    const uint32_t heads = static_cast<uint32_t>(a.b * a.h);
    const uint32_t slice = rest2 / heads;
    const uint32_t bh = rest2 - slice * heads;
    const int64_t v0 = static_cast<int64_t>(slice) * 16 * NDV;  // the slice's first dimension
    const int64_t dvs = a.dv - v0;                               // the values' dimensions from it
    const int64_t k_begin = sp * key_len;
    const int64_t k_end = k_begin + key_len < a.lk ? k_begin + key_len : a.lk;
    const int64_t hi = bh % a.h;
    const int64_t bi = bh / a.h;
    const int64_t kh = hi / (a.h / a.hk);
    const int64_t q0 = static_cast<int64_t>(qb) * kQueries;
    const int64_t qbase = bi * a.qnb3 + hi * a.qnb2;
    const int64_t kbase = bi * a.knb3 + kh * a.knb2;
    const int64_t vbase = bi * a.vnb3 + kh * a.vnb2 + v0;

    float4v o[NDV];
#pragma unroll
    for (int t = 0; t < NDV; ++t) o[t] = float4v{};
    float m = -INFINITY;
    double l = 0.0;
    const float *qw = qs + (wave * 16 + lr) * kWideLd + lg;

    // S^T = K Q^T for two tiles of 16 keys, over the chunks of the
    // dimensions, scaled, -inf past the split's keys: the lane's scores of its
    // query lr, keys 16 t + 4 lg + r; and the largest of the query's over its
    // four lanes.
    const auto block_scores = [&](int64_t k0, float4v(&s)[2]) {
        s[0] = float4v{};
        s[1] = float4v{};
        for (int e0 = 0; e0 < a.dp; e0 += kWideChunk) {
            const int dc = a.dp - e0 < kWideChunk ? static_cast<int>(a.dp - e0) : kWideChunk;
            __syncthreads();  // the last chunk's queries and keys are read
            for (int idx = tid; idx < kQueries * dc; idx += 256) {
                const int qi = idx / dc, e = idx - qi * dc;
                const int64_t i = q0 + qi;
                float x = 0.0f;
                if (e0 + e < a.d && i < a.lq) x = a.q[qbase + i * a.qnb1 + e0 + e];
                qs[qi * kWideLd + e] = bf16_operand(x, a.bf16);
            }
            for (int idx = tid; idx < kKeys * dc; idx += 256) {
                const int j = idx / dc, e = idx - j * dc;
                const int64_t key = k0 + j;
                ks[j * kWideLd + e] = (e0 + e < a.d && key < k_end)
                                          ? bf16_operand(load_kv<KHALF>(a.k, kbase + key * a.knb1 + e0 + e), a.bf16)
                                          : 0.0f;
            }
            __syncthreads();
            for (int e = 0; e < dc; e += 4) {
                const float qv = qw[e];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const float kv = ks[(16 * t + lr) * kWideLd + e + lg];
                    s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv, qv, s[t], 0, 0, 0);
                }
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t key = k0 + 16 * t + 4 * lg + r;
                const float x = key < k_end ? s[t][r] * a.scale : -INFINITY;
                s[t][r] = x;
                mx = fmaxf(mx, x);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        return fmaxf(mx, __shfl_xor(mx, 32, 64));
    };

    // Products in bfloat16 (one split of all the keys): each query's largest
    // score first, as the generic form takes it.
    if (a.bf16) {
        for (int64_t k0 = k_begin; k0 < k_end; k0 += kKeys) {
            float4v s[2];
            m = fmaxf(m, block_scores(k0, s));
        }
    }

    for (int64_t k0 = k_begin; k0 < k_end; k0 += kKeys) {
        float4v s[2];
        const float mx = block_scores(k0, s);
        __syncthreads();  // the last block's values are read
        for (int idx = tid; idx < kKeys * 16 * NDV; idx += 256) {
            const int j = idx / (16 * NDV), e = idx - j * (16 * NDV);
            const int64_t key = k0 + j;
            vs[j * a.ldv + e] =
                (e < dvs && key < k_end) ? bf16_operand(load_kv<VHALF>(a.v, vbase + key * a.vnb1 + e), a.bf16) : 0.0f;
        }
        __syncthreads();

        const float mnew = fmaxf(m, mx);
        const float alpha = m == -INFINITY ? 0.0f : cephes_exp(m - mnew);
        m = mnew;
        double part = 0.0;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = s[t][r] == -INFINITY ? 0.0f : cephes_exp(s[t][r] - mnew);
                s[t][r] = bf16_operand(p, a.bf16);  // the sum takes p as it is
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

    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int64_t i = q0 + wave * 16 + lr;
    if (i >= a.lq) return;
    if (part.o != nullptr) {
        const int64_t at = (static_cast<int64_t>(bh) * splits + sp) * a.lq + i;
        if (lg == 0 && slice == 0) {
            part.m[at] = m;
            part.l[at] = l;
        }
        float *po = part.o + at * a.dv + v0;
#pragma unroll
        for (int c = 0; c < NDV; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int e = 16 * c + 4 * lg + r;
                if (e < dvs) po[e] = o[c][r];
            }
        return;
    }
    const float reciprocal = static_cast<float>(1.0 / l);
    float *out = a.y + bi * a.ynb3 + i * a.ynb2 + hi * a.ynb1 + v0;
#pragma unroll
    for (int c = 0; c < NDV; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int e = 16 * c + 4 * lg + r;
            if (e < dvs) out[e] = o[c][r] * reciprocal;
        }
}

// Heads of up to 512 dimensions (more than 384) with single-precision keys
// and values (the VAE's middle block, 512): the wide form's products, softmax and sums, in the same
// order -- bit for bit its output -- with each wave's 16 queries held in
// registers for the whole split (lane (lr, lg) holds dimensions 4 j + lg of
// query lr: operand B of step j) and a block's 32 keys and their values
// staged whole in LDS, rows of DP + 4 and 16 NDV + 4 floats (64 banks for
// both reads), float4 copies: two barriers a block of keys, where the wide
// form restages its queries with every chunk of every block.
template <int DP, int NDV>
__global__ __launch_bounds__(256, 1) void attention_wide2_kernel(AttentionArgs a, int64_t splits, int64_t key_len,
                                                                  WidePartial part) {
    constexpr int kLdk = DP + 4, kLdv = 16 * NDV + 4;
    constexpr int NQ = DP / 4;
    extern __shared__ float lds[];
    float *ks = lds;                // [32][kLdk]
    float *vs = ks + kKeys * kLdk;  // [32][kLdv]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 15;
    const int lg = lane >> 4;

    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint32_t qb = b % static_cast<uint32_t>(a.qblocks);
    const uint32_t rest = b / static_cast<uint32_t>(a.qblocks);
    const int64_t sp = rest % splits;
    const uint32_t bh = static_cast<uint32_t>(rest / splits);
    const int64_t k_begin = sp * key_len;
    const int64_t k_end = k_begin + key_len < a.lk ? k_begin + key_len : a.lk;
    const int64_t hi = bh % a.h;
    const int64_t bi = bh / a.h;
    const int64_t kh = hi / (a.h / a.hk);
    const int64_t q0 = static_cast<int64_t>(qb) * kQueries;
    const float *kg = static_cast<const float *>(a.k) + bi * a.knb3 + kh * a.knb2;
    const float *vg = static_cast<const float *>(a.v) + bi * a.vnb3 + kh * a.vnb2;

    float qr[NQ];
    {
        const int64_t i = q0 + wave * 16 + lr;
        const float *qp = a.q + bi * a.qnb3 + hi * a.qnb2 + (i < a.lq ? i : 0) * a.qnb1;
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
            const int e = 4 * j + lg;
            qr[j] = (e < a.d && i < a.lq) ? qp[e] : 0.0f;
        }
    }
    float4v o[NDV];
#pragma unroll
    for (int t = 0; t < NDV; ++t) o[t] = float4v{};
    float m = -INFINITY;
    double l = 0.0;

    for (int64_t k0 = k_begin; k0 < k_end; k0 += kKeys) {
        __syncthreads();  // the last block's keys and values are read
        // A row's float4s past d (dv) and the rows past k_end are zeros.
        for (int idx = tid; idx < kKeys * (DP / 4); idx += 256) {
            const int j = idx / (DP / 4), e = 4 * (idx - j * (DP / 4));
            const int64_t key = k0 + j;
            float4v x = float4v{};
            if (e < a.d && key < k_end) x = *reinterpret_cast<const float4v *>(kg + key * a.knb1 + e);
            *reinterpret_cast<float4v *>(ks + j * kLdk + e) = x;
        }
        for (int idx = tid; idx < kKeys * 4 * NDV; idx += 256) {
            const int j = idx / (4 * NDV), e = 4 * (idx - j * (4 * NDV));
            const int64_t key = k0 + j;
            float4v x = float4v{};
            if (e < a.dv && key < k_end) x = *reinterpret_cast<const float4v *>(vg + key * a.vnb1 + e);
            *reinterpret_cast<float4v *>(vs + j * kLdv + e) = x;
        }
        __syncthreads();

        // S^T = K Q^T for two tiles of 16 keys: the lane's scores of its
        // query lr, keys 16 t + 4 lg + r; dimensions in order, four a step.
        float4v s[2] = {float4v{}, float4v{}};
#pragma unroll
        for (int j = 0; j < NQ; ++j)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const float kv = ks[(16 * t + lr) * kLdk + 4 * j + lg];
                s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv, qr[j], s[t], 0, 0, 0);
            }

        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t key = k0 + 16 * t + 4 * lg + r;
                const float x = key < k_end ? s[t][r] * a.scale : -INFINITY;
                s[t][r] = x;
                mx = fmaxf(mx, x);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(m, mx);
        const float alpha = m == -INFINITY ? 0.0f : cephes_exp(m - mnew);
        m = mnew;
        double psum = 0.0;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = s[t][r] == -INFINITY ? 0.0f : cephes_exp(s[t][r] - mnew);
                s[t][r] = p;
                psum += static_cast<double>(p);
            }
        l = l * static_cast<double>(alpha) + psum;
#pragma unroll
        for (int t = 0; t < NDV; ++t) o[t] *= alpha;

        // O^T += V^T P^T: k index 4 lg + r of each tile of 16 keys.
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float *vrow = vs + (16 * t + 4 * lg + r) * kLdv + lr;
#pragma unroll
                for (int c = 0; c < NDV; ++c) {
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[16 * c], s[t][r], o[c], 0, 0, 0);
                }
            }
    }

    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    const int64_t i = q0 + wave * 16 + lr;
    if (i >= a.lq) return;
    if (part.o != nullptr) {
        const int64_t at = (static_cast<int64_t>(bh) * splits + sp) * a.lq + i;
        if (lg == 0) {
            part.m[at] = m;
            part.l[at] = l;
        }
        float *po = part.o + at * a.dv;
#pragma unroll
        for (int c = 0; c < NDV; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int e = 16 * c + 4 * lg + r;
                if (e < a.dv) po[e] = o[c][r];
            }
        return;
    }
    const float reciprocal = static_cast<float>(1.0 / l);
    float *out = a.y + bi * a.ynb3 + i * a.ynb2 + hi * a.ynb1;
#pragma unroll
    for (int c = 0; c < NDV; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int e = 16 * c + 4 * lg + r;
            if (e < a.dv) out[e] = o[c][r] * reciprocal;
        }
}

// The splits of the keys of a query merged: each split's sum and output
// rescaled by exp(its maximum - the greatest), as the single pass rescales
// its running ones, the sum in double, the output times the reciprocal of
// the sum rounded to single precision.  A wave per query.
__global__ __launch_bounds__(256) void attention_combine_kernel(AttentionArgs a, int64_t splits, WidePartial part) {
    const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);  // (b h) lq + i
    const int lane = threadIdx.x & 63;
    if (item >= a.b * a.h * a.lq) return;
    const int64_t bh = item / a.lq, i = item - bh * a.lq;
    const int64_t hi = bh % a.h, bi = bh / a.h;
    const int64_t first = bh * splits * a.lq + i;  // split 0 of the query
    float mx = -INFINITY;
    for (int64_t sp = 0; sp < splits; ++sp) mx = fmaxf(mx, part.m[first + sp * a.lq]);
    double l = 0.0;
    for (int64_t sp = 0; sp < splits; ++sp) {
        const float ms = part.m[first + sp * a.lq];
        const float w = ms == -INFINITY ? 0.0f : cephes_exp(ms - mx);
        l += part.l[first + sp * a.lq] * static_cast<double>(w);
    }
    const float reciprocal = static_cast<float>(1.0 / l);
    float *out = a.y + bi * a.ynb3 + i * a.ynb2 + hi * a.ynb1;
    for (int64_t e = lane; e < a.dv; e += 64) {
        float acc = 0.0f;
        for (int64_t sp = 0; sp < splits; ++sp) {
            const float ms = part.m[first + sp * a.lq];
            const float w = ms == -INFINITY ? 0.0f : cephes_exp(ms - mx);
            acc = fmaf(part.o[(first + sp * a.lq) * a.dv + e], w, acc);
        }
        out[e] = acc * reciprocal;
    }
}

// ------------------------------------------------------------------ the fast form
//
// Single-precision keys and values, heads of D = d = dv dimensions (a multiple
// of 8), rows 16-byte aligned: the form SD's attention takes.  A workgroup of
// 4 waves takes 4 x 16 QT queries of one head, a wave 16 QT of them (QT tiles
// of 16), and goes through the keys KB at a time.  The products are those of
// the generic form above -- S^T = K Q^T and O^T = V^T P^T on the
// single-precision MFMA, the probabilities never leaving the registers --
// with every operand read from LDS feeding QT MFMAs, the queries held in
// registers, and the keys and values of the next KB loaded from HBM as float4
// while the MFMAs work on the current ones, into the other of two LDS buffers:
// one barrier per KB keys.  LDS rows are D + 4 floats for the keys (D / 4 + 1
// odd: the 64 lanes of an S operand read hit 64 banks) and 16 NDV + 4 for the
// values (4 mod 16: those of a V operand read hit 64 banks too).

template <int D, int QT, int KB>
struct Fast {
    static constexpr int kSteps = D / 4;            // k-steps of S, 4 dimensions each
    static constexpr int kNdv = (D + 15) / 16;       // tiles of 16 of the output's dimensions
    static constexpr int kLdk = D + 4;
    static constexpr int kLdv = 16 * kNdv + 4;
    static constexpr int kQueries = 4 * 16 * QT;     // a workgroup's
    static constexpr int kRow4 = D / 4;              // float4 of a row
    static constexpr int kF4 = KB * kRow4;           // float4 of KB rows
    static constexpr int kPer = (kF4 + 255) / 256;   // of them a thread loads
    static constexpr int kBuffer = KB * (kLdk + kLdv);  // floats of one LDS buffer
    static_assert(D % 8 == 0 && KB % 16 == 0, "shape");
};

// The KB keys and values from k0 into registers, float4 at a time; rows past
// lk read the last row (their scores are masked).
template <class F>
__device__ __forceinline__ void fast_load(float4v (&kr)[F::kPer], float4v (&vr)[F::kPer], const float *kg,
                                          const float *vg, int64_t k0, int64_t lk, int64_t knb1, int64_t vnb1,
                                          int tid) {
    // Every register is loaded (threads past the tile's last float4 load its
    // last one again and do not store it): a load under a condition would
    // keep the registers in scratch memory.
#pragma unroll
    for (int i = 0; i < F::kPer; ++i) {
        int idx = tid + 256 * i;
        idx = idx < F::kF4 ? idx : F::kF4 - 1;
        const int j = idx / F::kRow4;
        const int c4 = idx - j * F::kRow4;
        int64_t key = k0 + j;
        key = key < lk ? key : lk - 1;
        kr[i] = *reinterpret_cast<const float4v *>(kg + key * knb1 + 4 * c4);
        vr[i] = *reinterpret_cast<const float4v *>(vg + key * vnb1 + 4 * c4);
    }
}

// The registers into an LDS buffer: keys [KB][kLdk], then values [KB][kLdv].
template <class F, int KB>
__device__ __forceinline__ void fast_store(const float4v (&kr)[F::kPer], const float4v (&vr)[F::kPer], float *buf,
                                           int tid) {
#pragma unroll
    for (int i = 0; i < F::kPer; ++i) {
        const int idx = tid + 256 * i;
        if (F::kF4 % 256 == 0 || idx < F::kF4) {
            const int j = idx / F::kRow4;
            const int c4 = idx - j * F::kRow4;
            *reinterpret_cast<float4v *>(buf + j * F::kLdk + 4 * c4) = kr[i];
            *reinterpret_cast<float4v *>(buf + KB * F::kLdk + j * F::kLdv + 4 * c4) = vr[i];
        }
    }
}

// The online softmax of the wave's queries over KB keys, in base 2: s holds
// the products of the keys by the queries, scaled here by scale log2(e), so
// that each exponential is one v_exp_f32, exp2(s - max) = exp(scale (dot - max
// dot)).  With TAIL, keys from `valid` on are masked (exponential 0).  The
// running maximum m, the sum l of the exponentials in double precision and
// the output o are rescaled by exp2(old max - new max).
template <bool TAIL, int KB, int QT, int NDV>
__device__ __forceinline__ void fast_softmax(float4v (&s)[KB / 16][QT], float (&m)[QT], double (&l)[QT],
                                             float4v (&o)[QT][NDV], float scale2, int64_t valid, int lg) {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < KB / 16; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float x = s[kt][t][r] * scale2;
                if (TAIL && 16 * kt + 4 * lg + r >= valid) x = -INFINITY;
                s[kt][t][r] = x;
                mx = fmaxf(mx, x);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(m[t], mx);
        const float alpha = __builtin_amdgcn_exp2f(m[t] - mnew);  // 0 while m is -inf
        m[t] = mnew;
        double part = 0.0;
#pragma unroll
        for (int kt = 0; kt < KB / 16; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = __builtin_amdgcn_exp2f(s[kt][t][r] - mnew);  // 0 for a masked key
                s[kt][t][r] = p;
                part += static_cast<double>(p);
            }
        l[t] = l[t] * static_cast<double>(alpha) + part;
#pragma unroll
        for (int c = 0; c < NDV; ++c) o[t][c] *= alpha;
    }
}

template <int D, int QT, int KB>
__global__ __launch_bounds__(256, 2) void attention_fast_kernel(AttentionArgs a) {
    using F = Fast<D, QT, KB>;
    extern __shared__ float lds[];  // two buffers: keys [KB][kLdk], then values [KB][kLdv]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 15;
    const int lg = lane >> 4;

    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint32_t qb = b % static_cast<uint32_t>(a.qblocks);
    const uint32_t bh = b / static_cast<uint32_t>(a.qblocks);
    const int64_t hi = bh % a.h;
    const int64_t bi = bh / a.h;
    const int64_t kh = hi / (a.h / a.hk);
    const int64_t q0 = static_cast<int64_t>(qb) * F::kQueries + wave * 16 * QT;

    // The values' dimensions past D are never loaded: zeros, so that the
    // output rows past D (never stored) are finite.
    for (int idx = tid; idx < 2 * KB * (F::kLdv - D); idx += 256) {
        const int buf = idx / (KB * (F::kLdv - D));
        const int rest = idx - buf * KB * (F::kLdv - D);
        const int j = rest / (F::kLdv - D);
        const int e = D + rest - j * (F::kLdv - D);
        lds[buf * F::kBuffer + KB * F::kLdk + j * F::kLdv + e] = 0.0f;
    }

    // The wave's queries: operand B of S^T, lane (query lr, lg) holding
    // dimension 4 s + lg at step s.  Queries past lq read the last one.
    float q[QT][F::kSteps];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        int64_t i = q0 + 16 * t + lr;
        i = i < a.lq ? i : a.lq - 1;
        const float *qp = a.q + bi * a.qnb3 + hi * a.qnb2 + i * a.qnb1 + lg;
#pragma unroll
        for (int st = 0; st < F::kSteps; ++st) q[t][st] = qp[4 * st];
    }

    const float *kg = static_cast<const float *>(a.k) + bi * a.knb3 + kh * a.knb2;
    const float *vg = static_cast<const float *>(a.v) + bi * a.vnb3 + kh * a.vnb2;
    float4v kr[F::kPer], vr[F::kPer];

    float4v o[QT][F::kNdv];
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
        for (int c = 0; c < F::kNdv; ++c) o[t][c] = float4v{};
    float m[QT];
    double l[QT];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        m[t] = -INFINITY;
        l[t] = 0.0;
    }

    const float scale2 = a.scale * 1.44269504088896341f;  // scale log2(e)
    const int64_t nk = (a.lk + KB - 1) / KB;
    fast_load<F>(kr, vr, kg, vg, 0, a.lk, a.knb1, a.vnb1, tid);
    fast_store<F, KB>(kr, vr, lds, tid);
    __syncthreads();
    for (int64_t it = 0; it < nk; ++it) {
        const float *ks = lds + (it & 1) * F::kBuffer;
        const float *vs = ks + KB * F::kLdk;
        const int64_t k0 = it * KB;
        if (it + 1 < nk) fast_load<F>(kr, vr, kg, vg, k0 + KB, a.lk, a.knb1, a.vnb1, tid);

        // S^T for KB keys: lane holds the scores of its query lr (of each
        // tile t) for keys 16 kt + 4 lg + r.
        float4v s[KB / 16][QT];
#pragma unroll
        for (int kt = 0; kt < KB / 16; ++kt)
#pragma unroll
            for (int t = 0; t < QT; ++t) s[kt][t] = float4v{};
#pragma unroll
        for (int st = 0; st < F::kSteps; ++st)
#pragma unroll
            for (int kt = 0; kt < KB / 16; ++kt) {
                const float kv = ks[(16 * kt + lr) * F::kLdk + 4 * st + lg];
#pragma unroll
                for (int t = 0; t < QT; ++t) s[kt][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv, q[t][st], s[kt][t], 0, 0, 0);
            }

        // The online softmax of each query over these keys; the last block
        // of keys, past lk, by a form of its own that masks them.
        if (k0 + KB > a.lk) {
            fast_softmax<true, KB, QT, F::kNdv>(s, m, l, o, scale2, a.lk - k0, lg);
        } else {
            fast_softmax<false, KB, QT, F::kNdv>(s, m, l, o, scale2, KB, lg);
        }

        // O^T += V^T P^T: k index 4 lg + r of each tile of 16 keys.
#pragma unroll
        for (int kt = 0; kt < KB / 16; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < F::kNdv; ++c) {
                    const float vv = vs[(16 * kt + 4 * lg + r) * F::kLdv + 16 * c + lr];
#pragma unroll
                    for (int t = 0; t < QT; ++t)
                        o[t][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv, s[kt][t][r], o[t][c], 0, 0, 0);
                }

        if (it + 1 < nk) fast_store<F, KB>(kr, vr, lds + ((it + 1) & 1) * F::kBuffer, tid);
        __syncthreads();
    }

    // Each query's sum over its four lanes; lane holds O^T[16 c + 4 lg + r][lr].
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        double sum = l[t];
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        const float reciprocal = static_cast<float>(1.0 / sum);
        const int64_t i = q0 + 16 * t + lr;
        if (i >= a.lq) continue;
        float *out = a.y + bi * a.ynb3 + i * a.ynb2 + hi * a.ynb1;
#pragma unroll
        for (int c = 0; c < F::kNdv; ++c) {
            const int e = 16 * c + 4 * lg;
            if (e < D) {
                *reinterpret_cast<float4v *>(out + e) = o[t][c] * reciprocal;
            }
        }
    }
}

// ------------------------------------------------------------------ the split form
//
// The fast form's operands on the FP16 MFMA, v_mfma_f32_32x32x16_f16, the
// default.  Every single-precision key, query (times scale log2(e)) and value
// x is taken as two FP16 parts, h = fp16(x 2^-4) and l = fp16((x 2^-4 - h)
// 2^11), and every product as h h' + 2^-11 (h l' + l h'): h h' into one
// accumulator, the two others into a second, the two added once the sum is
// done.  That is 22 bits of each operand, the part l scaled into FP16's normal
// range so that it keeps its 11 bits for any |x| above 2^-20.  The
// exponentials, computed 2^11 times their value, are split as h + l with l
// the plain remainder, h h' + l h' into the first accumulator; the
// reference's metric stays at single precision's.
//
// Two launches.  The first splits the keys and values once, into the work
// buffer, as tiles of KB keys laid out as the second's LDS holds them: the
// keys' parts [KB][kLdk] twice, then the values' parts transposed,
// [kDvp][kLdv] twice, keys past lk and dimensions past D zero.  The second
// takes 32 queries a wave, 128 of one head a workgroup, and goes through the
// tiles in order, copying each whole from the work buffer into a ring of NS
// LDS buffers (global_load_lds_dwordx4, 1 KB an instruction, NS - 2 tiles
// ahead of the MFMAs; one barrier a tile).  S^T = K Q^T by tiles of 32 keys by
// the wave's 32 queries: lane l holds query l % 32, keys 8 (e / 4) + 4 (l /
// 32) + e % 4 of its accumulator element e.  Those are the operand B of O^T
// += V^T P^T as they stand when the MFMA's k index 8 (l / 32) + j of a chunk
// of 16 keys is taken for key 8 (j / 4) + 4 (l / 32) + j % 4; the values'
// columns are stored in that order of keys, so that a lane's eight keys of
// operand A are one 16-byte read.  The queries' parts stay in registers
// (operand B of S^T).  LDS rows are an odd number of 16-byte units long -- D
// padded to 16 and 8 halves more for the keys, KB + 8 halves for the values --
// which the MFMAs' reads of 32 rows take without bank conflicts.

template <int D, int KB>
struct Split {
    static constexpr int kDp = (D + 15) / 16 * 16;  // dimensions of the keys and queries, padded
    static constexpr int kSteps = kDp / 16;
    static constexpr int kDvp = (D + 31) / 32 * 32;  // of the values, whole tiles of 32
    static constexpr int kDvt = kDvp / 32;
    static constexpr int kTiles = KB / 32;           // tiles of 32 keys
    static constexpr int kLdk = kDp + 8;             // halves
    static constexpr int kLdv = KB + 8;              // halves
    static constexpr int kPlaneK = KB * kLdk;
    static constexpr int kPlaneV = kDvp * kLdv;
    static constexpr int kQueries = 128;  // a workgroup's
    // D = 16 n + 8: the scores' last step has 8 dimensions, and the keys' low
    // parts of those fill its other 8 (the keys' first plane holds l at
    // columns D .. D + 7 for dimensions D - 8 .. D - 1), so that the step
    // takes two MFMAs: h h' into the first accumulator, and (h l' + l h')
    // into the second from a lane of the upper half holding h' of the
    // dimension 8 below its own.
    static constexpr bool kHalfStep = D % 16 == 8;
    // The values' last tile of 32 dimensions holds kVLast of them; at 16 or
    // fewer its low parts go to its own spare rows kVLast .. 2 kVLast - 1 of
    // the first plane, and it takes two MFMAs (h + l) h' where the others
    // take three.  With 8 more rows spare those hold ones times 2^-4, so
    // that the MFMAs sum the exponentials beside the outputs.
    static constexpr int kVLast = D - 32 * (kDvt - 1);
    static constexpr bool kPackV = kVLast <= 16;
    static constexpr bool kSumRow = kPackV && 2 * kVLast + 8 <= 32;
    // The operands A of a tile's MFMAs read from LDS before the softmax's
    // maximum rather than next to the MFMAs, where the registers allow it
    // (their 44 more keep SD1.5's heads of 40 at two waves a SIMD).
    static constexpr bool kEarlyReads = D == 40;
    // The record holds only what the MFMAs read: the keys' second plane the
    // dimensions of the steps that take it (rows of kLdkl halves), the
    // values' second plane the tiles that take it (kDvlo rows).
    static constexpr int kLdkl = (kHalfStep ? kDp - 16 : kDp) + 8;
    static constexpr int kDvlo = kPackV ? kDvp - 32 : kDvp;
    static constexpr int kPlaneKl = KB * kLdkl;
    static constexpr int kValues = kPlaneK + kPlaneKl;  // halves before the values' planes
    static constexpr int kPlaneVl = kDvlo * kLdv;
    static constexpr int kHalves = kValues + kPlaneV + kPlaneVl;        // of a tile
    static constexpr int kRecord = (2 * kHalves + 1023) / 1024 * 1024;  // bytes of a tile, whole KB
    static constexpr int kCopies = kRecord / 1024;                      // 1 KB copies of a tile
    static constexpr int kPerWave = (kCopies + 3) / 4;
    // The LDS buffers of the form that splits the keys and values itself
    // (LOCAL): as large as both planes in full, for its staging.
    static constexpr int kLocalBuffer = (4 * (kPlaneK + kPlaneV) + 1023) / 1024 * 1024;
    static_assert(D % 8 == 0 && KB % 32 == 0, "shape");
    static_assert(!kHalfStep || kDp == D + 8, "the keys' low parts fill the last step's padding");
    static_assert((kLdkl / 8) % 2 == 1, "rows of an odd number of 16-byte units");
    static_assert((kLdk / 8) % 2 == 1 && (kLdv / 8) % 2 == 1, "rows of an odd number of 16-byte units");
};

constexpr float kPartUp = 2048.0f;  // the part l's scale, 2^11
constexpr float kPartDown = 1.0f / 2048.0f;

typedef _Float16 half4a __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void split_part(float x, _Float16 &h, _Float16 &l) {
    h = static_cast<_Float16>(x);
    l = static_cast<_Float16>((x - static_cast<float>(h)) * kPartUp);
}

// The key of column c of a tile's values: within a chunk of 16 columns,
// column 8 g + s holds key 8 (s / 4) + 4 g + s % 4.
__device__ __forceinline__ int key_of_column(int c) {
    const int g = (c >> 3) & 1, s = c & 7;
    return (c & ~15) + 8 * (s >> 2) + 4 * g + (s & 3);
}

// The keys of tile kt of (image bi, key head kh) split into their two parts,
// [KB][kLdk] twice, into `rec` (the work buffer's record or an LDS buffer),
// by the workgroup's threads: a thread a key's four dimensions, float4 loads.
// With kHalfStep the first plane's columns D .. D + 7 take the low parts of
// dimensions D - 8 .. D - 1, and the second plane's rows are kLdkl long.
template <int D, int KB>
__device__ __forceinline__ void split_keys(const AttentionArgs &a, int64_t bi, int64_t kh, int64_t kt, _Float16 *rec) {
    using S = Split<D, KB>;
    const float *kg = static_cast<const float *>(a.k) + bi * a.knb3 + kh * a.knb2;
    for (int idx = threadIdx.x; idx < KB * (S::kLdk / 4); idx += 256) {
        const int j = idx / (S::kLdk / 4);
        const int c4 = idx - j * (S::kLdk / 4);
        const bool slot = S::kHalfStep && 4 * c4 >= D && 4 * c4 < D + 8;
        const int src = slot ? 4 * c4 - 8 : 4 * c4;
        const int64_t key = kt * KB + j;
        float4v x = float4v{};
        if (key < a.lk && src < D) x = *reinterpret_cast<const float4v *>(kg + key * a.knb1 + src);
        half4a h, l;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            _Float16 hh, ll;
            split_part(x[r] * kSplitDown, hh, ll);
            h[r] = hh;
            l[r] = ll;
        }
        *reinterpret_cast<half4a *>(rec + j * S::kLdk + 4 * c4) = slot ? l : h;
        if (4 * c4 < S::kLdkl) *reinterpret_cast<half4a *>(rec + S::kPlaneK + j * S::kLdkl + 4 * c4) = l;
    }
}

// The values of tile kt split and transposed, [kDvp][kLdv] and [kDvlo][kLdv]
// after the keys' planes of `rec`, a thread four columns (four keys, in the order of
// key_of_column) of a dimension; `vt(j, dim)` gives value dim of key j of the
// tile (zero past lk).  With kPackV the first plane's rows D .. D + kVLast -
// 1 take the low parts of the last tile's dimensions, and with kSumRow its
// next 8 rows 2^-4 at every key.
template <int D, int KB, class V>
__device__ __forceinline__ void split_values(V vt, _Float16 *rec) {
    using S = Split<D, KB>;
    _Float16 *vh = rec + S::kValues;
    for (int idx = threadIdx.x; idx < S::kDvp * (S::kLdv / 4); idx += 256) {
        const int dim = idx / (S::kLdv / 4);
        const int c4 = idx - dim * (S::kLdv / 4);
        const bool low = S::kPackV && dim >= D && dim < D + S::kVLast;
        const bool ones = S::kSumRow && dim >= D + S::kVLast && dim < D + S::kVLast + 8;
        const int src = low ? dim - S::kVLast : dim;
        half4a h, l;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int c = 4 * c4 + u;
            const float x = c < KB && src < D ? vt(key_of_column(c), src) : 0.0f;
            _Float16 hh, ll;
            split_part(x * kSplitDown, hh, ll);
            h[u] = low ? ll : ones && c < KB ? static_cast<_Float16>(kSplitDown) : hh;
            l[u] = ll;
        }
        *reinterpret_cast<half4a *>(vh + dim * S::kLdv + 4 * c4) = h;
        if (dim < S::kDvlo) *reinterpret_cast<half4a *>(vh + S::kPlaneV + dim * S::kLdv + 4 * c4) = l;
    }
}

// The tiles of the keys and values of every (image, head of the keys), one
// workgroup a tile of nk a head.  Block (bi nk + kt) hk + kh: the heads of one
// tile of keys, whose rows lie side by side in memory ([b][lk][hk][d]) and
// share its lines, are consecutive blocks of one XCD, which its L2 serves
// together.
template <int D, int KB>
__global__ __launch_bounds__(256) void attention_tiles_kernel(AttentionArgs a, _Float16 *__restrict__ tiles,
                                                              uint32_t nk) {
    using S = Split<D, KB>;
    const uint32_t blk = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint32_t hk = static_cast<uint32_t>(a.hk);
    const uint32_t rest = blk / hk;
    const int64_t kh = blk - rest * hk;
    const int64_t bi = rest / nk;
    const int64_t kt = rest - static_cast<uint32_t>(bi) * nk;
    const int64_t bh = bi * a.hk + kh;
    _Float16 *rec = tiles + (bh * nk + kt) * (S::kRecord / 2);
    const float *vg = static_cast<const float *>(a.v) + bi * a.vnb3 + kh * a.vnb2;
    split_keys<D, KB>(a, bi, kh, kt, rec);
    // The values, transposed through LDS: rows read as float4, then a thread
    // four columns (four consecutive keys) of a dimension, consecutive threads
    // consecutive columns.
    __shared__ __attribute__((aligned(16))) float vt[KB][D + 4];
    for (int idx = threadIdx.x; idx < KB * (D / 4); idx += 256) {
        const int j = idx / (D / 4);
        const int c4 = idx - j * (D / 4);
        const int64_t key = kt * KB + j;
        float4v x = float4v{};
        if (key < a.lk) x = *reinterpret_cast<const float4v *>(vg + key * a.vnb1 + 4 * c4);
        *reinterpret_cast<float4v *>(&vt[j][4 * c4]) = x;
    }
    __syncthreads();
    split_values<D, KB>([&](int j, int dim) { return vt[j][dim]; }, rec);
}

// The greater of x on lanes i and i + 32 (the wave's two halves), on both:
// v_permlane32_swap of two copies leaves one with the lower half's x on
// every lane and the other with the upper's, with no trip through LDS.
__device__ __forceinline__ float halves_max(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    // The elements as scalars first: this compiler takes __builtin_bit_cast of
    // an element of a vector from the vector's first element.
    const unsigned lower = r[0], upper = r[1];
    return fmaxf(__builtin_bit_cast(float, lower), __builtin_bit_cast(float, upper));
}

// The online softmax of the wave's scores over KB keys, in base 2, in two
// halves: split_max, then split_exp.  The accumulators hold the products of
// the keys by the queries times scale log2(e), scaled by 2^-8 (the keys' and
// queries' 2^-4), as sh + 2^-11 sx; with MASK, keys from `valid` on are
// masked.  The running maximum m, in that scaled unit, moves only when a
// score passes it by more than 2^4 in exponential, so that the output's
// accumulators are rescaled (by exp2(256 (old max - new max))) seldom, and
// only while some query's maximum moves.  The exponentials go to p as 2^11
// exp2(256 (x - m)), below 2^15 -- the 2^11 so that their low FP16 parts stay
// normal down to exponentials of 2^-14, below which they weigh less than the
// rounding of the sum -- and, with SUM, their sum into l, taken 16 at a time
// as a tree in single precision and added in double (without, the MFMAs sum
// them from the values' rows of ones).
//
// split_max: the scores into p, the new maximum, the rescaling; returns the
// exponentials' shift.  The branch comes before the exponentials, so that
// those share a basic block with the next tile's MFMAs.
template <bool MASK, bool SUM, int KT, int DVT>
__device__ __forceinline__ float split_max(const float16v (&sh)[KT], const float16v (&sx)[KT], float (&p)[KT][16],
                                           float &m, double &l, float16v (&oh)[DVT], float16v (&ol)[DVT],
                                           int valid, int g) {
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            float x = __builtin_fmaf(sx[t][e], kPartDown, sh[t][e]);
            if (MASK && 32 * t + tile_row(e) + 4 * g >= valid) x = -INFINITY;
            p[t][e] = x;
            mx = fmaxf(mx, x);
        }
    mx = halves_max(mx);
    const float mnew = mx > m + 4.0f / 256.0f ? mx : m;
    if (__ballot(mnew != m) != 0) {
        const float alpha = __builtin_amdgcn_exp2f((m - mnew) * 256.0f);  // 0 while m is -inf
        if constexpr (SUM) l *= static_cast<double>(alpha);
#pragma unroll
        for (int c = 0; c < DVT; ++c) {
            oh[c] *= alpha;
            ol[c] *= alpha;
        }
        m = mnew;
    }
    return m * 256.0f - 11.0f;
}

// split_exp: the exponentials of the scores in p, their sum with SUM.
template <bool SUM, int KT>
__device__ __forceinline__ void split_exp(float (&p)[KT][16], float shift, double &l) {
    double part = 0.0;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
#pragma unroll
        for (int e = 0; e < 16; ++e) p[t][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(p[t][e], 256.0f, -shift));
        if constexpr (SUM) {
            float a8[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) a8[u] = p[t][2 * u] + p[t][2 * u + 1];
#pragma unroll
            for (int u = 0; u < 4; ++u) a8[u] = a8[2 * u] + a8[2 * u + 1];
            part += static_cast<double>((a8[0] + a8[1]) + (a8[2] + a8[3]));
        }
    }
    if constexpr (SUM) l += part;
}

// Partial results of the split form's key splits: per (b h, split, query)
// the running maximum, the sum and the unnormalised output.
struct KeyPartial {
    float *m;   // [b h][split][lq]
    double *l;  // [b h][split][lq]
    float *o;   // [b h][split][lq][dv], 16-byte aligned
};

template <int D, int KB, int NS, int OCC, bool PIPE, bool LOCAL>
__global__ __launch_bounds__(256, OCC) void attention_split_kernel(AttentionArgs a, const char *__restrict__ tiles,
                                                                   int64_t splits, int64_t per, KeyPartial part) {
    using S = Split<D, KB>;
    static_assert(NS >= 3 && (NS - 2) * S::kPerWave < 64, "stages");
    // LDS buffers of kStride bytes: a tile's record, or with LOCAL room for
    // the staging as well.
    constexpr int kStride = LOCAL ? S::kLocalBuffer : S::kRecord;
    static_assert(S::kQueries * D * 4 <= NS * kStride, "the queries' staging fits the ring");
    static_assert(KB * (D + 4) * 4 <= kStride, "a tile's values fit a buffer as they stand");
    extern __shared__ __attribute__((aligned(1024))) char sbuf[];  // NS buffers of kStride bytes

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 31;  // the lane's query, or its row of operand A
    const int g = lane >> 5;   // the lane's half of the wave
    float minus_one;           // -1, in a scalar register (see values below)
    asm("s_mov_b32 %0, -1.0" : "=s"(minus_one));

    // With key splits (splits > 1) the workgroup takes tiles [t0, t0 +
    // per) of the head's nk_all and writes partial results for
    // split_combine_kernel; nk is then its own count of tiles.
    // Consecutive blocks of one XCD: the query blocks of a head, which read
    // the same tiles of keys; with LOCAL (a few keys, every workgroup its own
    // copies), the heads of a query block instead, whose rows of queries and
    // of the output lie side by side in memory and share lines.
    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    uint32_t qb, rest;
    if constexpr (LOCAL) {
        const uint32_t heads = static_cast<uint32_t>(a.b * a.h);
        qb = b / heads;
        rest = b - qb * heads;
    } else {
        qb = b % static_cast<uint32_t>(a.qblocks);
        rest = b / static_cast<uint32_t>(a.qblocks);
    }
    const int64_t sp = static_cast<int64_t>(rest % static_cast<uint32_t>(splits));
    const uint32_t bh = rest / static_cast<uint32_t>(splits);
    const int64_t hi = bh % a.h;
    const int64_t bi = bh / a.h;
    const int64_t kh = hi / (a.h / a.hk);
    const int64_t q0 = static_cast<int64_t>(qb) * S::kQueries + wave * 32;
    const int64_t nk_all = (a.lk + KB - 1) / KB;
    const int64_t t0 = sp * per;
    const int64_t nk = t0 + per < nk_all ? per : nk_all - t0;
    const char *head = tiles + ((bi * a.hk + kh) * nk_all + t0) * S::kRecord;

    // Tile `t` into LDS buffer `stage`: the wave's kPerWave copies of 1 KB
    // (those past the tile's last repeat it).
    // The wave's index as a scalar, so that the copies' addresses are a
    // scalar base and the lane's fixed 16-byte offset.
    const int swave = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t lane16 = static_cast<uint32_t>(lane) * 16u;
    // The split's tiles as a buffer resource (its nk records, below 2^31
    // bytes: key_splits caps nk), so that each copy's address is the lane's
    // 16 bytes and a scalar offset.
    const __amdgpu_buffer_rsrc_t head_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char *>(head), 0, static_cast<int>(LOCAL ? 0 : nk * S::kRecord), 0x00020000);
    const auto issue = [&](int stage, int64_t t) {
#pragma unroll
        for (int i = 0; i < S::kPerWave; ++i) {
            int c = swave + 4 * i;
            c = c < S::kCopies ? c : S::kCopies - 1;
            copy_lds_buffer(head_rsrc, lane16, static_cast<uint32_t>(t * S::kRecord + c * 1024),
                            sbuf + stage * kStride + c * 1024);
        }
    };
    // The wave's queries, operand B of S^T: lane (query lr, half g) holds
    // dimensions 16 st + 8 g .. + 7 at step st; queries past lq read the
    // last.  With LOCAL (a few tiles of keys, so the queries' loads weigh)
    // the workgroup's queries go through LDS first, rows of D read as float4
    // by consecutive threads; otherwise each lane reads its own row.
    half8 qh[S::kSteps], ql[S::kSteps];
    const float qscale = a.scale * 1.44269504088896341f;  // scale log2(e), folded into the queries
    // The lane's query (row qp) into its parts.  With kHalfStep the last
    // step's upper half holds h' of the dimension 8 below its own where the
    // others hold l', and zero where they hold h'.
    const auto take_query = [&](const float *qp) {
#pragma unroll
        for (int st = 0; st < S::kSteps; ++st)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const bool slot = S::kHalfStep && st == S::kSteps - 1 && g == 1;
                const int dim = 16 * st + 8 * g + j - (slot ? 8 : 0);
                _Float16 h, l;
                split_part(dim < D ? (qp[dim] * qscale) * kSplitDown : 0.0f, h, l);
                qh[st][j] = slot ? static_cast<_Float16>(0.0f) : h;
                ql[st][j] = slot ? h : l;
            }
    };
    // LOCAL, where the staging fits: every load of the workgroup -- its
    // queries, and the keys and values of every tile -- in flight at once,
    // into registers; then the queries staged in buffers 1 .., the values as
    // they stand in the spare buffer NS - 1, tile 0's keys split into buffer
    // 0; past a barrier each lane's query from the staging; past another the
    // other tiles' keys split, the padding dimensions of the keys cleared and
    // every tile's values split and transposed from the staging.  One wait for
    // memory where a tile at a time takes one a tile.
    constexpr bool kBatch = LOCAL && (NS - 1) * KB * (D + 4) * 4 <= kStride &&
                            S::kQueries * D * 4 <= (NS - 2) * kStride;
    if constexpr (kBatch) {
        constexpr int kQ4 = S::kQueries * (D / 4);  // float4s of the workgroup's queries
        constexpr int kQPer = (kQ4 + 255) / 256;
        constexpr int kKV4 = (NS - 1) * KB * (D / 4);  // float4s of the keys (or values) of NS - 1 tiles
        constexpr int kKVPer = (kKV4 + 255) / 256;
        const float *qg = a.q + bi * a.qnb3 + hi * a.qnb2;
        const float *kg = static_cast<const float *>(a.k) + bi * a.knb3 + kh * a.knb2;
        const float *vg = static_cast<const float *>(a.v) + bi * a.vnb3 + kh * a.vnb2;
        const int64_t qrow0 = static_cast<int64_t>(qb) * S::kQueries;
        float4v qv[kQPer], kv[kKVPer], vv[kKVPer];
#pragma unroll
        for (int i = 0; i < kQPer; ++i) {
            const int idx = tid + 256 * i;
            qv[i] = float4v{};
            if (idx < kQ4) {
                const int r = idx / (D / 4), c4 = idx - r * (D / 4);
                const int64_t row = qrow0 + r < a.lq ? qrow0 + r : a.lq - 1;
                qv[i] = *reinterpret_cast<const float4v *>(qg + row * a.qnb1 + 4 * c4);
            }
        }
#pragma unroll
        for (int i = 0; i < kKVPer; ++i) {
            const int idx = tid + 256 * i;
            const int key = idx / (D / 4), c4 = idx - key * (D / 4);
            kv[i] = float4v{};
            vv[i] = float4v{};
            if (idx < kKV4 && key < a.lk) {
                kv[i] = *reinterpret_cast<const float4v *>(kg + key * a.knb1 + 4 * c4);
                vv[i] = *reinterpret_cast<const float4v *>(vg + key * a.vnb1 + 4 * c4);
            }
        }
        float *qstage = reinterpret_cast<float *>(sbuf + kStride);              // [kQueries][D]
        float *vstage = reinterpret_cast<float *>(sbuf + (NS - 1) * kStride);   // [key][D + 4]
        // Key `key`'s four dimensions 4 c4 .. split into its tile's two planes.
        const auto put_key = [&](int key, int c4, float4v x) {
            _Float16 *rec = reinterpret_cast<_Float16 *>(sbuf + (key / KB) * kStride);
            const int j = key % KB;
            half4a h, l;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                _Float16 hh, ll;
                split_part(x[r] * kSplitDown, hh, ll);
                h[r] = hh;
                l[r] = ll;
            }
            *reinterpret_cast<half4a *>(rec + j * S::kLdk + 4 * c4) = h;
            if (4 * c4 < S::kLdkl) *reinterpret_cast<half4a *>(rec + S::kPlaneK + j * S::kLdkl + 4 * c4) = l;
            if (S::kHalfStep && 4 * c4 >= D - 8) *reinterpret_cast<half4a *>(rec + j * S::kLdk + 4 * c4 + 8) = l;
        };
#pragma unroll
        for (int i = 0; i < kQPer; ++i) {
            const int idx = tid + 256 * i;
            if (idx < kQ4) {
                const int r = idx / (D / 4), c4 = idx - r * (D / 4);
                *reinterpret_cast<float4v *>(qstage + r * D + 4 * c4) = qv[i];
            }
        }
#pragma unroll
        for (int i = 0; i < kKVPer; ++i) {
            const int idx = tid + 256 * i;
            const int key = idx / (D / 4), c4 = idx - key * (D / 4);
            if (idx < kKV4) {
                *reinterpret_cast<float4v *>(vstage + key * (D + 4) + 4 * c4) = vv[i];
                if (key < KB) put_key(key, c4, kv[i]);
            }
        }
        __syncthreads();
        const float *qp = qstage + (wave * 32 + lr) * D;
        take_query(qp);
        __syncthreads();  // every wave's queries read before the tiles overwrite their staging
#pragma unroll
        for (int i = 0; i < kKVPer; ++i) {
            const int idx = tid + 256 * i;
            const int key = idx / (D / 4), c4 = idx - key * (D / 4);
            if (idx < kKV4 && key >= KB && key < nk * KB) put_key(key, c4, kv[i]);
        }
        constexpr int kPad4 = (S::kDp - D) / 4;  // float4s of padding dimensions a key
        if constexpr (kPad4 > 0 && !S::kHalfStep) {  // with kHalfStep the padding holds low parts
            for (int idx = tid; idx < nk * KB * kPad4; idx += 256) {
                const int key = idx / kPad4, c4 = D / 4 + (idx - key * kPad4);
                put_key(key, c4, float4v{});
            }
        }
        for (int64_t t = 0; t < nk; ++t) {
            const float *vt = vstage + t * KB * (D + 4);
            split_values<D, KB>([&](int j, int dim) { return vt[j * (D + 4) + dim]; },
                                reinterpret_cast<_Float16 *>(sbuf + t * kStride));
        }
        __syncthreads();
    } else {
        const float *qp;
        if constexpr (LOCAL) {
            float *qstage = reinterpret_cast<float *>(sbuf);  // [kQueries][D]
            const int64_t qrow0 = static_cast<int64_t>(qb) * S::kQueries;
            for (int idx = tid; idx < S::kQueries * (D / 4); idx += 256) {
                const int r = idx / (D / 4), c4 = idx - r * (D / 4);
                int64_t i = qrow0 + r;
                i = i < a.lq ? i : a.lq - 1;
                *reinterpret_cast<float4v *>(qstage + r * D + 4 * c4) =
                    *reinterpret_cast<const float4v *>(a.q + bi * a.qnb3 + hi * a.qnb2 + i * a.qnb1 + 4 * c4);
            }
            __syncthreads();
            qp = qstage + (wave * 32 + lr) * D;
        } else {
            int64_t i = q0 + lr;
            i = i < a.lq ? i : a.lq - 1;
            qp = a.q + bi * a.qnb3 + hi * a.qnb2 + i * a.qnb1;
        }
        take_query(qp);
        if constexpr (LOCAL) __syncthreads();  // every wave's queries read before the ring is filled
    }
    // LOCAL (the tiles fit the ring with a buffer to spare): the workgroup
    // splits the keys and values itself, tile t into buffer t, where the other
    // form copies the tiles made by attention_tiles_kernel; each tile's values
    // go first as they stand into the spare buffer, rows read as float4, and
    // are transposed from there.
    if constexpr (LOCAL && !kBatch) {
        const float *vg = static_cast<const float *>(a.v) + bi * a.vnb3 + kh * a.vnb2;
        float *vt = reinterpret_cast<float *>(sbuf + (NS - 1) * kStride);  // [KB][D + 4]
        for (int64_t t = 0; t < nk; ++t) {
            _Float16 *rec = reinterpret_cast<_Float16 *>(sbuf + t * kStride);
            split_keys<D, KB>(a, bi, kh, t, rec);
            for (int idx = tid; idx < KB * (D / 4); idx += 256) {
                const int j = idx / (D / 4), c4 = idx - j * (D / 4);
                const int64_t key = t * KB + j;
                float4v x = float4v{};
                if (key < a.lk) x = *reinterpret_cast<const float4v *>(vg + key * a.vnb1 + 4 * c4);
                *reinterpret_cast<float4v *>(vt + j * (D + 4) + 4 * c4) = x;
            }
            __syncthreads();
            split_values<D, KB>([&](int j, int dim) { return vt[j * (D + 4) + dim]; }, rec);
            __syncthreads();
        }
    }
    float16v oh[S::kDvt], ol[S::kDvt];
#pragma unroll
    for (int c = 0; c < S::kDvt; ++c) {
        oh[c] = float16v{};
        ol[c] = float16v{};
    }
    float m = -INFINITY;
    double l = 0.0;
    constexpr bool kSum = !S::kSumRow;  // the sum of the exponentials by VALU work, else by the MFMAs

    // The ring: tile t in buffer t % NS.  With PIPE the scores of tile t + 1
    // are taken while the exponentials of tile t are (the MFMAs of the one
    // beside the VALU work of the other), so a buffer is free once the
    // products by the values of the tile before the one being scored are
    // done: tile t + NS - 2 is copied once tile t is in.  Without, tile t +
    // NS - 1 is.
    constexpr int kAhead = PIPE ? NS - 2 : NS - 1;
    const auto sync = [&](int64_t t) {
        if constexpr (LOCAL) return;  // every tile in LDS since the start
        // The wave's copies of tile t are done once at most kAhead - 1
        // tiles' copies are outstanding after them (none, near the end);
        // every wave's are, past the barrier, which also ends every wave's
        // reads of the buffer the next copies go to.
        if (t + kAhead - 1 < nk) {
            wait_loads<(kAhead - 1) * S::kPerWave>();
        } else {
            wait_loads<0>();
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (t + kAhead < nk) issue(static_cast<int>((t + kAhead) % NS), t + kAhead);
    };
    // The operands A of a tile's MFMAs, read from LDS ahead of them (before
    // the softmax's maximum, so that the reads are done by the time the
    // MFMAs issue): the keys' parts of tile t, the values' of tile t.
    half8 kah[S::kSteps][S::kTiles], kal[S::kSteps][S::kTiles];
    half8 vah[S::kTiles][2][S::kDvt], val[S::kTiles][2][S::kDvt];
    const auto read_keys = [&](int64_t t) {
        const _Float16 *kbuf = reinterpret_cast<const _Float16 *>(sbuf + (t % NS) * kStride);
#pragma unroll
        for (int st = 0; st < S::kSteps; ++st)
#pragma unroll
            for (int u = 0; u < S::kTiles; ++u) {
                const _Float16 *kp = kbuf + (32 * u + lr) * S::kLdk + 16 * st + 8 * g;
                kah[st][u] = *reinterpret_cast<const half8 *>(kp);
                if (!S::kHalfStep || st < S::kSteps - 1)
                    kal[st][u] = *reinterpret_cast<const half8 *>(kbuf + S::kPlaneK + (32 * u + lr) * S::kLdkl + 16 * st + 8 * g);
            }
    };
    const auto read_values = [&](int64_t t) {
        const _Float16 *vbuf = reinterpret_cast<const _Float16 *>(sbuf + (t % NS) * kStride) + S::kValues;
#pragma unroll
        for (int u = 0; u < S::kTiles; ++u)
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int dt = 0; dt < S::kDvt; ++dt) {
                    const _Float16 *vp = vbuf + (32 * dt + lr) * S::kLdv + 32 * u + 16 * c + 8 * g;
                    vah[u][c][dt] = *reinterpret_cast<const half8 *>(vp);
                    if (!S::kPackV || dt < S::kDvt - 1) val[u][c][dt] = *reinterpret_cast<const half8 *>(vp + S::kPlaneV);
                }
    };
    // S^T of the tile whose keys read_keys read.
    const auto scores = [&](float16v (&sh)[S::kTiles], float16v (&sx)[S::kTiles]) {
#pragma unroll
        for (int u = 0; u < S::kTiles; ++u) {
            sh[u] = float16v{};
            sx[u] = float16v{};
        }
#pragma unroll
        for (int st = 0; st < S::kSteps; ++st)
#pragma unroll
            for (int u = 0; u < S::kTiles; ++u) {
                sh[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kah[st][u], qh[st], sh[u], 0, 0, 0);
                sx[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kah[st][u], ql[st], sx[u], 0, 0, 0);
                if (!S::kHalfStep || st < S::kSteps - 1)
                    sx[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kal[st][u], qh[st], sx[u], 0, 0, 0);
            }
    };
    // O^T += V^T P^T of tile t, a chunk of 16 keys at a time: the lane's
    // eight exponentials 8 c .. 8 c + 7 of a tile of 32 are its operand B.
    const auto values = [&](const float (&p)[S::kTiles][16]) {
#pragma unroll
        for (int u = 0; u < S::kTiles; ++u)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                // The exponentials (2^11 times, below 2^15) as two FP16 parts,
                // the second the remainder of the first, in pairs.
                half8 ph, pl;
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    const float x0 = p[u][8 * c + j], x1 = p[u][8 * c + j + 1];
                    const auto h = __builtin_amdgcn_cvt_pkrtz(x0, x1);
                    // x - h, each one v_fma_mix_f32 (its -1 unknown to the
                    // compiler, which would make it a conversion and a
                    // subtraction).
                    const auto r = __builtin_amdgcn_cvt_pkrtz(__builtin_fmaf(static_cast<float>(h[0]), minus_one, x0),
                                                              __builtin_fmaf(static_cast<float>(h[1]), minus_one, x1));
                    ph[j] = h[0];
                    ph[j + 1] = h[1];
                    pl[j] = r[0];
                    pl[j + 1] = r[1];
                }
#pragma unroll
                for (int dt = 0; dt < S::kDvt; ++dt) {
                    oh[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vah[u][c][dt], ph, oh[dt], 0, 0, 0);
                    oh[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vah[u][c][dt], pl, oh[dt], 0, 0, 0);
                    if (!S::kPackV || dt < S::kDvt - 1)  // the packed tile's low parts are rows of vah
                        ol[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(val[u][c][dt], ph, ol[dt], 0, 0, 0);
                }
            }
    };

    // The first kAhead tiles on their way, once the queries are in; then
    // every tile but the last (with PIPE, the next one's scores beside it),
    // and the last, masked where it is not full.
    if constexpr (!LOCAL) {
#pragma unroll
        for (int st = 0; st < kAhead; ++st) {
            if (st < nk) issue(st, st);
        }
    }
    const auto last = [&](float16v (&sh)[S::kTiles], float16v (&sx)[S::kTiles]) {
        float p[S::kTiles][16];
        const int valid = t0 + nk == nk_all ? static_cast<int>(a.lk - (nk_all - 1) * KB) : KB;
        if constexpr (S::kEarlyReads) read_values(nk - 1);
        const float shift = valid < KB ? split_max<true, kSum, S::kTiles, S::kDvt>(sh, sx, p, m, l, oh, ol, valid, g)
                                       : split_max<false, kSum, S::kTiles, S::kDvt>(sh, sx, p, m, l, oh, ol, KB, g);
        split_exp<kSum, S::kTiles>(p, shift, l);
        if constexpr (!S::kEarlyReads) read_values(nk - 1);
        values(p);
    };
    if constexpr (PIPE) {
        // Two sets of scores, a and b, taking turns (no copies between them).
        float16v sa[S::kTiles], xa[S::kTiles], sb[S::kTiles], xb[S::kTiles];
        const auto step = [&](int64_t it, float16v (&sh)[S::kTiles], float16v (&sx)[S::kTiles],
                              float16v (&nh)[S::kTiles], float16v (&nx)[S::kTiles]) {
            sync(it + 1);
            if constexpr (S::kEarlyReads) {
                read_keys(it + 1);
                read_values(it);
            }
            float p[S::kTiles][16];
            const float shift = split_max<false, kSum, S::kTiles, S::kDvt>(sh, sx, p, m, l, oh, ol, KB, g);
            if constexpr (!S::kEarlyReads) read_keys(it + 1);
            // The wave's MFMAs and exponentials ahead of the other wave's
            // maximum on the SIMD (s_setprio): the MFMAs then issue while
            // the other's VALU work runs, rather than after it.
            __builtin_amdgcn_s_setprio(1);
            scores(nh, nx);
            split_exp<kSum, S::kTiles>(p, shift, l);
            if constexpr (!S::kEarlyReads) read_values(it);
            values(p);
            __builtin_amdgcn_s_setprio(0);
        };
        sync(0);
        read_keys(0);
        scores(sa, xa);
        int64_t it = 0;
        for (; it + 2 < nk; it += 2) {
            step(it, sa, xa, sb, xb);
            step(it + 1, sb, xb, sa, xa);
        }
        if (it + 1 < nk) {
            step(it, sa, xa, sb, xb);
            last(sb, xb);
        } else {
            last(sa, xa);
        }
    } else {
        float16v sh[S::kTiles], sx[S::kTiles];
        for (int64_t it = 0; it + 1 < nk; ++it) {
            sync(it);
            read_keys(it);
            if constexpr (S::kEarlyReads) read_values(it);
            scores(sh, sx);
            float p[S::kTiles][16];
            split_exp<kSum, S::kTiles>(p, split_max<false, kSum, S::kTiles, S::kDvt>(sh, sx, p, m, l, oh, ol, KB, g), l);
            if constexpr (!S::kEarlyReads) read_values(it);
            values(p);
        }
        sync(nk - 1);
        read_keys(nk - 1);
        scores(sh, sx);
        last(sh, sx);
    }

    // The query's sum over its two lanes, or from the rows of ones (the same
    // on both); lane holds O^T[32 dt + 8 (e / 4) + 4 g + e % 4][lr], and the
    // values' 2^-4 comes back with the reciprocal.  The packed tile's low
    // parts are kVLast rows, kVLast / 2 elements, below its high parts.
    double sum;
    if constexpr (S::kSumRow) {
        sum = static_cast<double>(oh[S::kDvt - 1][S::kVLast]) * 16.0;
    } else {
        sum = l;
        sum += __shfl_xor(sum, 32, 64);
    }
    const auto low = [&](int dt, int e) {
        return S::kPackV && dt == S::kDvt - 1 ? oh[dt][e + S::kVLast / 2] : ol[dt][e];
    };
    const int64_t i = q0 + lr;
    if (i >= a.lq) return;
    if (splits > 1) {
        // The split's maximum (the same on the query's two lanes), sum and
        // unnormalised output.
        const int64_t at = (static_cast<int64_t>(bh) * splits + sp) * a.lq + i;
        if (g == 0) {
            part.m[at] = m;
            part.l[at] = sum;
        }
        float *o = part.o + at * a.dv;
#pragma unroll
        for (int dt = 0; dt < S::kDvt; ++dt)
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {
                const int dim = 32 * dt + 8 * e4 + 4 * g;
                if (dim < D) {
                    float4v r;
#pragma unroll
                    for (int u = 0; u < 4; ++u) r[u] = (oh[dt][4 * e4 + u] + low(dt, 4 * e4 + u) * kPartDown) * 16.0f;
                    *reinterpret_cast<float4v *>(o + dim) = r;
                }
            }
        return;
    }
    const float reciprocal = static_cast<float>(1.0 / sum);
    float *out = a.y + bi * a.ynb3 + i * a.ynb2 + hi * a.ynb1;
#pragma unroll
    for (int dt = 0; dt < S::kDvt; ++dt)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            const int dim = 32 * dt + 8 * e4 + 4 * g;
            if (dim < D) {
                float4v r;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    r[u] = ((oh[dt][4 * e4 + u] + low(dt, 4 * e4 + u) * kPartDown) * 16.0f) * reciprocal;
                }
                *reinterpret_cast<float4v *>(out + dim) = r;
            }
        }
}

// The key splits of the split form merged, query by query: each split's sum
// and output rescaled by 2^(256 (its maximum - the greatest)), as
// split_max rescales its running ones, the sum in double, the output
// times the reciprocal of the sum rounded to single precision.  A wave per
// query.
__global__ __launch_bounds__(256) void split_combine_kernel(AttentionArgs a, int64_t splits, KeyPartial part) {
    const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);  // (b h) lq + i
    const int lane = threadIdx.x & 63;
    if (item >= a.b * a.h * a.lq) return;
    const int64_t bh = item / a.lq, i = item - bh * a.lq;
    const int64_t hi = bh % a.h, bi = bh / a.h;
    const int64_t first = bh * splits * a.lq + i;  // split 0 of the query
    float mx = -INFINITY;
    for (int64_t sp = 0; sp < splits; ++sp) mx = fmaxf(mx, part.m[first + sp * a.lq]);
    double l = 0.0;
    for (int64_t sp = 0; sp < splits; ++sp) {
        const float w = __builtin_amdgcn_exp2f((part.m[first + sp * a.lq] - mx) * 256.0f);
        l += part.l[first + sp * a.lq] * static_cast<double>(w);
    }
    const float reciprocal = static_cast<float>(1.0 / l);
    float *out = a.y + bi * a.ynb3 + i * a.ynb2 + hi * a.ynb1;
    for (int64_t e = lane; e < a.dv; e += 64) {
        float acc = 0.0f;
        for (int64_t sp = 0; sp < splits; ++sp) {
            const float w = __builtin_amdgcn_exp2f((part.m[first + sp * a.lq] - mx) * 256.0f);
            acc = fmaf(part.o[(first + sp * a.lq) * a.dv + e], w, acc);
        }
        out[e] = acc * reciprocal;
    }
}

// The split form's shape for head size D: its tiles' keys, the stages of its
// ring, the workgroups a CU holds at least.
template <int D>
struct SplitShape {
    static constexpr int kKeys = 32;
    static constexpr int kStages = D <= 64 ? 4 : 3;
    static constexpr int kOcc = D <= 96 ? 2 : 1;
    static constexpr bool kPipe = D <= 64;  // registers for two sets of scores
};

// Splits of the keys where the split form's workgroups would leave CUs idle
// (the UNet's 32 x 32 and 16 x 16 maps): as many, of two tiles or more, as
// fill one round of one workgroup a CU; the tiles a split takes.
struct KeySplits {
    int64_t splits, per;
};

template <int D>
KeySplits key_splits(const AttentionArgs &a) {
    using SH = SplitShape<D>;
    using S = Split<D, SH::kKeys>;
    const int64_t nk = ceil_div(a.lk, SH::kKeys);
    const int64_t blocks = ceil_div(a.lq, S::kQueries) * a.h * a.b;
    int64_t sp = 1;
    if (nk >= SH::kStages && blocks > 0 && blocks < compute_units()) {  // the tiles' launch (not LOCAL)
        sp = compute_units() / blocks;
        sp = sp < nk / 2 ? sp : nk / 2;
        sp = sp < 1 ? 1 : sp;
    }
    // A split's tiles stay below 2^31 bytes, the reach of the kernel's buffer
    // resource.
    const int64_t most = (INT32_MAX - 1024) / S::kRecord;
    sp = ceil_div(nk, sp) > most ? ceil_div(nk, most) : sp;
    const int64_t per = ceil_div(nk, sp);
    return {ceil_div(nk, per), per};
}

// The partial results' layout in the work buffer from `at` on, and its bytes.
struct KeyPartialLayout {
    size_t l, m, o, bytes;
};

inline KeyPartialLayout key_partial_layout(const AttentionArgs &a, int64_t splits) {
    const size_t n = static_cast<size_t>(a.b * a.h * splits * a.lq);
    KeyPartialLayout k{};
    k.l = 0;
    k.m = n * 8;
    k.o = static_cast<size_t>(round_up(static_cast<int64_t>(n * 12), 256));
    k.bytes = k.o + n * static_cast<size_t>(a.dv) * 4;
    return k;
}

template <int D>
size_t split_tiles_bytes(const AttentionArgs &a) {
    using S = Split<D, SplitShape<D>::kKeys>;
    return static_cast<size_t>(a.b * a.hk) * static_cast<size_t>(ceil_div(a.lk, SplitShape<D>::kKeys)) * S::kRecord;
}

template <int D>
size_t split_work(const AttentionArgs &a) {
    const KeySplits ks = key_splits<D>(a);
    const size_t tiles = split_tiles_bytes<D>(a);
    return ks.splits > 1 ? tiles + key_partial_layout(a, ks.splits).bytes : tiles;
}

template <int D, bool LOCAL>
hipError_t launch_split_t(AttentionArgs a, void *work, hipStream_t stream) {
    using SH = SplitShape<D>;
    using S = Split<D, SH::kKeys>;
    a.qblocks = ceil_div(a.lq, S::kQueries);
    const size_t lds = static_cast<size_t>(SH::kStages) * (LOCAL ? S::kLocalBuffer : S::kRecord);
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void *>(&attention_split_kernel<D, SH::kKeys, SH::kStages, SH::kOcc, SH::kPipe, LOCAL>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (attr != hipSuccess) return attr;
    const int64_t nk = ceil_div(a.lk, SH::kKeys);
    const KeySplits ks = LOCAL ? KeySplits{1, nk} : key_splits<D>(a);
    KeyPartial part{};
    if (ks.splits > 1) {
        char *base = static_cast<char *>(work) + split_tiles_bytes<D>(a);
        const KeyPartialLayout k = key_partial_layout(a, ks.splits);
        part.l = reinterpret_cast<double *>(base + k.l);
        part.m = reinterpret_cast<float *>(base + k.m);
        part.o = reinterpret_cast<float *>(base + k.o);
    }
    dim3 grid(static_cast<uint32_t>(a.qblocks * a.h * a.b * ks.splits)), block(256);
    KernelScope scope("attention", stream);
    SDHIP_LAUNCH((attention_split_kernel<D, SH::kKeys, SH::kStages, SH::kOcc, SH::kPipe, LOCAL>), grid, block, lds,
                 stream, a, static_cast<const char *>(work), ks.splits, ks.per, part);
    if (ks.splits > 1) {
        SDHIP_LAUNCH(split_combine_kernel, dim3(static_cast<uint32_t>(ceil_div(a.b * a.h * a.lq, 4))), block, 0,
                     stream, a, ks.splits, part);
    }
    return hipGetLastError();
}

template <int D>
hipError_t launch_split(AttentionArgs a, void *work, hipStream_t stream) {
    using SH = SplitShape<D>;
    const int64_t nk = ceil_div(a.lk, SH::kKeys);
    // Keys and values that fit the ring with a buffer to spare
    // (cross-attention's 77 at heads of up to 64): each workgroup splits them
    // itself, with no launch before it.
    if (nk < SH::kStages) return launch_split_t<D, true>(a, nullptr, stream);
    // The tiles' grid is one dimension of 256-thread blocks: under 2^24 of
    // them (a work buffer of 14 KB or more a tile, past 230 GB, before that).
    if (nk * a.b * a.hk >= (int64_t{1} << 24)) return hipErrorInvalidValue;
    {
        KernelScope scope("attention.tiles", stream);
        SDHIP_LAUNCH((attention_tiles_kernel<D, SH::kKeys>), dim3(static_cast<uint32_t>(nk * a.b * a.hk)),
                     dim3(256), 0, stream, a, static_cast<_Float16 *>(work), static_cast<uint32_t>(nk));
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    return launch_split_t<D, false>(a, work, stream);
}

template <int D, int QT, int KB>
hipError_t launch_fast(AttentionArgs a, hipStream_t stream) {
    using F = Fast<D, QT, KB>;
    a.qblocks = ceil_div(a.lq, F::kQueries);
    const size_t lds = sizeof(float) * 2 * F::kBuffer;
    dim3 grid(static_cast<uint32_t>(a.qblocks * a.h * a.b)), block(256);
    KernelScope scope("attention", stream);
    SDHIP_LAUNCH((attention_fast_kernel<D, QT, KB>), grid, block, lds, stream, a);
    return hipGetLastError();
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Whether the fast form takes the operands: single-precision keys and values
// of d = dv dimensions, an instantiated head size, float4-aligned rows.
bool fast_form(const AttentionArgs &a) {
    const bool size = a.d == 32 || a.d == 40 || a.d == 64 || a.d == 80 || a.d == 96 || a.d == 128 || a.d == 160;
    return size && a.d == a.dv && !a.khalf && !a.vhalf && aligned16(a.q) && aligned16(a.k) && aligned16(a.v) &&
           aligned16(a.y) && a.qnb1 % 4 == 0 && a.qnb2 % 4 == 0 && a.qnb3 % 4 == 0 && a.knb1 % 4 == 0 &&
           a.knb2 % 4 == 0 && a.knb3 % 4 == 0 && a.vnb1 % 4 == 0 && a.vnb2 % 4 == 0 && a.vnb3 % 4 == 0 &&
           a.ynb1 % 4 == 0 && a.ynb2 % 4 == 0 && a.ynb3 % 4 == 0;
}

// Whether the split form takes the operands: the fast form's, unless the
// tuning asks for another, or for products in bfloat16 (which the generic and
// wide forms compute).
bool split_form(const AttentionArgs &a) {
    return fast_form(a) && a.lk > 0 && tuning().attention_generic == 0 && tuning().attention_fp32 == 0 && !a.bf16;
}

size_t split_form_work(const AttentionArgs &a) {
    switch (a.d) {
    case 32: return split_work<32>(a);
    case 40: return split_work<40>(a);
    case 64: return split_work<64>(a);
    case 80: return split_work<80>(a);
    case 96: return split_work<96>(a);
    case 128: return split_work<128>(a);
    default: return split_work<160>(a);
    }
}

hipError_t launch_split_form(AttentionArgs a, void *work, hipStream_t stream) {
    switch (a.d) {
    case 32: return launch_split<32>(a, work, stream);
    case 40: return launch_split<40>(a, work, stream);
    case 64: return launch_split<64>(a, work, stream);
    case 80: return launch_split<80>(a, work, stream);
    case 96: return launch_split<96>(a, work, stream);
    case 128: return launch_split<128>(a, work, stream);
    default: return launch_split<160>(a, work, stream);
    }
}

hipError_t launch_fast_form(AttentionArgs a, hipStream_t stream) {
    switch (a.d) {
    case 32: return launch_fast<32, 2, 64>(a, stream);
    case 40: return launch_fast<40, 2, 64>(a, stream);
    case 64: return launch_fast<64, 2, 64>(a, stream);
    case 80: return launch_fast<80, 2, 32>(a, stream);
    case 96: return launch_fast<96, 2, 32>(a, stream);
    case 128: return launch_fast<128, 1, 32>(a, stream);
    default: return launch_fast<160, 1, 32>(a, stream);
    }
}

template <int NDV>
hipError_t launch_wide(AttentionArgs a, void *work, hipStream_t stream) {
    a.ldv = 16 * NDV + 4;
    const WideSplits w = wide_splits(a);
    const WidePartial part = w.splits > 1 ? wide_partial(work, a, w.splits) : WidePartial{nullptr, nullptr, nullptr};
    const size_t lds = sizeof(float) * (kQueries * kWideLd + kKeys * kWideLd + kKeys * a.ldv);
    // Values of more than 16 NDV dimensions (heads past 512) in slices.
    const int64_t slices = ceil_div(a.dv, 16 * NDV);
    const int64_t blocks = a.qblocks * w.splits * a.h * a.b * slices;
    if (blocks >= (int64_t{1} << 24)) return hipErrorInvalidValue;  // 256-thread blocks of one dimension
    dim3 grid(static_cast<uint32_t>(blocks)), block(256);
    const auto launch = [&](auto kernel) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return e;
        SDHIP_LAUNCH(kernel, grid, block, lds, stream, a, w.splits, w.key_len, part);
        return hipGetLastError();
    };
    hipError_t e;
    // Single-precision keys and values of heads of 388 .. 512 dimensions (a
    // multiple of 4, rows float4-aligned): the queries held in registers,
    // the dimensions past d zeros that add nothing to the sums.
    const bool rows4 = a.knb1 % 4 == 0 && a.vnb1 % 4 == 0 && a.knb2 % 4 == 0 && a.vnb2 % 4 == 0 &&
                       a.knb3 % 4 == 0 && a.vnb3 % 4 == 0 && (reinterpret_cast<uintptr_t>(a.k) & 15) == 0 &&
                       (reinterpret_cast<uintptr_t>(a.v) & 15) == 0;
    if (!a.khalf && !a.vhalf && a.dp > 384 && a.dp <= 512 && a.d % 4 == 0 && a.dv % 4 == 0 && rows4 && NDV == 32 &&
        slices == 1 && tuning().attention_generic == 0 && !a.bf16) {
        const size_t lds2 = sizeof(float) * (kKeys * (512 + 4) + kKeys * (16 * NDV + 4));
        hipError_t e2 = hipFuncSetAttribute(reinterpret_cast<const void *>(attention_wide2_kernel<512, NDV>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds2));
        if (e2 != hipSuccess) return e2;
        SDHIP_LAUNCH((attention_wide2_kernel<512, NDV>), grid, block, lds2, stream, a, w.splits, w.key_len, part);
        e = hipGetLastError();
    } else if (a.khalf && a.vhalf) {
        e = launch(attention_wide_kernel<NDV, true, true>);
    } else if (a.khalf) {
        e = launch(attention_wide_kernel<NDV, true, false>);
    } else if (a.vhalf) {
        e = launch(attention_wide_kernel<NDV, false, true>);
    } else {
        e = launch(attention_wide_kernel<NDV, false, false>);
    }
    if (e != hipSuccess || w.splits == 1) return e;
    SDHIP_LAUNCH(attention_combine_kernel, dim3(static_cast<uint32_t>(ceil_div(a.b * a.h * a.lq, 4))),
                 dim3(256), 0, stream, a, w.splits, part);
    return hipGetLastError();
}

template <int NDV>
hipError_t launch_ndv(AttentionArgs a, hipStream_t stream) {
    a.ldv = 16 * NDV + 4;
    const size_t lds = sizeof(float) * (kQueries * a.ldq + kKeys * a.ldk + kKeys * a.ldv);
    dim3 grid(static_cast<uint32_t>(a.qblocks * a.h * a.b)), block(256);
    if (a.khalf && a.vhalf) {
        SDHIP_LAUNCH((attention_kernel<NDV, true, true>), grid, block, lds, stream, a);
    } else if (a.khalf) {
        SDHIP_LAUNCH((attention_kernel<NDV, true, false>), grid, block, lds, stream, a);
    } else if (a.vhalf) {
        SDHIP_LAUNCH((attention_kernel<NDV, false, true>), grid, block, lds, stream, a);
    } else {
        SDHIP_LAUNCH((attention_kernel<NDV, false, false>), grid, block, lds, stream, a);
    }
    return hipGetLastError();
}

}  // namespace

size_t attention_lds_bytes(int64_t d, int64_t dv) {
    const int64_t dp = round_up(d, 4);
    return sizeof(float) * static_cast<size_t>(kQueries * (dp + 1) + kKeys * (dp + 1) + kKeys * (16 * 16 + 4));
}

size_t attention_work_bytes(const AttentionArgs &a) {
    if (a.lq == 0 || a.h == 0 || a.b == 0 || a.lk == 0) return 0;
    if (split_form(a)) return split_form_work(a);
    if (wide_form(a)) {
        const WideSplits w = wide_splits(a);
        return w.splits > 1 ? static_cast<size_t>(a.b * a.h * w.splits * a.lq * (12 + 4 * a.dv)) : 0;
    }
    return 0;
}

hipError_t launch_attention(AttentionArgs a, void *work, hipStream_t stream) {
    if (a.lq == 0 || a.h == 0 || a.b == 0) return hipSuccess;  // no output
    if (split_form(a)) return launch_split_form(a, work, stream);
    if (fast_form(a) && tuning().attention_generic == 0 && !a.bf16) return launch_fast_form(a, stream);
    a.dp = static_cast<int>(round_up(a.d, 4));
    a.ldq = a.dp + 1;
    a.ldk = a.dp + 1;
    const int ndv = static_cast<int>(ceil_div(a.dv, 16));
    a.qblocks = ceil_div(a.lq, kQueries);
    KernelScope scope("attention", stream);
    if (wide_form(a)) {
        if (ndv <= 16) return launch_wide<16>(a, work, stream);
        if (ndv <= 24) return launch_wide<24>(a, work, stream);
        return launch_wide<32>(a, work, stream);
    }
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
