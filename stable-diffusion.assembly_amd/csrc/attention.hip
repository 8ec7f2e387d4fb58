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

template <int D, int QT, int KB>
hipError_t launch_fast(AttentionArgs a, hipStream_t stream) {
    using F = Fast<D, QT, KB>;
    a.qblocks = ceil_div(a.lq, F::kQueries);
    const size_t lds = sizeof(float) * 2 * F::kBuffer;
    dim3 grid(static_cast<uint32_t>(a.qblocks * a.h * a.b)), block(256);
    KernelScope scope("attention", stream);
    hipLaunchKernelGGL((attention_fast_kernel<D, QT, KB>), grid, block, lds, stream, a);
    return hipGetLastError();
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Whether the fast form takes the operands: single-precision keys and values
// of d = dv dimensions, an instantiated head size, float4-aligned rows.
bool fast_form(const AttentionArgs &a) {
    const bool size = a.d == 32 || a.d == 40 || a.d == 64 || a.d == 80 || a.d == 96 || a.d == 128 || a.d == 160;
    return size && a.d == a.dv && !a.khalf && !a.vhalf && aligned16(a.k) && aligned16(a.v) && aligned16(a.y) &&
           a.knb1 % 4 == 0 && a.knb2 % 4 == 0 && a.knb3 % 4 == 0 && a.vnb1 % 4 == 0 && a.vnb2 % 4 == 0 &&
           a.vnb3 % 4 == 0 && a.ynb1 % 4 == 0 && a.ynb2 % 4 == 0 && a.ynb3 % 4 == 0;
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
    if (a.lq == 0 || a.h == 0 || a.b == 0) return hipSuccess;  // no output
    if (fast_form(a) && tuning().attention_generic == 0) return launch_fast_form(a, stream);
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
