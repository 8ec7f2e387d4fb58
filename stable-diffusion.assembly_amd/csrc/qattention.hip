// Self-attention with quantized products, the bits mode of FLASH_ATTN_EXT
// (attention.cc:597-824), on gfx950's integer MFMA, v_mfma_i32_16x16x64_i8.
//
// Quantization, bit for bit as the reference's C++ form does it (quant.cc):
//   keys, signed, one group over the head's dimensions (over_dims,
//     attention.cc:632-637: 4 ceil(d / 4) numbers): s = max |k| / wmax,
//     q = clamp(rint(k / s), -wmax, wmax), offset = s * sum(q);
//   queries, unsigned with a zero point, one group likewise; their scale and
//     offset then multiplied by the softmax's scale (attention.cc:754-764);
//   values, signed, per (dimension, group of keys) (over_keys, 639-643);
//   exponentials, unsigned with a zero point, per (query, group of keys).
// The scores are the quantized products scaled back as quant.cc:150-155 does,
// t = fma(sa sb, S, 0), t = fma(-oa, ob, t); their maximum per query over
// every key (the first pass); then, group by group in key order (the second
// pass), the scores again (the same integers and roundings), their
// exponentials exp(s - max) -- Cephes' form (scalar_math.h:34-51), and for
// the keys past the last multiple of 8 of the last stretch of key_block keys,
// the correctly rounded exp the reference's std::exp gives (attention.cc:288-
// 301) -- summed in double, quantized, and the group's product with the
// values added to the output, t = fma(sa sb, S, t), t = fma(-oa, ob, t).  The
// output is t * float(1 / sum).
//
// The MFMA multiplies signed bytes: the unsigned operands (queries,
// exponentials) are stored as q - 128 and the integer sums restored exactly
// as S = sum((q - 128) w) + 128 sum(w), sum(w) the signed operand's integer
// sum over the group.
//
// A workgroup of 4 waves takes 64 queries of one head, a wave 16.  The
// scores are computed transposed, keys by queries: lane (query lr, lg) holds
// keys 16 kt + 4 lg + r of each tile of 16.  The exponentials' bytes of a
// group are then already where the product with the values wants them, as
// operand B of 64 keys: lane lg's 16 bytes are positions 16 lg + 4 kt + r --
// the values' bytes are stored in that order (position p = 64 c + 16 kg +
// 4 kt + r holds key 64 c + 16 kt + 4 kg + r of the group).

#include "attention.h"
#include "host.h"
#include "profile.h"

namespace sdhip {

namespace {

__device__ __forceinline__ float qa_clamp(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

__device__ __forceinline__ float load_num(const void *p, int64_t at, bool half) {
    if (half) return static_cast<float>(static_cast<const _Float16 *>(p)[at]);
    return static_cast<const float *>(p)[at];
}

// ------------------------------------------------------------------ operands

// The three quantizers run as one launch: first the values' blocks, then the
// keys', then the queries'.  A key or a query takes 16 lanes, each lane 4
// consecutive numbers of every 64 of the slot (sd <= 64 kQaSteps), held in
// registers between the group's maximum and its quantization; the maxima and
// the integer sums are exact whatever the order of their reductions.
constexpr int kQaLanes = 16;
constexpr int kQaSteps = 8;  // the most 64-byte steps of a slot (sd <= 512)
constexpr int kQaItems = 256 / kQaLanes;

__device__ __forceinline__ float qa_lanes_max(float v) {
#pragma unroll
    for (int off = kQaLanes / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ float qa_lanes_min(float v) {
#pragma unroll
    for (int off = kQaLanes / 2; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ int qa_lanes_sum(int v) {
#pragma unroll
    for (int off = kQaLanes / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Numbers e .. e + 3 of the row at element `base` of p, zeros from `limit`:
// one 16-byte load where the four are single precision, inside the row and
// 16-byte aligned.
__device__ __forceinline__ void qa_load4(const void *p, int64_t base, int64_t e, int64_t limit, bool half,
                                         float (&x)[4]) {
    const float *f = half ? nullptr : static_cast<const float *>(p) + base + e;
    if (!half && e + 4 <= limit && (reinterpret_cast<uintptr_t>(f) & 15) == 0) {
        const float4v v = *reinterpret_cast<const float4v *>(f);
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = v[r];
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) x[r] = e + r < limit ? load_num(p, base + e + r, half) : 0.0f;
    }
}

__device__ __forceinline__ uint32_t qa_byte(int q, int r) { return static_cast<uint32_t>(q & 0xff) << (8 * r); }

// Keys: 16 a block, each over its sd slot (zeros past d), its scale, offset
// and integer sum.  Keys from lk to lkp: zeros.
__device__ __forceinline__ void qa_keys_block(const QAttentionArgs &a, int64_t blk) {
    const int64_t item = blk * kQaItems + (threadIdx.x / kQaLanes);
    if (item >= a.b * a.hk * a.lkp) return;
    const int l = threadIdx.x % kQaLanes;
    const int64_t j = item % a.lkp;
    const int64_t head = item / a.lkp;  // bi * hk + kh
    const int64_t bi = head / a.hk, kh = head % a.hk;
    const bool valid = j < a.lk;
    const int64_t base = bi * a.knb3 + kh * a.knb2 + (valid ? j : 0) * a.knb1;
    const int64_t limit = valid ? a.d : 0;
    const int steps = static_cast<int>(a.sd / 64);
    float x[kQaSteps][4] = {};
    float m = 0.0f;
#pragma unroll
    for (int st = 0; st < kQaSteps; ++st) {
        if (st < steps) {
            qa_load4(a.k, base, 64 * st + 4 * l, limit, a.khalf, x[st]);
#pragma unroll
            for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(x[st][r]));
        }
    }
    m = qa_lanes_max(m);
    const float wmax = static_cast<float>(a.wmax);
    const float s = __fdiv_rn(m, wmax);
    const float inverse = s > 0.0f ? __fdiv_rn(1.0f, s) : 0.0f;
    int sum = 0;
    int8_t *dst = a.kq + item * a.sd;
#pragma unroll
    for (int st = 0; st < kQaSteps; ++st) {
        if (st < steps) {
            const int64_t e = 64 * st + 4 * l;
            uint32_t word = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int q = 0;
                if (e + r < limit) q = static_cast<int>(qa_clamp(rintf(__fmul_rn(x[st][r], inverse)), -wmax, wmax));
                word |= qa_byte(q, r);
                sum += q;
            }
            *reinterpret_cast<uint32_t *>(dst + e) = word;
        }
    }
    sum = qa_lanes_sum(sum);
    if (l == 0) {
        a.ks[item] = s;
        a.ko[item] = __fmul_rn(s, static_cast<float>(sum));
        a.ksum[item] = sum;
    }
}

// Values: a block per (image, key head, group of keys, 64 dimensions), per
// (dimension, group) the group's bytes in the order of operand A (below), its
// scale, offset and integer sum, stored [head][group][dvp].  Keys past lk and
// dimensions past dv: zeros.  A wave takes 16 dimensions, a lane one of them
// and every fourth run of 4 consecutive keys of the slot: key w = 64 chunk +
// 16 kt + 4 kg + r sits at position p = 64 chunk + 16 kg + 4 kt + r, so that a
// run's 4 bytes are one word.  Slots of up to 256 keys are held in registers
// between the group's maximum and its quantization; longer ones (groups of up
// to 1024 keys) are read twice.
constexpr int kQaRuns = 256 / 16;  // the most runs a lane holds (slot <= 256)

__device__ __forceinline__ int64_t qa_value_position(int64_t w0) {
    return (w0 & ~63) + 16 * ((w0 >> 2) & 3) + 4 * ((w0 >> 4) & 3);
}

__device__ __forceinline__ void qa_values_block_long(const QAttentionArgs &a, int64_t blk) {
    const int64_t chunks = (a.dvp + 63) / 64;
    const int64_t cc = blk % chunks;
    const int64_t rest = blk / chunks;
    const int64_t g = rest % a.groups;
    const int64_t head = rest / a.groups;
    const int64_t bi = head / a.hk, kh = head % a.hk;
    const int lane = threadIdx.x & 63;
    const int64_t c = cc * 64 + (threadIdx.x >> 6) * 16 + (lane & 15);
    const int rg = lane >> 4;
    const int runs = static_cast<int>(a.slot / 16);
    const bool dim = c < a.dv;
    const int64_t base = bi * a.vnb3 + kh * a.vnb2 + (dim ? c : 0);
    const auto load_run = [&](int i, float (&x)[4]) {
        const int64_t w0 = 4 * (rg + 4 * i);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t key = g * a.group + w0 + r;
            x[r] = dim && w0 + r < a.group && key < a.lk ? load_num(a.v, base + key * a.vnb1, a.vhalf) : 0.0f;
        }
    };
    float m = 0.0f;
    for (int i = 0; i < runs; ++i) {
        float x[4];
        load_run(i, x);
#pragma unroll
        for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(x[r]));
    }
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    const float wmax = static_cast<float>(a.wmax);
    const float s = __fdiv_rn(m, wmax);
    const float inverse = s > 0.0f ? __fdiv_rn(1.0f, s) : 0.0f;
    int sum = 0;
    int8_t *dst = a.vq + ((head * a.dvp + c) * a.groups + g) * a.slot;
    for (int i = 0; i < runs; ++i) {
        float x[4];
        load_run(i, x);
        uint32_t word = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int q = static_cast<int>(qa_clamp(rintf(__fmul_rn(x[r], inverse)), -wmax, wmax));
            word |= qa_byte(q, r);
            sum += q;
        }
        if (c < a.dvp) *reinterpret_cast<uint32_t *>(dst + qa_value_position(4 * (rg + 4 * i))) = word;
    }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    if (rg == 0 && c < a.dvp) {
        const int64_t at = (head * a.groups + g) * a.dvp + c;
        a.vs[at] = s;
        a.vo[at] = __fmul_rn(s, static_cast<float>(sum));
        a.vsum[at] = sum;
    }
}

__device__ __forceinline__ void qa_values_block(const QAttentionArgs &a, int64_t blk) {
    const int64_t chunks = (a.dvp + 63) / 64;
    const int64_t cc = blk % chunks;
    const int64_t rest = blk / chunks;
    const int64_t g = rest % a.groups;
    const int64_t head = rest / a.groups;
    const int64_t bi = head / a.hk, kh = head % a.hk;
    const int lane = threadIdx.x & 63;
    const int64_t c = cc * 64 + (threadIdx.x >> 6) * 16 + (lane & 15);
    const int rg = lane >> 4;  // runs rg, rg + 4, ...
    const int runs = static_cast<int>(a.slot / 16);
    const bool dim = c < a.dv;
    const int64_t base = bi * a.vnb3 + kh * a.vnb2 + (dim ? c : 0);
    float x[kQaRuns][4] = {};
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < kQaRuns; ++i) {
        if (i < runs) {
            const int64_t w0 = 4 * (rg + 4 * i);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t key = g * a.group + w0 + r;
                if (dim && w0 + r < a.group && key < a.lk) x[i][r] = load_num(a.v, base + key * a.vnb1, a.vhalf);
                m = fmaxf(m, fabsf(x[i][r]));
            }
        }
    }
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    const float wmax = static_cast<float>(a.wmax);
    const float s = __fdiv_rn(m, wmax);
    const float inverse = s > 0.0f ? __fdiv_rn(1.0f, s) : 0.0f;
    int sum = 0;
    int8_t *dst = a.vq + ((head * a.dvp + c) * a.groups + g) * a.slot;
#pragma unroll
    for (int i = 0; i < kQaRuns; ++i) {
        if (i < runs) {
            const int64_t w0 = 4 * (rg + 4 * i);
            uint32_t word = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int q = static_cast<int>(qa_clamp(rintf(__fmul_rn(x[i][r], inverse)), -wmax, wmax));
                word |= qa_byte(q, r);
                sum += q;
            }
            if (c < a.dvp) *reinterpret_cast<uint32_t *>(dst + qa_value_position(w0)) = word;
        }
    }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    if (rg == 0 && c < a.dvp) {
        const int64_t at = (head * a.groups + g) * a.dvp + c;
        a.vs[at] = s;
        a.vo[at] = __fmul_rn(s, static_cast<float>(sum));
        a.vsum[at] = sum;
    }
}

// Queries: 16 a block, each over its sd slot as q - 128 (the group's tail past
// d its zero point, the slot past the group 0: the keys' bytes there are 0),
// its scale and offset times the softmax's scale.  Queries from lq to lqp:
// zeros.
__device__ __forceinline__ void qa_queries_block(const QAttentionArgs &a, int64_t blk) {
    const int64_t item = blk * kQaItems + (threadIdx.x / kQaLanes);
    if (item >= a.b * a.h * a.lqp) return;
    const int l = threadIdx.x % kQaLanes;
    const int64_t i = item % a.lqp;
    const int64_t head = item / a.lqp;  // bi * h + hh
    const int64_t bi = head / a.h, hh = head % a.h;
    const bool valid = i < a.lq;
    const int64_t base = bi * a.qnb3 + hh * a.qnb2 + (valid ? i : 0) * a.qnb1;
    const int64_t limit = valid ? a.d : 0;
    const int steps = static_cast<int>(a.sd / 64);
    float x[kQaSteps][4] = {};
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int st = 0; st < kQaSteps; ++st) {
        if (st < steps) {
            qa_load4(a.q, base, 64 * st + 4 * l, limit, false, x[st]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                lo = fminf(lo, x[st][r]);
                hi = fmaxf(hi, x[st][r]);
            }
        }
    }
    lo = qa_lanes_min(lo);
    hi = qa_lanes_max(hi);
    const float levels = static_cast<float>(a.levels);
    const float s = __fdiv_rn(__fsub_rn(hi, lo), levels);
    const float inverse = s > 0.0f ? __fdiv_rn(1.0f, s) : 0.0f;
    const float zero = rintf(__fmul_rn(-lo, inverse));
    int8_t *dst = a.qq + item * a.sd;
#pragma unroll
    for (int st = 0; st < kQaSteps; ++st) {
        if (st < steps) {
            const int64_t e = 64 * st + 4 * l;
            uint32_t word = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float q = 128.0f;
                if (e + r < a.d) {
                    q = qa_clamp(__fadd_rn(rintf(__fmul_rn(x[st][r], inverse)), zero), 0.0f, levels);
                } else if (e + r < a.gd) {
                    q = zero;
                }
                word |= qa_byte(static_cast<int>(q) - 128, r);
            }
            *reinterpret_cast<uint32_t *>(dst + e) = word;
        }
    }
    if (l == 0) {
        a.qs[item] = __fmul_rn(s, a.scale);
        a.qo[item] = __fmul_rn(__fmul_rn(s, zero), a.scale);
    }
}

struct QaOperandBlocks {
    int64_t values, keys, queries;
};

QaOperandBlocks qa_operand_blocks(const QAttentionArgs &a) {
    return {a.b * a.hk * a.groups * ceil_div(a.dvp, 64), ceil_div(a.b * a.hk * a.lkp, kQaItems),
            ceil_div(a.b * a.h * a.lqp, kQaItems)};
}

__global__ __launch_bounds__(256) void qa_operands_kernel(QAttentionArgs a, QaOperandBlocks n) {
    const int64_t blk = blockIdx.x;
    if (blk < n.values) {
        if (a.slot <= 16 * kQaRuns) {
            qa_values_block(a, blk);
        } else {
            qa_values_block_long(a, blk);
        }
    } else if (blk < n.values + n.keys) {
        qa_keys_block(a, blk - n.values);
    } else {
        qa_queries_block(a, blk - n.values - n.keys);
    }
}

// ------------------------------------------------------------------ attention

// The scores of the 16 keys j0 .. j0 + 15 (j0 a multiple of 4; the lane's
// are j0 + 4 lg + r) for the lane's query: the integer products over the sd
// bytes, restored, and scaled back.
template <int SUBS>
__device__ __forceinline__ float4v qa_scores(const QAttentionArgs &a, const int8_t *kq, const float *ks,
                                             const float *ko, const int32_t *ksum, const int4v (&qb)[SUBS],
                                             float qs, float qo, int64_t j0, int lr, int lg) {
    int4v acc = int4v{};
    const int8_t *krow = kq + (j0 + lr) * a.sd + 16 * lg;
#pragma unroll
    for (int sub = 0; sub < SUBS; ++sub) {
        const int4v av = *reinterpret_cast<const int4v *>(krow + 64 * sub);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, qb[sub], acc, 0, 0, 0);
    }
    const int64_t j = j0 + 4 * lg;
    const float4v s4 = *reinterpret_cast<const float4v *>(ks + j);
    const float4v o4 = *reinterpret_cast<const float4v *>(ko + j);
    const int4v n4 = *reinterpret_cast<const int4v *>(ksum + j);
    float4v out;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float sum = static_cast<float>(acc[r] + 128 * n4[r]);
        float t = __builtin_fmaf(__fmul_rn(s4[r], qs), sum, 0.0f);
        out[r] = __builtin_fmaf(-o4[r], qo, t);
    }
    return out;
}

// A workgroup per (64 queries, head, image, chunk of up to 256 dimensions of
// the values); NDV the most tiles of 16 dimensions of a chunk the instance
// takes.  A group of keys is taken a part of 16 GT keys at a time (GT tiles
// of 16): groups of up to 16 GT keys in one part, their exponentials held in
// registers from their quantization's statistics to their product; longer
// groups (16 GT = 256) in parts computed twice, once for the group's
// statistics and sum, once for the product.
template <int SUBS, int NDV, int GT, bool LONG>
__global__ __launch_bounds__(256) void qa_attention_kernel(QAttentionArgs a) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    constexpr int64_t kPart = 16 * GT;

    const uint32_t blk = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint32_t qb_ = blk % static_cast<uint32_t>(a.qblocks);
    const uint32_t rest = blk / static_cast<uint32_t>(a.qblocks);
    const uint32_t bh = rest % static_cast<uint32_t>(a.h * a.b);
    const int64_t c0 = static_cast<int64_t>(rest / static_cast<uint32_t>(a.h * a.b)) * a.dvc;  // the chunk's first dimension
    const int64_t hh = bh % a.h;
    const int64_t bi = bh / a.h;
    const int64_t kh = hh / (a.h / a.hk);
    const int64_t head_k = bi * a.hk + kh;
    const int64_t i0 = static_cast<int64_t>(qb_) * 64 + wave * 16;  // the wave's first query
    const int64_t qrow = (bi * a.h + hh) * a.lqp + i0 + lr;        // the lane's query, in qq / qs / qo

    // Operand B of the scores: the lane's query, bytes 64 sub + 16 lg.
    int4v qbv[SUBS];
#pragma unroll
    for (int sub = 0; sub < SUBS; ++sub)
        qbv[sub] = *reinterpret_cast<const int4v *>(a.qq + qrow * a.sd + 64 * sub + 16 * lg);
    const float qs = a.qs[qrow], qo = a.qo[qrow];

    const int8_t *kq = a.kq + head_k * a.lkp * a.sd;
    const float *ks = a.ks + head_k * a.lkp;
    const float *ko = a.ko + head_k * a.lkp;
    const int32_t *ksum = a.ksum + head_k * a.lkp;

    // First pass: the greatest score of each query over the keys.
    // Tiles wholly of keys take no test per key, four at a time with every
    // load of the four issued first.
    float top = -INFINITY;
    const int64_t whole = a.lk / 16;
    const int64_t tiles = (a.lk + 15) / 16;
    int64_t kt0 = 0;
    for (; kt0 + 4 <= whole; kt0 += 4) {
        float4v sc[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) sc[u] = qa_scores<SUBS>(a, kq, ks, ko, ksum, qbv, qs, qo, 16 * (kt0 + u), lr, lg);
#pragma unroll
        for (int u = 0; u < 4; ++u) top = fmaxf(fmaxf(top, fmaxf(sc[u][0], sc[u][1])), fmaxf(sc[u][2], sc[u][3]));
    }
    for (int64_t kt = kt0; kt < tiles; ++kt) {
        const float4v sc = qa_scores<SUBS>(a, kq, ks, ko, ksum, qbv, qs, qo, 16 * kt, lr, lg);
        if (kt < whole) {
            top = fmaxf(fmaxf(top, fmaxf(sc[0], sc[1])), fmaxf(sc[2], sc[3]));
            continue;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (16 * kt + 4 * lg + r < a.lk) top = fmaxf(top, sc[r]);
    }
    top = fmaxf(top, __shfl_xor(top, 16, 64));
    top = fmaxf(top, __shfl_xor(top, 32, 64));

    // Second pass, group by group, over the chunk's ndv tiles of dimensions.
    const int64_t left = (a.dvp - c0) / 16;
    const int ndv = static_cast<int>(left < NDV ? left : NDV);
    float t[NDV][4];
#pragma unroll
    for (int c = 0; c < NDV; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) t[c][r] = 0.0f;
    double total = 0.0;
    const float levels = static_cast<float>(a.levels);
    const int8_t *vq = a.vq + (head_k * a.dvp + c0) * a.groups * a.slot;
    const float *vs = a.vs + head_k * a.groups * a.dvp + c0;
    const float *vo = a.vo + head_k * a.groups * a.dvp + c0;
    const int32_t *vsum = a.vsum + head_k * a.groups * a.dvp + c0;
    const int parts = LONG ? static_cast<int>((a.group + kPart - 1) / kPart) : 1;
    for (int64_t g = 0; g < a.groups; ++g) {
        const int64_t gbase = g * a.group;
        // The exponentials of part p of the group: tile kt, keys gbase + p
        // kPart + 16 kt + 4 lg + r, zero past the group and past lk; with
        // `stats` their sum, least and greatest taken too.
        float e[GT][4];
        float lo = 0.0f, hi = 0.0f;
        const auto exps = [&](int p, bool stats) {
            const int64_t rel0 = p * kPart;
            const int64_t end = gbase + rel0 + kPart;
            const bool plain = a.group % 16 == 0 && rel0 + kPart <= a.group && end <= a.lk && end <= a.tail_from;
            if (plain) {
                // Whole tiles of keys, none past tail_from: every tile's
                // scores (their loads issued together), then Cephes'
                // exponential of each in one straight run, then the
                // statistics in the order of the keys.
                float4v sc[GT];
#pragma unroll
                for (int kt = 0; kt < GT; ++kt)
                    sc[kt] = qa_scores<SUBS>(a, kq, ks, ko, ksum, qbv, qs, qo, gbase + rel0 + 16 * kt, lr, lg);
#pragma unroll
                for (int kt = 0; kt < GT; ++kt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) e[kt][r] = cephes_exp(__fsub_rn(sc[kt][r], top));
                if (stats) {
#pragma unroll
                    for (int kt = 0; kt < GT; ++kt)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            total += static_cast<double>(e[kt][r]);
                            lo = fminf(lo, e[kt][r]);
                            hi = fmaxf(hi, e[kt][r]);
                        }
                }
                return;
            }
#pragma unroll
            for (int kt = 0; kt < GT; ++kt) {
                const int64_t rel = rel0 + 16 * kt;  // the tile's first key, in the group
                if (rel >= a.group || gbase + rel >= a.lk) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) e[kt][r] = 0.0f;
                    continue;
                }
                const float4v sc = qa_scores<SUBS>(a, kq, ks, ko, ksum, qbv, qs, qo, gbase + rel, lr, lg);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t jr = rel + 4 * lg + r;
                    const int64_t j = gbase + jr;
                    const bool key = jr < a.group && j < a.lk;
                    float x = 0.0f;
                    if (key) {
                        const float arg = __fsub_rn(sc[r], top);
                        x = j < a.tail_from ? cephes_exp(arg) : static_cast<float>(exp(static_cast<double>(arg)));
                    }
                    if (stats && key) {
                        total += static_cast<double>(x);
                        lo = fminf(lo, x);
                        hi = fmaxf(hi, x);
                    }
                    e[kt][r] = x;
                }
            }
        };
        for (int p = 0; p < parts; ++p) exps(p, true);
        lo = fminf(lo, __shfl_xor(lo, 16, 64));
        lo = fminf(lo, __shfl_xor(lo, 32, 64));
        hi = fmaxf(hi, __shfl_xor(hi, 16, 64));
        hi = fmaxf(hi, __shfl_xor(hi, 32, 64));
        const float es = __fdiv_rn(__fsub_rn(hi, lo), levels);
        const float inverse = es > 0.0f ? __fdiv_rn(1.0f, es) : 0.0f;
        const float zero = rintf(__fmul_rn(-lo, inverse));
        const float eo = __fmul_rn(es, zero);

        // The group's product with the values, 64 keys (four tiles) at a time,
        // over the group's slot.
        int4v acc[NDV];
#pragma unroll
        for (int c = 0; c < NDV; ++c) acc[c] = int4v{};
        for (int p = 0; p < parts; ++p) {
            if (LONG) exps(p, false);  // a long group's part again: the same exponentials
#pragma unroll
            for (int chunk = 0; chunk < (GT + 3) / 4; ++chunk) {
                const int64_t pos = p * kPart + 64 * chunk;  // the chunk's first position in the slot
                if (pos >= a.slot) continue;
                // The bytes q - 128 of the quantized exponentials (q an
                // integer in [0, 255]): q packed as an unsigned byte, its top
                // bit flipped.
                int4v bv;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    uint32_t word = 0;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int kt = 4 * chunk + w;
                        float q = 0.0f;
                        if (kt < GT) q = qa_clamp(__fadd_rn(rintf(__fmul_rn(e[kt][r], inverse)), zero), 0.0f, levels);
                        word = __builtin_amdgcn_cvt_pk_u8_f32(q, r, word);
                    }
                    bv[w] = static_cast<int>(word ^ 0x80808080u);
                }
                // Positions of the slot past the group's keys hold value
                // bytes of 0, which the exponentials' bytes there multiply.
#pragma unroll
                for (int c = 0; c < NDV; ++c) {
                    if (c >= ndv) continue;
                    const int4v av =
                        *reinterpret_cast<const int4v *>(vq + ((16 * c + lr) * a.groups + g) * a.slot + pos + 16 * lg);
                    acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, acc[c], 0, 0, 0);
                }
            }
        }
        // Scaled back into the output, dimensions c0 + 16 c + 4 lg + r.
#pragma unroll
        for (int c = 0; c < NDV; ++c) {
            if (c >= ndv) continue;
            const int64_t at = g * a.dvp + 16 * c + 4 * lg;
            const float4v s4 = *reinterpret_cast<const float4v *>(vs + at);
            const float4v o4 = *reinterpret_cast<const float4v *>(vo + at);
            const int4v n4 = *reinterpret_cast<const int4v *>(vsum + at);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float sum = static_cast<float>(acc[c][r] + 128 * n4[r]);
                t[c][r] = __builtin_fmaf(__fmul_rn(s4[r], es), sum, t[c][r]);
                t[c][r] = __builtin_fmaf(-o4[r], eo, t[c][r]);
            }
        }
    }

    total += __shfl_xor(total, 16, 64);
    total += __shfl_xor(total, 32, 64);
    const float reciprocal = static_cast<float>(1.0 / total);
    const int64_t i = i0 + lr;
    if (i >= a.lq) return;
    float *out = a.y + bi * a.ynb3 + i * a.ynb2 + hh * a.ynb1 + c0;
#pragma unroll
    for (int c = 0; c < NDV; ++c) {
        if (c >= ndv) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t dim = 16 * c + 4 * lg + r;
            if (c0 + dim < a.dv) out[dim] = __fmul_rn(t[c][r], reciprocal);
        }
    }
}

template <int SUBS, int NDV>
hipError_t launch_qa_gt(const QAttentionArgs &a, hipStream_t stream, dim3 grid) {
    const int64_t gt = (a.group + 15) / 16;
    if (gt <= 4) {
        SDHIP_LAUNCH((qa_attention_kernel<SUBS, NDV, 4, false>), grid, dim3(256), 0, stream, a);
    } else if (gt <= 8) {
        SDHIP_LAUNCH((qa_attention_kernel<SUBS, NDV, 8, false>), grid, dim3(256), 0, stream, a);
    } else if (gt <= 16) {
        SDHIP_LAUNCH((qa_attention_kernel<SUBS, NDV, 16, false>), grid, dim3(256), 0, stream, a);
    } else {
        // Groups of more than 256 keys, in parts of 256.
        SDHIP_LAUNCH((qa_attention_kernel<SUBS, NDV, 16, true>), grid, dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

template <int SUBS>
hipError_t launch_qa_ndv(const QAttentionArgs &a, hipStream_t stream, dim3 grid) {
    // Instances of 2, 4, 8 and 16 tiles of dimensions (a chunk's tiles past
    // its own are skipped).  With parts of 256 keys the instance of 8 spills
    // its registers where that of 16 does not (the compiler's resource
    // usage): it takes those.
    const int64_t tiles = a.dvc / 16;
    if (tiles <= 2) return launch_qa_gt<SUBS, 2>(a, stream, grid);
    if (tiles <= 4) return launch_qa_gt<SUBS, 4>(a, stream, grid);
    if (tiles <= 8 && a.group <= 128) return launch_qa_gt<SUBS, 8>(a, stream, grid);
    return launch_qa_gt<SUBS, 16>(a, stream, grid);
}

}  // namespace

QAttentionLayout qattention_layout(QAttentionArgs &a) {
    a.gd = round_up(a.d, 4);
    // Slots of 1, 2, 4 or 8 steps of 64 bytes (the kernels' instances); the
    // bytes past gd are 0 in the keys and the queries.
    a.sd = round_up(a.gd, 64);
    if (a.sd == 192) a.sd = 256;
    if (a.sd > 256) a.sd = 512;
    a.groups = ceil_div(a.lk, a.group);
    // The keys' rows: a tile of 16 starting at any key of the last group (a
    // multiple of 4) stays inside them.
    a.lkp = round_up(a.groups * a.group + 15, 16);
    a.lqp = round_up(a.lq, 64);
    a.slot = round_up(a.group, 64);
    a.dvp = round_up(a.dv, 16);
    // The values' dimensions a workgroup takes: all of them up to 256, else
    // chunks of 256.
    a.dvc = a.dvp <= 256 ? a.dvp : 256;
    // Stretches of key_block keys (attention.cc:663-664); the keys past the
    // last multiple of 8 of the last one take std::exp (attention.cc:288-301).
    const int64_t last = (a.lk - 1) / a.key_block * a.key_block;
    a.tail_from = last + (a.lk - last) / 8 * 8;
    a.qblocks = ceil_div(a.lq, 64);
    QAttentionLayout l{};
    size_t at = 0;
    const auto take = [&](int64_t bytes) {
        const size_t here = at;
        at += static_cast<size_t>(round_up(bytes, 256));
        return here;
    };
    const int64_t heads_k = a.b * a.hk, heads = a.b * a.h;
    l.kq = take(heads_k * a.lkp * a.sd);
    l.ks = take(heads_k * a.lkp * 4);
    l.ko = take(heads_k * a.lkp * 4);
    l.ksum = take(heads_k * a.lkp * 4);
    l.vq = take(heads_k * a.dvp * a.groups * a.slot);
    l.vs = take(heads_k * a.groups * a.dvp * 4);
    l.vo = take(heads_k * a.groups * a.dvp * 4);
    l.vsum = take(heads_k * a.groups * a.dvp * 4);
    l.qq = take(heads * a.lqp * a.sd);
    l.qs = take(heads * a.lqp * 4);
    l.qo = take(heads * a.lqp * 4);
    l.total = at;
    return l;
}

hipError_t launch_quantized_attention(QAttentionArgs a, void *work, hipStream_t stream) {
    const QAttentionLayout l = qattention_layout(a);
    char *base = static_cast<char *>(work);
    a.kq = reinterpret_cast<int8_t *>(base + l.kq);
    a.ks = reinterpret_cast<float *>(base + l.ks);
    a.ko = reinterpret_cast<float *>(base + l.ko);
    a.ksum = reinterpret_cast<int32_t *>(base + l.ksum);
    a.vq = reinterpret_cast<int8_t *>(base + l.vq);
    a.vs = reinterpret_cast<float *>(base + l.vs);
    a.vo = reinterpret_cast<float *>(base + l.vo);
    a.vsum = reinterpret_cast<int32_t *>(base + l.vsum);
    a.qq = reinterpret_cast<int8_t *>(base + l.qq);
    a.qs = reinterpret_cast<float *>(base + l.qs);
    a.qo = reinterpret_cast<float *>(base + l.qo);
    {
        KernelScope scope("qattention.operands", stream);
        const QaOperandBlocks n = qa_operand_blocks(a);
        SDHIP_LAUNCH(qa_operands_kernel, dim3(static_cast<uint32_t>(n.values + n.keys + n.queries)), dim3(256), 0,
                     stream, a, n);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    KernelScope scope("qattention", stream);
    const dim3 grid(static_cast<uint32_t>(a.qblocks * a.h * a.b * ceil_div(a.dvp, a.dvc)));
    switch (a.sd / 64) {
    case 1: return launch_qa_ndv<1>(a, stream, grid);
    case 2: return launch_qa_ndv<2>(a, stream, grid);
    case 4: return launch_qa_ndv<4>(a, stream, grid);
    default: return launch_qa_ndv<8>(a, stream, grid);
    }
}

}  // namespace sdhip
