// The bits mode of the linear layers (quant.h, quant.cc, mul_mat.cc:378-646)
// on gfx950's integer MFMA.
//
// Quantization, bit for bit as the reference's C++ form does it:
//   inputs, per (row, group of k) (quant.cc:282-315): lo = min(0, min x),
//     hi = max(0, max x), s = (hi - lo) / levels, inv = s > 0 ? 1 / s : 0,
//     z = rint(-lo * inv), q = clamp(rint(x * inv) + z, 0, levels), the
//     group's tail the zero point z; offset = s * z;
//   weights, per (column, group) or per whole column (quant.cc:204-243):
//     s = max |w| / wmax, inv = s > 0 ? 1 / s : 0,
//     q = clamp(rint(w * inv), -wmax, wmax); offset = s * sum(q).
// Every operation is an IEEE one (correctly rounded division, round to
// nearest-even), so the bytes, scales and offsets are the reference's.
//
// Products: the MFMA multiplies signed bytes, so the inputs are stored as
// q - 128 and the group's integer sum restored exactly as
// S = sum((q - 128) w) + 128 sum(w).  Each group then adds to the output, in
// the reference's order and roundings (quant.cc:150-155):
//     t = fma(sa * sb, float(S), t);  t = fma(-oa, ob, t)
// so that the result is the reference's C++ result, bit for bit, when the
// sum starts from the same number (0, or the residual with from_redirect).
//
// Layout in the work buffer: each group of k padded to a slot (a multiple
// of 64 bytes, the MFMA's k), cut into steps of 64 bytes; the bytes held
// step-major, inputs [step][M][64] and weights [step][N][64], so that one
// step of 32 consecutive rows is 2 KB in a row; then the scales, offsets
// and (weights) integer sums, group-major, [groups][rows].

#include "host.h"
#include "profile.h"
#include "quant.h"

namespace sdhip {

namespace {

struct Quant {
    int group;  // numbers of k sharing a scale
    int levels;
    int wmax;
    int weight_groups;
};

Quant quant_of(const Tuning &t) {
    Quant q;
    int quads = t.group / 4;
    quads = quads < 1 ? 1 : (quads > 256 ? 256 : quads);
    q.group = 4 * quads;
    const int ib = t.input_bits < 2 ? 2 : (t.input_bits > 8 ? 8 : t.input_bits);
    const int wb = t.bits < 2 ? 2 : (t.bits > 8 ? 8 : t.bits);
    q.levels = (1 << ib) - 1;
    q.wmax = (1 << (wb - 1)) - 1;
    q.weight_groups = t.weight_group != 0;
    return q;
}

struct Layout {
    int64_t groups, slot, kp;  // groups of k, bytes a group takes, bytes a row takes
    int64_t m, n;              // rows of the inputs and of the weights
    size_t xq, xs, xo, wq, ws, wo, wsum, total;
};

Layout layout_of(int64_t K, int64_t N, int64_t M, const Quant &q) {
    Layout l{};
    l.groups = ceil_div(K, q.group);
    l.slot = round_up(q.group, 64);
    l.kp = l.groups * l.slot;
    l.m = M;
    l.n = N;
    size_t at = 0;
    const auto take = [&](size_t bytes) {
        const size_t here = at;
        at += static_cast<size_t>(round_up(static_cast<int64_t>(bytes), 256));
        return here;
    };
    l.xq = take(static_cast<size_t>(M * l.kp));
    l.xs = take(static_cast<size_t>(M * l.groups) * 4);
    l.xo = take(static_cast<size_t>(M * l.groups) * 4);
    l.wq = take(static_cast<size_t>(N * l.kp));
    l.ws = take(static_cast<size_t>(N * l.groups) * 4);
    l.wo = take(static_cast<size_t>(N * l.groups) * 4);
    l.wsum = take(static_cast<size_t>(N * l.groups) * 4);
    l.total = at;
    return l;
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ int wave_isum(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

// ------------------------------------------------------------------ inputs

// The rows of the inputs: x[m][k], rows ldx apart.
struct RowsSrc {
    const float *x;
    int64_t ldx;
    __device__ float operator()(int64_t m, int64_t k) const { return x[m * ldx + k]; }
};

// One wave per (row, group): the group's least and greatest (with 0), its
// scale and zero point, and its bytes, stored as q - 128.  Src gives the
// inputs' numbers: rows of x, or a convolution's columns.
template <class Src>
__global__ __launch_bounds__(256) void quantize_inputs_kernel(Src src, int64_t M, int64_t K, Quant q, Layout l,
                                                              int8_t *__restrict__ xq, float *__restrict__ xs,
                                                              float *__restrict__ xo) {
    const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (item >= M * l.groups) return;
    const int lane = threadIdx.x & 63;
    const int64_t m = item / l.groups;
    const int64_t g = item - m * l.groups;
    const int64_t k0 = g * q.group;
    const int64_t n = K - k0 < q.group ? K - k0 : q.group;
    const auto row = [&](int64_t e) { return src(m, k0 + e); };
    float lo = 0.0f, hi = 0.0f;
    for (int64_t e = lane; e < n; e += 64) {
        const float v = row(e);
        lo = fminf(lo, v);
        hi = fmaxf(hi, v);
    }
    lo = wave_min(lo);
    hi = wave_max(hi);
    const float levels = static_cast<float>(q.levels);
    const float s = __fdiv_rn(__fsub_rn(hi, lo), levels);
    const float inverse = s > 0.0f ? __fdiv_rn(1.0f, s) : 0.0f;
    const float zero = rintf(__fmul_rn(-lo, inverse));
    // Slot byte e: step g (slot / 64) + e / 64, byte e % 64.
    int8_t *dst = xq + (g * (l.slot / 64) * l.m + m) * 64;
    for (int64_t e = lane; e < l.slot; e += 64) {
        float v = 0.0f;
        if (e < n) {
            v = clampf(__fadd_rn(rintf(__fmul_rn(row(e), inverse)), zero), 0.0f, levels);
        } else if (e < q.group) {
            v = zero;  // the group's tail stands for zeros
        } else {
            v = 128.0f;  // the slot's padding: 0 after the shift, times a weight of 0
        }
        dst[(e >> 6) * l.m * 64 + (e & 63)] = static_cast<int8_t>(static_cast<int>(v) - 128);
    }
    if (lane == 0) {
        xs[g * l.m + m] = s;
        xo[g * l.m + m] = __fmul_rn(s, zero);
    }
}

// x from another lane of its row of 16 by a DPP move (CTRL: quad_perm 0x00
// .. 0xFF, row_mirror 0x140, row_half_mirror 0x141); every lane reads one.
template <int CTRL>
__device__ __forceinline__ float row_dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// The same quantizer for groups of 64 that fill their slots (K a multiple of
// 64, rows of x 16-byte aligned): 16 lanes a (row, group), each lane 4
// consecutive numbers (one 16-byte load), the least and greatest reduced
// over the 16 lanes, and the lane's 4 bytes written as one word -- a wave
// takes 4 groups, where the general kernel takes one, with no loop.  The
// same IEEE operations in the same order: the same bytes, scales and
// offsets.
__global__ __launch_bounds__(256) void quantize_inputs64_kernel(const float *__restrict__ x, int64_t ldx, int64_t M,
                                                                int64_t groups, float levels,
                                                                int8_t *__restrict__ xq, float *__restrict__ xs,
                                                                float *__restrict__ xo) {
    const int64_t seg = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 4;
    if (seg >= M * groups) return;
    const int j = threadIdx.x & 15;
    // Consecutive segments along the rows, so that a wave's bytes are
    // consecutive in xq ([group][row][64]).
    const int64_t g = seg / M;
    const int64_t m = seg - g * M;
    const float4v v = *reinterpret_cast<const float4v *>(x + m * ldx + 64 * g + 4 * j);
    float lo = fminf(fminf(fminf(0.0f, v[0]), fminf(v[1], v[2])), v[3]);
    float hi = fmaxf(fmaxf(fmaxf(0.0f, v[0]), fmaxf(v[1], v[2])), v[3]);
    // Over the 16 lanes of the segment (a DPP row) by DPP moves, no trip
    // through LDS: neighbours in the quad, the other pair of the quad, the
    // other quad of the half row (its mirror), the other half (the row's
    // mirror).  Least and greatest do not depend on the order.
    lo = fminf(lo, row_dpp<0xB1>(lo));
    hi = fmaxf(hi, row_dpp<0xB1>(hi));
    lo = fminf(lo, row_dpp<0x4E>(lo));
    hi = fmaxf(hi, row_dpp<0x4E>(hi));
    lo = fminf(lo, row_dpp<0x141>(lo));
    hi = fmaxf(hi, row_dpp<0x141>(hi));
    lo = fminf(lo, row_dpp<0x140>(lo));
    hi = fmaxf(hi, row_dpp<0x140>(hi));
    const float s = __fdiv_rn(__fsub_rn(hi, lo), levels);
    const float inverse = s > 0.0f ? __fdiv_rn(1.0f, s) : 0.0f;
    const float zero = rintf(__fmul_rn(-lo, inverse));
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float q = clampf(__fadd_rn(rintf(__fmul_rn(v[e], inverse)), zero), 0.0f, levels);
        word |= static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int>(q) - 128)) << (8 * e);
    }
    *reinterpret_cast<uint32_t *>(xq + (g * M + m) * 64 + 4 * j) = word;
    if (j == 0) {
        xs[g * M + m] = s;
        xo[g * M + m] = __fmul_rn(s, zero);
    }
}

// ------------------------------------------------------------------ weights

// One wave per column (a row of W): the whole row's greatest magnitude when
// the weights have one scale a row, then group by group the scale, the
// bytes and their sum.
// W: the weights' type, FP16 or single precision (quantize_weights_f16 and
// _f32, quant.cc:366-380: the same quantizer of their widened values).
// `stretch`, with one scale a row (weight_groups = 0): the stretches of k
// the row is quantized in, a multiple of the group, their scale the
// stretch's greatest (Winograd's weights, quantized a stretch of input
// channels at a time, winograd.cc:1917-1930); 0 for the whole row.
template <class W>
__global__ __launch_bounds__(256) void quantize_weights_kernel(const W *__restrict__ w, int64_t ldw, int64_t N,
                                                               int64_t K, Quant q, Layout l, int8_t *__restrict__ wq,
                                                               float *__restrict__ ws, float *__restrict__ wo,
                                                               int32_t *__restrict__ wsum, int64_t stretch) {
    const int64_t n = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    const int lane = threadIdx.x & 63;
    const W *row = w + n * ldw;
    float row_max = 0.0f;
    int64_t stretch_of = -1;  // the stretch row_max is of
    const float wmax = static_cast<float>(q.wmax);
    for (int64_t g = 0; g < l.groups; ++g) {
        const int64_t k0 = g * q.group;
        const int64_t cnt = K - k0 < q.group ? K - k0 : q.group;
        if (!q.weight_groups) {
            const int64_t st = stretch > 0 ? k0 / stretch : 0;
            if (st != stretch_of) {
                const int64_t s0 = stretch > 0 ? st * stretch : 0;
                const int64_t s1 = stretch > 0 && s0 + stretch < K ? s0 + stretch : K;
                float mm = 0.0f;
                for (int64_t e = s0 + lane; e < s1; e += 64) mm = fmaxf(mm, fabsf(static_cast<float>(row[e])));
                row_max = wave_max(mm);
                stretch_of = st;
            }
        }
        float m = row_max;
        if (q.weight_groups) {
            float mm = 0.0f;
            for (int64_t e = lane; e < cnt; e += 64) mm = fmaxf(mm, fabsf(static_cast<float>(row[k0 + e])));
            m = wave_max(mm);
        }
        const float s = __fdiv_rn(m, wmax);
        const float inverse = s > 0.0f ? __fdiv_rn(1.0f, s) : 0.0f;
        int8_t *dst = wq + (g * (l.slot / 64) * l.n + n) * 64;
        int sum = 0;
        for (int64_t e = lane; e < l.slot; e += 64) {
            int v = 0;
            if (e < cnt) {
                v = static_cast<int>(clampf(rintf(__fmul_rn(static_cast<float>(row[k0 + e]), inverse)), -wmax, wmax));
            }
            dst[(e >> 6) * l.n * 64 + (e & 63)] = static_cast<int8_t>(v);
            sum += v;
        }
        sum = wave_isum(sum);
        if (lane == 0) {
            ws[g * l.n + n] = s;
            wo[g * l.n + n] = __fmul_rn(s, static_cast<float>(sum));
            wsum[g * l.n + n] = sum;
        }
    }
}

// ------------------------------------------------------------------ products

// A block of 64 rows (tokens) by 64 columns (features) by 4 waves of 32 x 32,
// each 2 x 2 tiles of 16 x 16 on v_mfma_i32_16x16x64_i8; k a group's slot at
// a time through LDS, double-buffered.  After each group the lane's 16
// integer sums are scaled into its 16 single-precision outputs.  GATED: the
// block's 64 columns are 32 features of the first half and the same 32 of
// the second, each wave's two column tiles a pair (x, gate).
constexpr int kQB = 64;
constexpr int kQLd = 64 + 16;  // bytes per LDS row

struct QgemmArgs {
    const int8_t *xq, *wq;
    const float *xs, *xo, *ws, *wo;
    const int32_t *wsum;
    float *y;
    int64_t ldy;
    int64_t M, N, half;
    int64_t ne1, ne2;
    int64_t groups, slot, kp;
    int64_t xrows, wrows;  // rows of the layouts: the step and group strides (x 64 bytes, x 1)
    int64_t col_blocks;
    // qgemm3: the workgroups' order, along the rows of x within a column
    // block (row_blocks of them) where that reads less, else along the
    // column blocks within a row block.
    int64_t row_blocks;
    int32_t by_columns;
    int32_t from_redirect;
    DevChain chain;
};

template <bool GATED>
__global__ __launch_bounds__(256) void qgemm_kernel(QgemmArgs p) {
    __shared__ __attribute__((aligned(16))) int8_t la[2][kQB * kQLd];
    __shared__ __attribute__((aligned(16))) int8_t lb[2][kQB * kQLd];
    __shared__ float sa[2][kQB], oa[2][kQB], sb[2][kQB], ob[2][kQB];
    __shared__ int32_t qs[2][kQB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave >> 1, wc = wave & 1;
    const int lr = lane & 15, lg = lane >> 4;

    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t mb = b / p.col_blocks;
    const int64_t nb = b % p.col_blocks;
    const int64_t m0 = mb * kQB;
    const int64_t n0 = nb * (GATED ? kQB / 2 : kQB);
    // The global row of W that LDS row r of the block holds, or -1.
    const auto w_row = [&](int r) -> int64_t {
        if (GATED) {
            const int side = (r >> 4) & 1;
            const int64_t f = n0 + 16 * (r >> 5) + (r & 15);
            return f < p.half ? side * p.half + f : -1;
        }
        return n0 + r < p.N ? n0 + r : -1;
    };

    // Global loads: 64 rows x 64 bytes of each operand = 256 x 16 bytes, one
    // a thread each; the group's scales by the first threads.
    const int lrow = tid >> 2, lq = (tid & 3) * 16;
    const int64_t arow = m0 + lrow < p.M ? m0 + lrow : -1;
    const int64_t brow = w_row(lrow);
    int4v ra, rb;
    float rsa = 0.f, roa = 0.f, rsb = 0.f, rob = 0.f;
    int32_t rqs = 0;
    const auto load = [&](int64_t g, int64_t sub) {
        const int64_t step = g * (p.slot / 64) + sub;
        ra = arow >= 0 ? *reinterpret_cast<const int4v *>(p.xq + (step * p.xrows + arow) * 64 + lq) : int4v{};
        rb = brow >= 0 ? *reinterpret_cast<const int4v *>(p.wq + (step * p.wrows + brow) * 64 + lq) : int4v{};
        if (tid < kQB) {
            const int64_t r = m0 + tid;
            rsa = r < p.M ? p.xs[g * p.xrows + r] : 0.0f;
            roa = r < p.M ? p.xo[g * p.xrows + r] : 0.0f;
        } else if (tid < 2 * kQB) {
            const int64_t c = w_row(tid - kQB);
            rsb = c >= 0 ? p.ws[g * p.wrows + c] : 0.0f;
            rob = c >= 0 ? p.wo[g * p.wrows + c] : 0.0f;
            rqs = c >= 0 ? p.wsum[g * p.wrows + c] : 0;
        }
    };
    const auto store = [&](int buf) {
        *reinterpret_cast<int4v *>(&la[buf][lrow * kQLd + lq]) = ra;
        *reinterpret_cast<int4v *>(&lb[buf][lrow * kQLd + lq]) = rb;
        if (tid < kQB) {
            sa[buf][tid] = rsa;
            oa[buf][tid] = roa;
        } else if (tid < 2 * kQB) {
            sb[buf][tid - kQB] = rsb;
            ob[buf][tid - kQB] = rob;
            qs[buf][tid - kQB] = rqs;
        }
    };

    // The outputs: tile (i, j) of the wave, lane rows 4 lg + e, column lr.
    float t[2][2][4];
    if (!GATED && p.from_redirect) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int64_t n = n0 + wc * 32 + 16 * j + lr;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t m = m0 + wr * 32 + 16 * i + 4 * lg + e;
                    t[i][j][e] = (m < p.M && n < p.N) ? p.y[m * p.ldy + n] : 0.0f;
                }
            }
    } else {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) t[i][j][e] = 0.0f;
    }

    const int64_t subs = p.slot / 64;
    const int64_t steps = p.groups * subs;
    load(0, 0);
    store(0);
    __syncthreads();
    int4v acc[2][2];
    for (int64_t s = 0; s < steps; ++s) {
        const int cur = s & 1;
        const int64_t g = s / subs, sub = s - g * subs;
        if (s + 1 < steps) load((s + 1) / subs, (s + 1) % subs);
        if (sub == 0) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = int4v{};
        }
        int4v a[2], bv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            a[i] = *reinterpret_cast<const int4v *>(&la[cur][(wr * 32 + 16 * i + lr) * kQLd + 16 * lg]);
#pragma unroll
        for (int j = 0; j < 2; ++j)
            bv[j] = *reinterpret_cast<const int4v *>(&lb[cur][(wc * 32 + 16 * j + lr) * kQLd + 16 * lg]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], bv[j], acc[i][j], 0, 0, 0);
        if (sub == subs - 1) {
            // The group's sums into the outputs, as quant.cc:150-155 does.
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int col = wc * 32 + 16 * j + lr;
                const float cs = sb[cur][col], co = ob[cur][col];
                const int32_t shift = 128 * qs[cur][col];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int row = wr * 32 + 16 * i + 4 * lg + e;
                        const float ab = __fmul_rn(sa[cur][row], cs);
                        const float sum = static_cast<float>(acc[i][j][e] + shift);
                        float v = __builtin_fmaf(ab, sum, t[i][j][e]);
                        t[i][j][e] = __builtin_fmaf(-oa[cur][row], co, v);
                    }
            }
        }
        if (s + 1 < steps) store(cur ^ 1);
        __syncthreads();
    }

    // The chain, then the stores (or the gated GELU of the pair).
    const uint32_t ne1 = static_cast<uint32_t>(p.ne1), ne2 = static_cast<uint32_t>(p.ne2);
    const auto row_off = [&](const DevStep &st, int64_t m) -> int64_t {
        if (st.flat123) return m * st.nb[1];
        uint32_t i1, i2, i3;
        split_index(static_cast<uint32_t>(m), ne1, ne2, i1, i2, i3);
        return i1 * st.nb[1] + i2 * st.nb[2] + i3 * st.nb[3];
    };
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t mbase = m0 + wr * 32 + 16 * i + 4 * lg;
        const auto row = [&](int e) -> int64_t { return mbase + e < p.M ? mbase + e : p.M - 1; };
        if (GATED) {
            const int64_t f = n0 + 16 * wc + lr;
            const int64_t fc = f < p.half ? f : p.half - 1;
            float xv[4], gv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                xv[e] = t[i][0][e];
                gv[e] = t[i][1][e];
            }
            apply_chain_block(p.chain, xv, [&](int s, int e) {
                return fc * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e));
            });
            apply_chain_block(p.chain, gv, [&](int s, int e) {
                return (p.half + fc) * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e));
            });
            if (f >= p.half) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (mbase + e < p.M) p.y[(mbase + e) * p.ldy + f] = xv[e] * gelu(gv[e]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int64_t n = n0 + wc * 32 + 16 * j + lr;
                const int64_t nc = n < p.N ? n : p.N - 1;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = t[i][j][e];
                apply_chain_block(p.chain, v, [&](int s, int e) {
                    return nc * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e));
                });
                if (n >= p.N) continue;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (mbase + e < p.M) p.y[(mbase + e) * p.ldy + n] = v[e];
                }
            }
        }
    }
}

// The same products by wider tiles on v_mfma_i32_32x32x32_i8, fed by a ring
// of LDS stages.
//
// Per group a wave's MFMAs are few and its dequantisation long -- five VALU
// operations an output (the sums kept in VGPRs, no AGPR reads), the
// reference's fma order fixed by bit-exactness -- so the VALU bounds the
// kernel, and what matters is that every SIMD has work and that a wave's
// VALU overlaps another's MFMAs and loads: two workgroups a CU (at most 256
// registers a lane, 4 stages of LDS a workgroup).  The loads of a step are
// issued S - 1 steps ahead, straight into LDS by global_load_lds (no
// register staging), with the wave's own wait for its copies and a bare
// s_barrier the only synchronisation.
//
// A workgroup of 4 waves (2 x 2) covers 64 TM rows of x (tokens) by 64 TJ rows
// of W (features; GATED, TJ = 2: 64 features and their 64 gates, each wave's
// two column tiles a pair).  A stage holds the step's rows of bytes of each
// operand (the layouts are step-major, so each is contiguous), the row
// scales and offsets of its group and the column scales, offsets and sums.
// The 16-byte piece p of a row r lands at p ^ s(r), s(r) = ((r >> 1) ^
// (r >> 2)) & 3 (the copies pick which global piece each lane brings), so
// that the 32 rows a fragment read takes spread over the banks.  Lane l of
// a wave takes 32 bytes of its row at byte 32 (l / 32) of the step's 64, the
// first 16 to the first MFMA and the rest to the second: A and B take the
// same order of k, and integer sums do not depend on it.
template <int TM, int TJ>
struct QStage {
    static constexpr int kXRows = 64 * TM;
    static constexpr int kWRows = 64 * TJ;      // rows of W a workgroup
    static constexpr int kA = kXRows * 64;       // bytes of x a step
    static constexpr int kB = kWRows * 64;       // bytes of W a step
    static constexpr int kSa = kA + kB;          // offsets of the scales
    static constexpr int kOa = kSa + kXRows * 4;
    static constexpr int kSb = kOa + kXRows * 4;
    static constexpr int kOb = kSb + kWRows * 4;
    static constexpr int kQs = kOb + kWRows * 4;
    static constexpr int kBytes = kQs + kWRows * 4;
    static constexpr int kUnits16 = (kA + kB) / 1024;                 // 1 KB copies
    static constexpr int kUnits4 = (2 * kXRows + 3 * kWRows) / 64;     // 256-byte copies
    static constexpr int kC16 = kUnits16 / 4;                         // a wave's, a step
    static constexpr int kC4 = (kUnits4 + 3) / 4;
    static constexpr int kCopies = kC16 + kC4;
    static_assert(kUnits16 % 4 == 0, "1 KB copies shared evenly");
};

__device__ __forceinline__ int qswizzle(int row) { return ((row >> 1) ^ (row >> 2)) & 3; }

template <bool GATED, int TM, int S, int TJ>
__global__ __launch_bounds__(256) void qgemm3_kernel(QgemmArgs p) {
    static_assert(!GATED || TJ == 2, "the gated products pair two column tiles");
    using L = QStage<TM, TJ>;
    constexpr int BM = L::kXRows;
    __shared__ __attribute__((aligned(1024))) char lds[S * L::kBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave >> 1, wc = wave & 1;
    const int r32 = lane & 31, h = lane >> 5;

    // An XCD takes consecutive workgroups of this order (xcd_swizzle), which
    // share the operand the order holds fixed in its L2.
    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint32_t major = p.by_columns ? static_cast<uint32_t>(p.row_blocks) : static_cast<uint32_t>(p.col_blocks);
    const uint32_t bq = b / major, br = b - bq * major;
    const int64_t mb = p.by_columns ? br : bq;
    const int64_t nb = p.by_columns ? bq : br;
    const int64_t m0 = mb * BM;
    const int64_t n0 = nb * (GATED ? 64 : L::kWRows);
    // The W row of block row r (clamped): GATED, rows 0..63 features n0 +
    // r and rows 64..127 their gates.
    const auto w_row = [&](int r) -> int64_t {
        if (GATED) {
            const int64_t f = n0 + (r & 63);
            return (r >> 6) * p.half + (f < p.half ? f : p.half - 1);
        }
        return n0 + r < p.N ? n0 + r : p.N - 1;
    };
    const auto x_row = [&](int r) -> int64_t { return m0 + r < p.M ? m0 + r : p.M - 1; };

    // This wave's copies a step: 1 KB units wave + 4 q (x's rows first, 16
    // rows a unit, then W's), then 256-byte units wave + 4 q of the scales
    // (sa, oa: TM units each, sb, ob, qs: TJ each, 64 rows a unit); waves
    // past the last unit repeat it.  Per copy: the lane's source, advanced a
    // step (bytes) or a group (scales) at a time, and the unit's place in a
    // stage.
    constexpr int C16 = L::kC16, C4 = L::kC4;
    const int8_t *src16[C16];
    int dst16[C16];
    bool x16[C16];
#pragma unroll
    for (int q = 0; q < C16; ++q) {
        const int u = wave + 4 * q;
        const bool isx = u < L::kA / 1024;
        const int ub = isx ? u : u - L::kA / 1024;
        const int row = 16 * ub + (lane >> 2);
        const int piece = (lane & 3) ^ qswizzle(row);
        x16[q] = isx;
        src16[q] = isx ? p.xq + x_row(row) * 64 + 16 * piece : p.wq + w_row(row) * 64 + 16 * piece;
        dst16[q] = (isx ? 0 : L::kA) + 16 * ub * 64;
    }
    const char *src4[C4];
    int dst4[C4];
    bool x4[C4];
#pragma unroll
    for (int q = 0; q < C4; ++q) {
        int u = wave + 4 * q;
        u = u < L::kUnits4 ? u : L::kUnits4 - 1;
        // Units [0, TM): sa; [TM, 2 TM): oa; then sb, ob, qs TJ each.
        const char *base;
        int off;
        if (u < 2 * TM) {
            const int v = u % TM, row = 64 * v + lane;
            base = reinterpret_cast<const char *>((u < TM ? p.xs : p.xo) + x_row(row));
            off = (u < TM ? L::kSa : L::kOa) + 256 * v;
            x4[q] = true;
        } else {
            const int w = (u - 2 * TM) / TJ, v = (u - 2 * TM) % TJ, row = 64 * v + lane;
            base = w == 0   ? reinterpret_cast<const char *>(p.ws + w_row(row))
                   : w == 1 ? reinterpret_cast<const char *>(p.wo + w_row(row))
                            : reinterpret_cast<const char *>(p.wsum + w_row(row));
            off = (w == 0 ? L::kSb : w == 1 ? L::kOb : L::kQs) + 256 * v;
            x4[q] = false;
        }
        src4[q] = base;
        dst4[q] = off;
    }
    const int subs = static_cast<int>(p.slot / 64);
    const int steps = static_cast<int>(p.groups) * subs;
    // The copies' sources advance a step at a time (the bytes) or a group at
    // a time (the scales), and stop at the last step, which the copies past
    // it repeat; counters, not divisions, track the step and group.
    const int64_t xstep = p.xrows * 64, wstep = p.wrows * 64;
    const int64_t xgroup = p.xrows * 4, wgroup = p.wrows * 4;
    int copied = 0, copy_sub = 0;  // the step the next copies bring, and its place in its group
    const auto copy_step = [&](int stage) {
        char *base = lds + stage * L::kBytes;
#pragma unroll
        for (int q = 0; q < C16; ++q) copy_lds(src16[q], base + dst16[q]);
#pragma unroll
        for (int q = 0; q < C4; ++q) copy_lds4(src4[q], base + dst4[q]);
        if (copied + 1 < steps) {
            ++copied;
#pragma unroll
            for (int q = 0; q < C16; ++q) src16[q] += x16[q] ? xstep : wstep;
            if (++copy_sub == subs) {
                copy_sub = 0;
#pragma unroll
                for (int q = 0; q < C4; ++q) src4[q] += x4[q] ? xgroup : wgroup;
            }
        }
    };

    // The outputs: tile (i, j) of the wave, lane column r32, rows
    // 8 (e / 4) + 4 h + e % 4.
    float t[TM][TJ][16];
    const auto out_row = [&](int i, int e) -> int64_t { return m0 + wr * 32 * TM + 32 * i + 4 * h + tile_row(e); };
    const auto out_col = [&](int j) -> int64_t { return n0 + 32 * TJ * wc + 32 * j + r32; };
    if (!GATED && p.from_redirect) {
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int64_t n = out_col(j);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int64_t m = out_row(i, e);
                    t[i][j][e] = (m < p.M && n < p.N) ? p.y[m * p.ldy + n] : 0.0f;
                }
        }
    } else {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) t[i][j][e] = 0.0f;
    }

    // Fragment reads: A tile i at block row wr 32 TM + 32 i + r32, B tile j
    // at block row (GATED: j 64 + wc 32 + r32; else wc 32 TJ + 32 j + r32),
    // the two 16-byte pieces 2 h and 2 h + 1 at their swizzled places.
    int aread[TM][2], bread[TJ][2], brow[TJ];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int row = wr * 32 * TM + 32 * i + r32;
#pragma unroll
        for (int q = 0; q < 2; ++q) aread[i][q] = row * 64 + (((2 * h + q) ^ qswizzle(row)) << 4);
    }
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int row = GATED ? 64 * j + 32 * wc + r32 : 32 * TJ * wc + 32 * j + r32;
        brow[j] = row;
#pragma unroll
        for (int q = 0; q < 2; ++q) bread[j][q] = L::kA + row * 64 + (((2 * h + q) ^ qswizzle(row)) << 4);
    }

    int16v acc[TM][TJ];
    const auto compute = [&](int stage, int sub) {
        const char *base = lds + stage * L::kBytes;
        int4v a[TM][2], bv[TJ][2];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int q = 0; q < 2; ++q) a[i][q] = *reinterpret_cast<const int4v *>(base + aread[i][q]);
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) bv[j][q] = *reinterpret_cast<const int4v *>(base + bread[j][q]);
        // A group's first step starts its sums from zero (a branch uniform
        // over the workgroup).
        if (sub == 0) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i][0], bv[j][0], int16v{}, 0, 0, 0);
        } else {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i][0], bv[j][0], acc[i][j], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i][1], bv[j][1], acc[i][j], 0, 0, 0);
        if (sub != subs - 1) return;
        // The group's sums into the outputs, as quant.cc:150-155 does:
        // t = fma(sa sb, S, t); t = fma(-oa, ob, t).
        const float *sa = reinterpret_cast<const float *>(base + L::kSa);
        const float *oa = reinterpret_cast<const float *>(base + L::kOa);
        const float *sb = reinterpret_cast<const float *>(base + L::kSb);
        const float *ob = reinterpret_cast<const float *>(base + L::kOb);
        const int32_t *qs = reinterpret_cast<const int32_t *>(base + L::kQs);
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const float cs = sb[brow[j]], nco = -ob[brow[j]];
            const int32_t shift = 128 * qs[brow[j]];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int e4 = 0; e4 < 4; ++e4) {
                    const int row = wr * 32 * TM + 32 * i + 4 * h + 8 * e4;
                    const float4v sa4 = *reinterpret_cast<const float4v *>(sa + row);
                    const float4v oa4 = *reinterpret_cast<const float4v *>(oa + row);
#pragma unroll
                    for (int e1 = 0; e1 < 4; ++e1) {
                        const int e = 4 * e4 + e1;
                        const float ab = __fmul_rn(sa4[e1], cs);
                        const float sum = static_cast<float>(acc[i][j][e] + shift);
                        const float v = __builtin_fmaf(ab, sum, t[i][j][e]);
                        t[i][j][e] = __builtin_fmaf(oa4[e1], nco, v);
                    }
                }
        }
    };

    // The residual's loads done before any copy is in flight, so that the
    // compiler need not wait for the copies to know t is there.
    wait_loads<0>();
    static_assert((S & (S - 1)) == 0, "stages a power of two");
    constexpr int kBehind = (S - 2) * L::kCopies;  // a wave's copies behind a step's
#pragma unroll
    for (int q = 0; q < S - 1; ++q) copy_step(q);
    int sub = 0;
    for (int s = 0; s < steps; ++s) {
        // This wave's copies of step s are in (those of the S - 2 steps after
        // it may still be in flight), and every wave's, past the barrier --
        // which also means every wave is done with the stage the next copies
        // overwrite, read at step s - 1.
        wait_loads<kBehind>();
        barrier_only();
        copy_step((s + S - 1) & (S - 1));
        compute(s & (S - 1), sub);
        sub = sub + 1 == subs ? 0 : sub + 1;
    }
    // No copy may still be landing in LDS when the workgroup ends.
    wait_loads<0>();

    // The chain, then the stores (or the gated GELU of the pair).
    const uint32_t ne1 = static_cast<uint32_t>(p.ne1), ne2 = static_cast<uint32_t>(p.ne2);
    const auto row_off = [&](const DevStep &st, int64_t m) -> int64_t {
        if (st.flat123) return m * st.nb[1];
        uint32_t i1, i2, i3;
        split_index(static_cast<uint32_t>(m), ne1, ne2, i1, i2, i3);
        return i1 * st.nb[1] + i2 * st.nb[2] + i3 * st.nb[3];
    };
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const auto row = [&](int e) -> int64_t {
            const int64_t m = out_row(i, e);
            return m < p.M ? m : p.M - 1;
        };
        if (GATED) {
            const int64_t f = n0 + 32 * wc + r32;
            const int64_t fc = f < p.half ? f : p.half - 1;
            apply_chain_block(p.chain, t[i][0], [&](int s, int e) {
                return fc * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e));
            });
            apply_chain_block(p.chain, t[i][1], [&](int s, int e) {
                return (p.half + fc) * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e));
            });
            if (f >= p.half) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t m = out_row(i, e);
                if (m < p.M) p.y[m * p.ldy + f] = t[i][0][e] * gelu(t[i][1][e]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int64_t n = out_col(j);
                const int64_t nc = n < p.N ? n : p.N - 1;
                apply_chain_block(p.chain, t[i][j], [&](int s, int e) {
                    return nc * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e));
                });
                if (n >= p.N) continue;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int64_t m = out_row(i, e);
                    if (m < p.M) p.y[m * p.ldy + n] = t[i][j][e];
                }
            }
        }
    }
}

constexpr int kQStages = 4;
static_assert(2 * kQStages * QStage<2, 2>::kBytes <= 160 * 1024, "two workgroups' rings fit a CU's LDS");
static_assert((kQStages - 2) * QStage<2, 2>::kCopies < 64, "vmcnt");

// Workgroups of 128 rows of x by 128 of W where the launch still gives every
// SIMD two waves, else 64 by 128, else (not gated) 64 by 64: the block's
// products and sums are the same whatever its shape.
// The workgroups go along the rows of x within a column block of W where x
// is the smaller operand (the gated FF-in's 1976 x 1280 bytes of x against
// 10240 x 1280 of W): each XCD then reads W's column blocks once and holds
// all of x in its L2, where the other order reads all of W once per pass of
// an XCD's workgroups over a row block.
template <bool GATED>
hipError_t launch_qgemm2(QgemmArgs p, hipStream_t stream) {
    const int64_t cols = GATED ? p.half : p.N;
    p.by_columns = p.M < (GATED ? 2 * p.half : p.N) ? 1 : 0;
    const int64_t cols128 = ceil_div(cols, GATED ? 64 : 128);
    if (ceil_div(p.M, 128) * cols128 >= 512) {
        p.col_blocks = cols128;
        p.row_blocks = ceil_div(p.M, 128);
        SDHIP_LAUNCH((qgemm3_kernel<GATED, 2, kQStages, 2>), dim3(static_cast<uint32_t>(p.row_blocks * p.col_blocks)),
                     dim3(256), 0, stream, p);
    } else if (GATED || ceil_div(p.M, 64) * cols128 >= 512) {
        p.col_blocks = cols128;
        p.row_blocks = ceil_div(p.M, 64);
        SDHIP_LAUNCH((qgemm3_kernel<GATED, 1, kQStages, 2>), dim3(static_cast<uint32_t>(p.row_blocks * p.col_blocks)),
                     dim3(256), 0, stream, p);
    } else {
        p.col_blocks = ceil_div(cols, 64);
        p.row_blocks = ceil_div(p.M, 64);
        SDHIP_LAUNCH((qgemm3_kernel<false, 1, kQStages, 1>), dim3(static_cast<uint32_t>(p.row_blocks * p.col_blocks)),
                     dim3(256), 0, stream, p);
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ convolutions

// The columns of a direct convolution (conv2d.cc:228-316): position m = (n,
// oy, ox), k = ic KH KW + kh KW + kw, zeros outside the image.
struct ColumnsSrc {
    ConvArgs c;
    __device__ float operator()(int64_t m, int64_t k) const {
        uint32_t ox, oy, n;
        split_index(static_cast<uint32_t>(m), static_cast<uint32_t>(c.ow), static_cast<uint32_t>(c.oh), ox, oy, n);
        const int64_t ic = k / c.taps, t = k - ic * c.taps;
        const int64_t kh = t / c.kw, kw = t - kh * c.kw;
        const int64_t iy = static_cast<int64_t>(oy) * c.s1 - c.p1 + kh * c.d1;
        const int64_t ix = static_cast<int64_t>(ox) * c.s0 - c.p0 + kw * c.d0;
        if (iy < 0 || iy >= c.ih || ix < 0 || ix >= c.iw) return 0.0f;
        return c.x[static_cast<int64_t>(n) * c.xnb3 + ic * c.xnb2 + iy * c.xnb1 + ix];
    }
};

// t[p][oc] = y at (position p, channel oc): the residual the quantized sums
// begin from (conv2d.cc:466-468, accumulate with from_redirect).
__global__ __launch_bounds__(256) void conv_gather_kernel(ConvArgs c, float *__restrict__ t) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= c.P * c.oc) return;
    const int64_t p = i / c.oc, oc = i - p * c.oc;
    uint32_t ox, oy, n;
    split_index(static_cast<uint32_t>(p), static_cast<uint32_t>(c.ow), static_cast<uint32_t>(c.oh), ox, oy, n);
    t[i] = c.y[static_cast<int64_t>(n) * c.ynb3 + oc * c.ynb2 + static_cast<int64_t>(oy) * c.ynb1 + ox];
}

// y at (p, oc) = the chain of t[p][oc] over the positions of channel oc
// (apply_chain_positions, conv2d.cc:472-474).
__global__ __launch_bounds__(256) void conv_scatter_kernel(ConvArgs c, const float *__restrict__ t) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= c.P * c.oc) return;
    const int64_t oc = i / c.P, p = i - oc * c.P;  // consecutive threads: consecutive positions
    uint32_t ox, oy, n;
    split_index(static_cast<uint32_t>(p), static_cast<uint32_t>(c.ow), static_cast<uint32_t>(c.oh), ox, oy, n);
    float v[1] = {t[p * c.oc + oc]};
    const int64_t in_image = static_cast<int64_t>(oy) * c.ow + ox;
    apply_chain_block<1>(c.chain, v, [&](int s, int) -> int64_t {
        const DevStep &st = c.chain.steps[s];
        const int64_t xy =
            st.flat01 ? in_image * st.nb[0] : static_cast<int64_t>(ox) * st.nb[0] + static_cast<int64_t>(oy) * st.nb[1];
        return xy + static_cast<int64_t>(n) * st.nb[3] + oc * st.nb[2];
    });
    c.y[static_cast<int64_t>(n) * c.ynb3 + oc * c.ynb2 + static_cast<int64_t>(oy) * c.ynb1 + ox] = v[0];
}

// Row i of F(2x2)'s B^T of four numbers (winograd.cc:321-332).
__device__ __forceinline__ float bt2(int i, float d0, float d1, float d2, float d3) {
    return i == 0 ? __fsub_rn(d0, d2) : i == 1 ? __fadd_rn(d1, d2) : i == 2 ? __fsub_rn(d2, d1) : __fsub_rn(d1, d3);
}

// The transformed inputs of F(2x2) in single precision, as the reference's
// transform_inputs_small computes them (each row of d by bt(s), then the rows
// by bt(r), winograd.cc:631-672): v[xi][tile][ic], a thread per (tile,
// channel).
__global__ __launch_bounds__(256) void wq_inputs_kernel(ConvArgs c, int64_t tw, int64_t th, int64_t tiles,
                                                        float *__restrict__ v) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= tiles * c.ic) return;
    const int64_t tile = i / c.ic, ic = i - tile * c.ic;
    const int64_t per = tw * th;
    const int64_t n = tile / per, r = tile - n * per, ty = r / tw, tx = r - ty * tw;
    const float *plane = c.x + n * c.xnb3 + ic * c.xnb2;
    float d[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int64_t y = 2 * ty - c.p1 + a, x = 2 * tx - c.p0 + b;
            d[a][b] = (y >= 0 && y < c.ih && x >= 0 && x < c.iw) ? plane[y * c.xnb1 + x] : 0.0f;
        }
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
        float row[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) row[a] = bt2(s4, d[a][0], d[a][1], d[a][2], d[a][3]);
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) v[((r4 * 4 + s4) * tiles + tile) * c.ic + ic] = bt2(r4, row[0], row[1], row[2], row[3]);
    }
}

// The transformed kernels of F(2x2) in single precision, as the reference's
// transform_weights computes them (G g a column at a time, then (G g) G^T a
// row at a time, each sum of three left to right and halved after,
// winograd.cc:681-729): u[xi][oc][ic], a thread per (oc, channel).
template <class W>
__global__ __launch_bounds__(256) void wq_weights_kernel(const W *__restrict__ w, int64_t oc, int64_t ic,
                                                         float *__restrict__ u) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= oc * ic) return;
    const W *g = w + i * 9;
    float t[4][3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const float g0 = static_cast<float>(g[j]), g1 = static_cast<float>(g[3 + j]), g2 = static_cast<float>(g[6 + j]);
        t[0][j] = g0;
        t[1][j] = __fmul_rn(0.5f, __fadd_rn(__fadd_rn(g0, g1), g2));
        t[2][j] = __fmul_rn(0.5f, __fadd_rn(__fsub_rn(g0, g1), g2));
        t[3][j] = g2;
    }
    const int64_t plane = oc * ic;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float a = t[r][0], b = t[r][1], d = t[r][2];
        u[(r * 4 + 0) * plane + i] = a;
        u[(r * 4 + 1) * plane + i] = __fmul_rn(0.5f, __fadd_rn(__fadd_rn(a, b), d));
        u[(r * 4 + 2) * plane + i] = __fmul_rn(0.5f, __fadd_rn(__fsub_rn(a, b), d));
        u[(r * 4 + 3) * plane + i] = d;
    }
}

// Y = A^T M A of F(2x2) as the reference's transform_outputs sums it (rows 0
// and 1 of A^T M, then their columns, left to right, winograd.cc:509-623),
// added to y with from_redirect, then the chain over the positions; m
// [xi][tile][oc], a thread per (oc, tile).
__global__ __launch_bounds__(256) void wq_outputs_kernel(ConvArgs c, int64_t tw, int64_t th, int64_t tiles,
                                                         const float *__restrict__ m) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= tiles * c.oc) return;
    const int64_t tile = i / c.oc, oc = i - tile * c.oc;
    const int64_t per = tw * th;
    const int64_t n = tile / per, r = tile - n * per, ty = r / tw, tx = r - ty * tw;
    float v[16];
#pragma unroll
    for (int xi = 0; xi < 16; ++xi) v[xi] = m[(xi * tiles + tile) * c.oc + oc];
    float a0[4], a1[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        a0[j] = __fadd_rn(__fadd_rn(v[j], v[4 + j]), v[8 + j]);
        a1[j] = __fsub_rn(__fsub_rn(v[4 + j], v[8 + j]), v[12 + j]);
    }
    const float out[2][2] = {{__fadd_rn(__fadd_rn(a0[0], a0[1]), a0[2]), __fsub_rn(__fsub_rn(a0[1], a0[2]), a0[3])},
                             {__fadd_rn(__fadd_rn(a1[0], a1[1]), a1[2]), __fsub_rn(__fsub_rn(a1[1], a1[2]), a1[3])}};
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int64_t oy = 2 * ty + a, ox = 2 * tx + b;
            if (oy >= c.oh || ox >= c.ow) continue;
            float *p = c.y + n * c.ynb3 + oc * c.ynb2 + oy * c.ynb1 + ox;
            float val[1] = {c.from_redirect ? __fadd_rn(*p, out[a][b]) : out[a][b]};
            const int64_t in_image = oy * c.ow + ox;
            apply_chain_block<1>(c.chain, val, [&](int s, int) -> int64_t {
                const DevStep &st = c.chain.steps[s];
                const int64_t xy = st.flat01 ? in_image * st.nb[0] : ox * st.nb[0] + oy * st.nb[1];
                return xy + n * st.nb[3] + oc * st.nb[2];
            });
            *p = val[0];
        }
}

// The quantized product of rows [m0, m0 + rows) of the inputs' layout by
// rows [n0, n0 + cols) of the weights' (qgemm), into t (rows ldt apart),
// begun from t where from_redirect; no chain.
hipError_t launch_qgemm_part(const Layout &l, int8_t *xq, float *xs, float *xo, int8_t *wq, float *ws, float *wo,
                             int32_t *wsum, int64_t m0, int64_t rows, int64_t n0, int64_t cols, float *t, int64_t ldt,
                             int32_t from_redirect, hipStream_t stream) {
    QgemmArgs p{};
    p.xq = xq + m0 * 64;
    p.xs = xs + m0;
    p.xo = xo + m0;
    p.wq = wq + n0 * 64;
    p.ws = ws + n0;
    p.wo = wo + n0;
    p.wsum = wsum + n0;
    p.xrows = l.m;
    p.wrows = l.n;
    p.y = t;
    p.ldy = ldt;
    p.M = rows;
    p.N = cols;
    p.ne1 = rows;
    p.ne2 = 1;
    p.groups = l.groups;
    p.slot = l.slot;
    p.kp = l.kp;
    p.from_redirect = from_redirect;
    if (tuning().qgemm_core == 1) {
        p.col_blocks = ceil_div(cols, kQB);
        const dim3 grid(static_cast<uint32_t>(ceil_div(rows, kQB) * p.col_blocks));
        SDHIP_LAUNCH(qgemm_kernel<false>, grid, dim3(256), 0, stream, p);
        return hipGetLastError();
    }
    return launch_qgemm2<false>(p, stream);
}

}  // namespace

// ------------------------------------------------------------------ convolutions: host

namespace {

struct QconvLayout {
    Layout q;       // the quantized operands
    size_t t;       // direct: t[P][OC]; Winograd: M[16][tiles][OC]
    size_t v, u;    // Winograd: V[16][tiles][IC], U[16][OC][IC] in single precision
    size_t total;
};

QconvLayout qconv_layout(const ConvArgs &c, bool winograd, int64_t tiles, const Quant &q) {
    QconvLayout l{};
    size_t at = 0;
    const auto take = [&](size_t bytes) {
        const size_t here = at;
        at += static_cast<size_t>(round_up(static_cast<int64_t>(bytes), 256));
        return here;
    };
    if (winograd) {
        l.q = layout_of(c.ic, 16 * c.oc, 16 * tiles, q);
        const size_t qbase = take(l.q.total);
        (void)qbase;  // the quantized operands first, at 0
        l.t = take(static_cast<size_t>(16 * tiles * c.oc) * 4);
        l.v = take(static_cast<size_t>(16 * tiles * c.ic) * 4);
        l.u = take(static_cast<size_t>(16 * c.oc * c.ic) * 4);
    } else {
        l.q = layout_of(c.K, c.oc, c.P, q);
        take(l.q.total);
        l.t = take(static_cast<size_t>(c.P * c.oc) * 4);
    }
    l.total = at;
    return l;
}

int64_t qtiles(const ConvArgs &c) { return c.n * ceil_div(c.ow, 2) * ceil_div(c.oh, 2); }

// The stretch of input channels whose transformed weights are quantized at
// a time (winograd.cc:1859-1866 with plan and plan_small, 236-266): the
// blocks of input channels of the reference's single-precision plan, in
// groups; weight_group = 0 gives each stretch a scale of its own.
int64_t winograd_stretch(const ConvArgs &c, const Quant &q) {
    const Tuning &t = tuning();
    const bool small = c.n * ceil_div(c.ow, 2) * ceil_div(c.oh, 2) <= t.winograd_small_tiles;
    const int64_t want = small ? (t.winograd_small_kc > 8 ? t.winograd_small_kc : 8) : t.winograd_kc;
    const int64_t kc = c.ic < want ? c.ic : want;
    const int64_t stretch = kc / q.group * q.group;
    return stretch > q.group ? stretch : q.group;
}

}  // namespace

size_t quantized_conv_work_size(const ConvArgs &c, bool winograd) {
    return qconv_layout(c, winograd, qtiles(c), quant_of(tuning())).total;
}

sdhip_status quantized_conv(const ConvArgs &c, bool winograd, void *work, hipStream_t stream) {
    const Quant q = quant_of(tuning());
    const int64_t tiles = qtiles(c);
    const QconvLayout L = qconv_layout(c, winograd, tiles, q);
    const Layout &l = L.q;
    char *base = static_cast<char *>(work);
    int8_t *xq = reinterpret_cast<int8_t *>(base + l.xq);
    float *xs = reinterpret_cast<float *>(base + l.xs);
    float *xo = reinterpret_cast<float *>(base + l.xo);
    int8_t *wq = reinterpret_cast<int8_t *>(base + l.wq);
    float *ws = reinterpret_cast<float *>(base + l.ws);
    float *wo = reinterpret_cast<float *>(base + l.wo);
    int32_t *wsum = reinterpret_cast<int32_t *>(base + l.wsum);
    float *t = reinterpret_cast<float *>(base + L.t);
    const auto grid = [](int64_t n) { return dim3(static_cast<uint32_t>(ceil_div(n, 256))); };
    if (!winograd) {
        // conv2d.cc:338-483: the columns quantized per (position, group), the
        // kernels per (output channel, group) or per whole row; the sums in
        // t[p][oc], begun from the residual where from_redirect; then the
        // chain into y.
        {
            KernelScope scope("qconv.quantize", stream);
            SDHIP_LAUNCH(quantize_inputs_kernel<ColumnsSrc>, dim3(ceil_div(c.P * l.groups, 4)), dim3(256), 0,
                         stream, ColumnsSrc{c}, c.P, c.K, q, l, xq, xs, xo);
            if (c.w32 != nullptr) {
                SDHIP_LAUNCH(quantize_weights_kernel<float>, dim3(ceil_div(c.oc, 4)), dim3(256), 0, stream, c.w32,
                             c.K, c.oc, c.K, q, l, wq, ws, wo, wsum, int64_t{0});
            } else {
                SDHIP_LAUNCH(quantize_weights_kernel<_Float16>, dim3(ceil_div(c.oc, 4)), dim3(256), 0, stream,
                             c.w, c.K, c.oc, c.K, q, l, wq, ws, wo, wsum, int64_t{0});
            }
            if (c.from_redirect) SDHIP_LAUNCH(conv_gather_kernel, grid(c.P * c.oc), dim3(256), 0, stream, c, t);
        }
        {
            KernelScope scope("qconv.products", stream);
            const hipError_t e = launch_qgemm_part(l, xq, xs, xo, wq, ws, wo, wsum, 0, c.P, 0, c.oc, t, c.oc,
                                                   c.from_redirect, stream);
            if (e != hipSuccess) return launched(e, "quantized conv2d products");
        }
        KernelScope scope("qconv.outputs", stream);
        SDHIP_LAUNCH(conv_scatter_kernel, grid(c.P * c.oc), dim3(256), 0, stream, c, t);
        return launched(hipGetLastError(), "quantized conv2d");
    }
    // winograd.cc:1826-2103: F(2x2) whatever F(4x4) would take; the points'
    // operands quantized per (tile, group) and (output channel, group or
    // stretch); sixteen quantized products; the outputs' transform and chain.
    const int64_t tw = ceil_div(c.ow, 2), th = ceil_div(c.oh, 2);
    float *v = reinterpret_cast<float *>(base + L.v);
    float *u = reinterpret_cast<float *>(base + L.u);
    {
        KernelScope scope("qwinograd2.transforms", stream);
        SDHIP_LAUNCH(wq_inputs_kernel, grid(tiles * c.ic), dim3(256), 0, stream, c, tw, th, tiles, v);
        if (c.w32 != nullptr) {
            SDHIP_LAUNCH(wq_weights_kernel<float>, grid(c.oc * c.ic), dim3(256), 0, stream, c.w32, c.oc, c.ic, u);
        } else {
            SDHIP_LAUNCH(wq_weights_kernel<_Float16>, grid(c.oc * c.ic), dim3(256), 0, stream, c.w, c.oc, c.ic,
                         u);
        }
    }
    {
        KernelScope scope("qwinograd2.quantize", stream);
        SDHIP_LAUNCH(quantize_inputs_kernel<RowsSrc>, dim3(ceil_div(16 * tiles * l.groups, 4)), dim3(256), 0,
                     stream, RowsSrc{v, c.ic}, 16 * tiles, c.ic, q, l, xq, xs, xo);
        SDHIP_LAUNCH(quantize_weights_kernel<float>, dim3(ceil_div(16 * c.oc, 4)), dim3(256), 0, stream, u, c.ic,
                     16 * c.oc, c.ic, q, l, wq, ws, wo, wsum, winograd_stretch(c, q));
    }
    {
        KernelScope scope("qwinograd2.products", stream);
        for (int xi = 0; xi < 16; ++xi) {
            const hipError_t e = launch_qgemm_part(l, xq, xs, xo, wq, ws, wo, wsum, xi * tiles, tiles, xi * c.oc, c.oc,
                                                   t + xi * tiles * c.oc, c.oc, 0, stream);
            if (e != hipSuccess) return launched(e, "quantized winograd products");
        }
    }
    KernelScope scope("qwinograd2.outputs", stream);
    SDHIP_LAUNCH(wq_outputs_kernel, grid(tiles * c.oc), dim3(256), 0, stream, c, tw, th, tiles, t);
    return launched(hipGetLastError(), "quantized winograd");
}

size_t quantized_linear_work_size(int64_t K, int64_t N, int64_t M) {
    return layout_of(K, N, M, quant_of(tuning())).total;
}

sdhip_status quantized_linear(const MulMatArgs &a, bool gated, void *work, hipStream_t stream) {
    const Quant q = quant_of(tuning());
    const Layout l = layout_of(a.K, a.N, a.M, q);
    char *base = static_cast<char *>(work);
    int8_t *xq = reinterpret_cast<int8_t *>(base + l.xq);
    float *xs = reinterpret_cast<float *>(base + l.xs);
    float *xo = reinterpret_cast<float *>(base + l.xo);
    // The quantized weights: kept in the store when it has room for them
    // (quantized layouts are kept by default, store.cc:64-99), else derived
    // into the work buffer at every call.
    const size_t wbytes = l.total - l.wq;
    const int64_t ne[4] = {a.K, a.N, 1, 1};
    const int64_t esize = a.w32 != nullptr ? 4 : 2;
    const int64_t ld = a.w32 != nullptr ? a.ldw32 : a.ldw;
    const int64_t nb[4] = {esize, esize * ld, esize * ld * a.N, esize * ld * a.N};
    const void *wsrc = a.w32 != nullptr ? static_cast<const void *>(a.w32) : static_cast<const void *>(a.w);
    const uint64_t variant = static_cast<uint64_t>(q.group) | static_cast<uint64_t>(q.wmax) << 16 |
                             static_cast<uint64_t>(q.weight_groups) << 24;
    bool ready = false;
    char *kept = static_cast<char *>(store_entry(wsrc, a.w32 != nullptr ? SDHIP_TYPE_F32 : SDHIP_TYPE_F16, ne, nb,
                                                 kStoreQuantizedLinear, variant,
                                                 static_cast<size_t>(esize * (ld * (a.N - 1) + a.K)), wbytes, stream,
                                                 ready));
    char *wbase = kept != nullptr ? kept : base + l.wq;  // the weights' parts, at their offsets from l.wq
    int8_t *wq = reinterpret_cast<int8_t *>(wbase);
    float *ws = reinterpret_cast<float *>(wbase + (l.ws - l.wq));
    float *wo = reinterpret_cast<float *>(wbase + (l.wo - l.wq));
    int32_t *wsum = reinterpret_cast<int32_t *>(wbase + (l.wsum - l.wq));
    {
        KernelScope scope("quantize_inputs", stream);
        const bool fast = q.group == 64 && l.slot == 64 && a.K % 64 == 0 && a.ldx % 4 == 0 &&
                          (reinterpret_cast<uintptr_t>(a.x) & 15) == 0;
        if (fast) {
            SDHIP_LAUNCH(quantize_inputs64_kernel, dim3(ceil_div(a.M * l.groups, 16)), dim3(256), 0, stream, a.x,
                         a.ldx, a.M, l.groups, static_cast<float>(q.levels), xq, xs, xo);
        } else {
            SDHIP_LAUNCH(quantize_inputs_kernel<RowsSrc>, dim3(ceil_div(a.M * l.groups, 4)), dim3(256), 0, stream,
                         RowsSrc{a.x, a.ldx}, a.M, a.K, q, l, xq, xs, xo);
        }
    }
    if (!ready) {
        KernelScope scope("quantize_weights", stream);
        if (a.w32 != nullptr) {
            SDHIP_LAUNCH(quantize_weights_kernel<float>, dim3(ceil_div(a.N, 4)), dim3(256), 0, stream, a.w32,
                         a.ldw32, a.N, a.K, q, l, wq, ws, wo, wsum, int64_t{0});
        } else {
            SDHIP_LAUNCH(quantize_weights_kernel<_Float16>, dim3(ceil_div(a.N, 4)), dim3(256), 0, stream, a.w,
                         a.ldw, a.N, a.K, q, l, wq, ws, wo, wsum, int64_t{0});
        }
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return launched(err, "quantize_weights");
        if (kept != nullptr) store_publish(kept);
    }
    QgemmArgs p{};
    p.xq = xq;
    p.wq = wq;
    p.xs = xs;
    p.xo = xo;
    p.ws = ws;
    p.wo = wo;
    p.wsum = wsum;
    p.y = a.y;
    p.ldy = a.ldy;
    p.M = a.M;
    p.N = a.N;
    p.half = a.half;
    p.ne1 = a.ne1;
    p.ne2 = a.ne2;
    p.groups = l.groups;
    p.slot = l.slot;
    p.kp = l.kp;
    p.xrows = l.m;
    p.wrows = l.n;
    p.from_redirect = a.from_redirect;
    p.chain = a.chain;
    KernelScope scope(gated ? "qgemm_gated" : "qgemm", stream);
    if (tuning().qgemm_core != 1) {
        const hipError_t err = gated ? launch_qgemm2<true>(p, stream) : launch_qgemm2<false>(p, stream);
        return launched(err, gated ? "quantized mul_mat_gated" : "quantized mul_mat");
    }
    const int64_t cols = gated ? a.half : a.N;
    p.col_blocks = ceil_div(cols, gated ? kQB / 2 : kQB);
    const dim3 grid(static_cast<uint32_t>(ceil_div(a.M, kQB) * p.col_blocks));
    if (gated) {
        SDHIP_LAUNCH(qgemm_kernel<true>, grid, dim3(256), 0, stream, p);
    } else {
        SDHIP_LAUNCH(qgemm_kernel<false>, grid, dim3(256), 0, stream, p);
    }
    return launched(hipGetLastError(), gated ? "quantized mul_mat_gated" : "quantized mul_mat");
}

}  // namespace sdhip
