// The products of FP16 weights by single-precision activations on gfx950's
// FP16 MFMA (v_mfma_f32_32x32x16_f16): MUL_MAT (mul_mat.cc), MUL_MAT with the
// gated GELU after it (mul_mat.cc:889-1058), the direct convolution
// (conv2d.cc), and the alpha^2 products of Winograd's convolution
// (winograd.cc), each with its chain applied while the output tile is in
// registers.
//
// Precision.  The weights are FP16 and so exact as FP16 MFMA operands; each
// activation x is split into two FP16 parts (device.h, split2), and every
// product is taken as w*hi + w*lo, two MFMAs into the same single-precision
// accumulator: 22 bits of x, as the reference's AMX-FP16 form takes it
// (x86_64/amx_fp16.S: the weights exact, x in two FP16 parts), where ggml
// rounds x to FP16 (11 bits).  Winograd's transformed weights are not FP16
// numbers: both operands are split there and the products taken as
// a_hi b_hi + a_hi b_lo + a_lo b_hi, three MFMAs (the fourth, a_lo b_lo, is
// below 2^-22 of the product).
//
// Shape.  A workgroup of 4 waves (2 x 2) computes a block of BM x BN of
// C = A B^T, A and B both K-contiguous rows, in steps of BK = 32 of K.  The
// rows go from global memory into registers two steps ahead of the MFMAs
// (two register stages, two LDS buffers), are split where they are single
// precision and written to LDS as FP16; each wave computes its TM x TN tiles
// of 32 x 32 from LDS, two K-steps of 16 a step.
//   MUL_MAT:     A = x (tokens, split), B = W (features): C[token][feature]
//   convolution: A = W (output channels), B = the image's columns (split),
//                C[channel][position]
//   Winograd:    A = U[xi] (output channels; two FP16 planes, or single
//                precision with each column scaled and split here), B = V[xi]
//                (tiles; two FP16 planes, split by the inputs' transform)
// so that the output's contiguous dimension is always C's column, lane % 32
// of the MFMA's result, and a wave's stores are 128-byte rows.

#include <type_traits>

#include "device.h"
#include "kernels.h"
#include "profile.h"

namespace sdhip {

namespace {

constexpr int kBK = 32;
constexpr int kLdk = kBK + 8;  // halves per LDS row: 80 bytes, 16-byte aligned, skewed across banks

// Which operands are single precision, split into two FP16 planes.
// kSplitNone: the products of 16 bits (bits=16): the single-precision
// operand rounded to FP16, its first part alone, one MFMA a product.
// kBf16: the same in bfloat16 (half_format=1): both operands rounded to
// bfloat16 (to nearest, ties to even, as vcvtne2ps2bf16 rounds them), one
// bfloat16 MFMA a product; the LDS planes hold their bits.
enum Split { kSplitA = 0, kSplitB = 1, kSplitBoth = 2, kSplitNone = 3, kBf16 = 4 };

constexpr int planes_a(int mode) { return mode == kSplitB || mode == kSplitNone || mode == kBf16 ? 1 : 2; }
constexpr int planes_b(int mode) { return mode == kSplitA || mode == kSplitNone || mode == kBf16 ? 1 : 2; }

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// The bits of x rounded to bfloat16 (to nearest, ties to even), in a 16-bit
// container of the LDS planes' type.
__device__ __forceinline__ _Float16 bf16_bits(float x) {
    const __bf16 b = static_cast<__bf16>(x);
    return __builtin_bit_cast(_Float16, b);
}

// ------------------------------------------------------------------ MFMA core

// acc[i][j] += A rows (32 i ..) x B rows (32 j ..) over one BK step held in
// LDS: two MFMAs per tile and K-step of 16 with one operand split, three
// with both.
template <int TM, int TN, int MODE>
__device__ __forceinline__ void mfma_step(float16v (&acc)[TM][TN], const _Float16 *a_hi, const _Float16 *a_lo,
                                          const _Float16 *b_hi, const _Float16 *b_lo, int lane) {
    const int r = lane & 31;
    const int kh = (lane >> 5) * 8;
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 16) {
        half8 a[TM], al[TM], b[TN], bl[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            a[i] = *reinterpret_cast<const half8 *>(a_hi + (32 * i + r) * kLdk + ks + kh);
            if (planes_a(MODE) == 2) al[i] = *reinterpret_cast<const half8 *>(a_lo + (32 * i + r) * kLdk + ks + kh);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            b[j] = *reinterpret_cast<const half8 *>(b_hi + (32 * j + r) * kLdk + ks + kh);
            if (planes_b(MODE) == 2) bl[j] = *reinterpret_cast<const half8 *>(b_lo + (32 * j + r) * kLdk + ks + kh);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                if constexpr (MODE == kBf16) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[i]),
                                                                        __builtin_bit_cast(bf16x8, b[j]), acc[i][j],
                                                                        0, 0, 0);
                    continue;
                }
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
                if (planes_a(MODE) == 2) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], b[j], acc[i][j], 0, 0, 0);
                }
                if (planes_b(MODE) == 2) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bl[j], acc[i][j], 0, 0, 0);
                }
            }
        }
    }
}

// ------------------------------------------------------------------ loaders

// Every loader takes BR rows x BK of K into registers (load) and writes them
// to LDS as FP16 (store), one or two planes; a thread's rows are fixed over K,
// so their first elements are found once (init).

// K-contiguous single-precision rows, split into hi and lo planes.  Rows at or
// past `rows`, and k at or past K, are zeros.  VEC: every row start and ld are
// multiples of 4 floats.  FULL (with VEC): K a multiple of BK, and rows past
// the end read the block's first row instead, whose products are never
// stored -- the loads then have no conditions, and so no branches that would
// wait on the loads before them.
// BF (with !LO): the first parts in bfloat16 instead.
template <int BR, bool VEC, bool FULL, bool LO = true, bool BF = false>
struct F32Rows {
    static_assert(!BF || !LO, "the bfloat16 form takes the first parts alone");
    static constexpr int kQuads = BR * kBK / 4 / 256;  // float4 per thread
    static_assert(kQuads >= 1, "tile too small for 256 threads");
    static_assert(!FULL || VEC, "FULL loads are vector loads");
    float4 v[kQuads];
    const float *row[kQuads];
    int64_t K;

    template <class RowOf>
    __device__ void init(const float *base, int64_t ld, RowOf row_of, int64_t k_, int tid) {
        K = k_;
#pragma unroll
        for (int i = 0; i < kQuads; ++i) {
            const int idx = tid + 256 * i;
            int64_t r = row_of(idx / (kBK / 4));
            if (FULL && r < 0) r = row_of(0);
            row[i] = r >= 0 ? base + r * ld + (idx % (kBK / 4)) * 4 : nullptr;
        }
    }

    __device__ void load(int64_t k0, int tid) {
#pragma unroll
        for (int i = 0; i < kQuads; ++i) {
            if (FULL) {
                v[i] = *reinterpret_cast<const float4 *>(row[i] + k0);
                continue;
            }
            const int64_t k = k0 + ((tid + 256 * i) % (kBK / 4)) * 4;
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row[i] != nullptr) {
                const float *p = row[i] + k0;
                if (VEC && k + 4 <= K) {
                    x = *reinterpret_cast<const float4 *>(p);
                } else {
                    if (k + 0 < K) x.x = p[0];
                    if (k + 1 < K) x.y = p[1];
                    if (k + 2 < K) x.z = p[2];
                    if (k + 3 < K) x.w = p[3];
                }
            }
            v[i] = x;
        }
    }

    __device__ void store(_Float16 *hi, _Float16 *lo, int tid) const {
#pragma unroll
        for (int i = 0; i < kQuads; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / (kBK / 4);
            const int kq = (idx % (kBK / 4)) * 4;
            half4 h, l;
            if constexpr (BF) {
                h[0] = bf16_bits(v[i].x * kSplitDown);
                h[1] = bf16_bits(v[i].y * kSplitDown);
                h[2] = bf16_bits(v[i].z * kSplitDown);
                h[3] = bf16_bits(v[i].w * kSplitDown);
                *reinterpret_cast<half4 *>(hi + r * kLdk + kq) = h;
                continue;
            }
            _Float16 a, b;
            split2(v[i].x, a, b); h[0] = a; l[0] = b;
            split2(v[i].y, a, b); h[1] = a; l[1] = b;
            split2(v[i].z, a, b); h[2] = a; l[2] = b;
            split2(v[i].w, a, b); h[3] = a; l[3] = b;
            *reinterpret_cast<half4 *>(hi + r * kLdk + kq) = h;
            // !LO: the first parts alone (the products of 16 bits).
            if (LO) *reinterpret_cast<half4 *>(lo + r * kLdk + kq) = l;
        }
    }
};

// F32Rows's rows with each column k multiplied by scale[k] before the split
// (K a multiple of BK, every row start and ld multiples of 4 floats): a
// thread's four columns are the same at every row it takes, so one float4 of
// scales a step serves them all.
template <int BR, bool FULL>
struct ScaledF32Rows {
    F32Rows<BR, true, FULL> rows;
    const float *scale;
    float4 f;

    template <class RowOf>
    __device__ void init(const float *base, int64_t ld, RowOf row_of, int64_t k_, int tid, const float *scale_) {
        rows.init(base, ld, row_of, k_, tid);
        scale = scale_ + (tid % (kBK / 4)) * 4;
    }

    __device__ void load(int64_t k0, int tid) {
        rows.load(k0, tid);
        f = *reinterpret_cast<const float4 *>(scale + k0);
    }

    __device__ void store(_Float16 *hi, _Float16 *lo, int tid) {
#pragma unroll
        for (int i = 0; i < F32Rows<BR, true, FULL>::kQuads; ++i) {
            rows.v[i].x *= f.x;
            rows.v[i].y *= f.y;
            rows.v[i].z *= f.z;
            rows.v[i].w *= f.w;
        }
        rows.store(hi, lo, tid);
    }
};

// K-contiguous 16-bit rows into LDS, PLANES of them at once (one, or the two
// parts hi and lo of a split operand, `ld_plane` elements apart); `row_of(r)`
// gives the global row of LDS row r, or -1.  FULL as for F32Rows.  BLOCKED
// (with FULL): the rows held in blocks of one K-step, [k / 32][row][k % 32],
// `ld` then 32 and `step` elements from one block to the next, so that a
// step's rows are whole cache lines in a row.
// BF: each FP16 number rounded to bfloat16 on its way into LDS.
template <int BR, bool VEC, bool FULL, int PLANES = 1, bool BLOCKED = false, bool BF = false>
struct F16Rows {
    static_assert(!BF || PLANES == 1, "the bfloat16 form takes one plane");
    static constexpr int kOcts = BR * kBK / 8 / 256;  // 8 halves per load
    static_assert(kOcts >= 1, "tile too small for 256 threads");
    static_assert(!FULL || VEC, "FULL loads are vector loads");
    static_assert(!BLOCKED || FULL, "BLOCKED rows are FULL ones");
    half8 v[PLANES][kOcts];
    const _Float16 *row[kOcts];
    int64_t K, plane, step;

    template <class RowOf>
    __device__ void init(const _Float16 *base, int64_t ld, RowOf row_of, int64_t k_, int tid, int64_t ld_plane = 0,
                         int64_t step_ = 0) {
        K = k_;
        plane = ld_plane;
        step = step_;
#pragma unroll
        for (int i = 0; i < kOcts; ++i) {
            const int idx = tid + 256 * i;
            int64_t r = row_of(idx / (kBK / 8));
            if (FULL && r < 0) r = row_of(0);
            row[i] = r >= 0 ? base + r * ld + (idx % (kBK / 8)) * 8 : nullptr;
        }
    }

    __device__ void load(int64_t k0, int tid) {
#pragma unroll
        for (int i = 0; i < kOcts; ++i) {
#pragma unroll
            for (int q = 0; q < PLANES; ++q) {
                if (FULL) {
                    const int64_t off = BLOCKED ? (k0 / kBK) * step : k0;
                    v[q][i] = *reinterpret_cast<const half8 *>(row[i] + q * plane + off);
                    continue;
                }
                const int64_t k = k0 + ((tid + 256 * i) % (kBK / 8)) * 8;
                half8 x = {};
                if (row[i] != nullptr) {
                    const _Float16 *p = row[i] + q * plane + k0;
                    if (VEC && k + 8 <= K) {
                        x = *reinterpret_cast<const half8 *>(p);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            if (k + e < K) x[e] = p[e];
                        }
                    }
                }
                v[q][i] = x;
            }
        }
    }

    __device__ void store(_Float16 *dst, _Float16 *dst_lo, int tid) const {
#pragma unroll
        for (int i = 0; i < kOcts; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / (kBK / 8);
            const int kq = (idx % (kBK / 8)) * 8;
            if constexpr (BF) {
                half8 b;
#pragma unroll
                for (int e = 0; e < 8; ++e) b[e] = bf16_bits(static_cast<float>(v[0][i][e]));
                *reinterpret_cast<half8 *>(dst + r * kLdk + kq) = b;
                continue;
            }
            *reinterpret_cast<half8 *>(dst + r * kLdk + kq) = v[0][i];
            if (PLANES == 2) *reinterpret_cast<half8 *>(dst_lo + r * kLdk + kq) = v[PLANES - 1][i];
        }
    }
};

// The columns of the image for BN positions p (of all images, n * OH * OW +
// oy * OW + ox) by BK of K = (ic, kh, kw), read from the image where im2col
// would have put them, split, into LDS as [position][k].  A thread takes one
// position and 4 consecutive k: consecutive threads read consecutive
// positions, which are consecutive in a row of the image at stride 1.  FULL
// (1x1 kernels, K = IC a multiple of BK): positions past the last read the
// block's first, never stored, and the loads have no conditions.
// BF (with !LO): the first parts in bfloat16 instead.
template <int BN, bool POINTWISE, bool FULL, bool K3 = false, bool LO = true, bool BF = false>
struct Columns {
    static_assert(!BF || !LO, "the bfloat16 form takes the first parts alone");
    static constexpr int kLoads = BN * kBK / 4 / 256;
    static_assert(!FULL || POINTWISE, "FULL columns are those of 1x1 kernels");
    float v[kLoads][4];
    const ConvArgs *c;
    // Per load slot, fixed over K: the image's first element (or -1 past the
    // last position) and the position's first input row and column.
    int64_t base[kLoads];
    int32_t iy0[kLoads], ix0[kLoads];

    __device__ void init(const ConvArgs &args, int64_t p0, int tid) {
        c = &args;
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int idx = tid + 256 * i;
            int64_t pos = p0 + idx % BN;
            base[i] = -1;
            if (pos >= args.P) {
                if (!FULL) continue;
                pos = p0;
            }
            uint32_t ox, oy, n;
            split_index(static_cast<uint32_t>(pos), static_cast<uint32_t>(args.ow), static_cast<uint32_t>(args.oh), ox,
                        oy, n);
            base[i] = static_cast<int64_t>(n) * args.xnb3;
            if (POINTWISE) {
                base[i] += static_cast<int64_t>(oy) * args.xnb1 + ox;
            } else {
                iy0[i] = static_cast<int32_t>(oy) * args.s1 - args.p1;
                ix0[i] = static_cast<int32_t>(ox) * args.s0 - args.p0;
            }
        }
    }

    __device__ void load(int64_t k0, int tid) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int idx = tid + 256 * i;
            const int kq = (idx / BN) * 4;
            if (FULL) {
                const float *img = c->x + base[i] + (k0 + kq) * c->xnb2;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[i][e] = img[e * c->xnb2];
                continue;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) v[i][e] = 0.0f;
            if (base[i] < 0) continue;
            const float *img = c->x + base[i];
            if (POINTWISE) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t k = k0 + kq + e;
                    if (k < c->K) v[i][e] = img[k * c->xnb2];
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t k = static_cast<uint32_t>(k0 + kq + e);
                    if (k >= c->K) continue;
                    // K3: 3x3 kernels, the divisions by constants.
                    const uint32_t taps = K3 ? 9u : static_cast<uint32_t>(c->taps);
                    const uint32_t kwidth = K3 ? 3u : static_cast<uint32_t>(c->kw);
                    const uint32_t ic = k / taps;
                    const uint32_t t = k - ic * taps;
                    const uint32_t kh = t / kwidth;
                    const uint32_t kw = t - kh * kwidth;
                    const int32_t iy = iy0[i] + static_cast<int32_t>(kh) * c->d1;
                    const int32_t ix = ix0[i] + static_cast<int32_t>(kw) * c->d0;
                    if (iy >= 0 && iy < c->ih && ix >= 0 && ix < c->iw) {
                        v[i][e] = img[static_cast<int64_t>(ic) * c->xnb2 + static_cast<int64_t>(iy) * c->xnb1 + ix];
                    }
                }
            }
        }
    }

    __device__ void store(_Float16 *hi, _Float16 *lo, int tid) const {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int idx = tid + 256 * i;
            const int pl = idx % BN;
            const int kq = (idx / BN) * 4;
            half4 h, l;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                _Float16 a, b;
                if constexpr (BF) {
                    a = bf16_bits(v[i][e] * kSplitDown);
                    b = a;
                } else {
                    split2(v[i][e], a, b);
                }
                h[e] = a;
                l[e] = b;
            }
            *reinterpret_cast<half4 *>(hi + pl * kLdk + kq) = h;
            if (LO) *reinterpret_cast<half4 *>(lo + pl * kLdk + kq) = l;
        }
    }
};

// ------------------------------------------------------------------ main loop

// The K loop of a block: loads NS steps ahead of the MFMAs, through NS
// register stages (la[], lb[], stage q holding the steps s = q mod NS) and two
// LDS buffers (step s in buffer s % 2).  After the MFMAs of step t, the data
// of step t + 1 goes from its stage into the other buffer, and past the
// barrier that stage's loads of step t + 1 + NS go out.  Every load and store
// is unconditional -- past the last step they repeat it, into a buffer no wave
// reads again -- so that the compiler counts the loads in flight exactly and
// waits only for the ones a store needs; only the MFMAs of steps past the
// last are skipped, by a branch uniform over the block.
template <int TM, int TN, int MODE, int NS, class LA, class LB>
__device__ __forceinline__ void main_loop(float16v (&acc)[TM][TN], LA (&la)[NS], LB (&lb)[NS], _Float16 *lds,
                                          int64_t steps, int tid, int lane, int wr, int wc) {
    static_assert(NS % 2 == 0, "stages pair with the two LDS buffers");
    constexpr int BM = 64 * TM, BN = 64 * TN;
    constexpr int PA = planes_a(MODE), PB = planes_b(MODE);
    constexpr int kBuf = (PA * BM + PB * BN) * kLdk;
    _Float16 *buf[2] = {lds, lds + kBuf};
    const auto a_hi = [&](int b) { return buf[b]; };
    const auto a_lo = [&](int b) { return buf[b] + BM * kLdk; };
    const auto b_hi = [&](int b) { return buf[b] + PA * BM * kLdk; };
    const auto b_lo = [&](int b) { return buf[b] + (PA * BM + BN) * kLdk; };
    const auto compute = [&](int b) {
        mfma_step<TM, TN, MODE>(acc, a_hi(b) + wr * 32 * TM * kLdk, a_lo(b) + wr * 32 * TM * kLdk,
                                b_hi(b) + wc * 32 * TN * kLdk, b_lo(b) + wc * 32 * TN * kLdk, lane);
    };
    const auto store = [&](int stage, int b) {
        la[stage].store(a_hi(b), a_lo(b), tid);
        lb[stage].store(b_hi(b), b_lo(b), tid);
    };
    // The scheduler keeps the loads where they are written: issued as early
    // as the registers allow, not moved down to the stores that use them.
    const auto load = [&](int stage, int64_t s) {
        __builtin_amdgcn_sched_barrier(0);
        la[stage].load(s * kBK, tid);
        lb[stage].load(s * kBK, tid);
        __builtin_amdgcn_sched_barrier(0);
    };
    const int64_t last = steps - 1;
    const auto at = [&](int64_t s) { return s < last ? s : last; };

#pragma unroll
    for (int q = 0; q < NS; ++q) load(q, at(q));
    store(0, 0);
    lds_barrier();
    load(0, at(NS));
    // At the top of each pass: buffer 0 holds step s, stages 1 .. NS - 1 steps
    // s + 1 .. s + NS - 1, stage 0 step s + NS on its way.  One exit, at the
    // top, so that every path into the loop has the same loads in flight.
    for (int64_t s = 0; s < steps; s += NS) {
#pragma unroll
        for (int q = 0; q < NS; ++q) {
            if (s + q < steps) compute(q & 1);
            store((q + 1) % NS, (q + 1) & 1);
            lds_barrier();
            load((q + 1) % NS, at(s + q + 1 + NS));
        }
    }
}

template <int TM, int TN, int MODE>
constexpr int lds_halves() {
    return 2 * (planes_a(MODE) * 64 * TM + planes_b(MODE) * 64 * TN) * kLdk;
}

// ------------------------------------------------------------------ MUL_MAT

// C[m][n] = sum_k x[m][k] W[n][k] for rows m of x (single precision, split)
// and rows n of W (FP16), the chain applied, into y[m * ldy + n].  With GATED,
// the block's 128 rows of W are 64 features of the first half and the same 64
// of the second (the gate), each wave's two column tiles a pair, and the
// block writes out[m * ldo + j] = P[m][j] GELU(P[m][half + j]).
template <int TM, int TN, bool GATED, bool VECX, bool VECW, bool FULL, int NS, int WP = 1, int HALF = 0>
__global__ __launch_bounds__(256) void mul_mat_kernel(MulMatArgs p) {
    constexpr int BM = 64 * TM;
    constexpr int BN = 64 * TN;
    // WP: the weights' planes, 1 (FP16 weights) or 2 (single-precision ones
    // split, w_plane apart): then three MFMAs a product, x and W both split.
    // HALF: the products of 16 bits, x rounded to FP16 (1) or both operands
    // to bfloat16 (2), one MFMA a product.
    static_assert(!HALF || WP == 1, "products of 16 bits take FP16 weights");
    constexpr int MODE = HALF == 2 ? kBf16 : HALF ? kSplitNone : WP == 2 ? kSplitBoth : kSplitA;
    static_assert(!GATED || TN == 2, "the gated form pairs two column tiles");
    __shared__ __attribute__((aligned(16))) _Float16 lds[lds_halves<TM, TN, MODE>()];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave >> 1;  // wave row (0, 1)
    const int wc = wave & 1;   // wave column

    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t mb = b / p.col_blocks;
    const int64_t nb = b % p.col_blocks;
    const int64_t m0 = mb * BM;
    const int64_t n0 = nb * (GATED ? BN / 2 : BN);

    const auto x_row = [&](int r) -> int64_t { return m0 + r < p.M ? m0 + r : -1; };
    const auto w_row = [&](int r) -> int64_t {
        if (GATED) {
            const int wq = r / 64;
            const int side = (r / 32) & 1;
            const int64_t f = n0 + 32 * wq + (r & 31);
            return f < p.half ? side * p.half + f : -1;
        }
        const int64_t f = n0 + r;
        return f < p.N ? f : -1;
    };

    float16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = float16v{};

    F32Rows<BM, VECX, FULL, !HALF, HALF == 2> xa[NS];
    F16Rows<BN, VECW, FULL, WP, false, HALF == 2> wb[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        xa[s].init(p.x, p.ldx, x_row, p.K, tid);
        wb[s].init(p.w, p.ldw, w_row, p.K, tid, p.w_plane);
    }
    main_loop<TM, TN, MODE, NS>(acc, xa, wb, lds, (p.K + kBK - 1) / kBK, tid, lane, wr, wc);
    // The product's factor: x's split took 2^-4, and split weights 2^s of their row.
    const auto up = [&](int64_t feature) -> float { return WP == 2 ? kSplitUp * p.w_scale[feature] : kSplitUp; };

    // The epilogue: rows m of the tile, column (feature) lane % 32; a tile's
    // 16 values of the lane at a time, their loads before their stores.  A
    // tile wholly inside the output addresses its rows as a stride from its
    // first; at the last rows, rows past M read the last row and are not
    // stored.
    const int col = lane & 31;
    const int64_t lane_row = 4 * (lane >> 5);
    const uint32_t ne1 = static_cast<uint32_t>(p.ne1), ne2 = static_cast<uint32_t>(p.ne2);
    const auto row_off = [&](const DevStep &st, int64_t m) -> int64_t {
        if (st.flat123) return m * st.nb[1];
        uint32_t i1, i2, i3;
        split_index(static_cast<uint32_t>(m), ne1, ne2, i1, i2, i3);
        return i1 * st.nb[1] + i2 * st.nb[2] + i3 * st.nb[3];
    };
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int64_t tile0 = m0 + wr * 32 * TM + 32 * i;
        const int64_t mbase = tile0 + lane_row;
        const bool full = tile0 + 32 <= p.M;
        // The tile's rows all of one matrix (i2, i3): every operand strided by
        // nb[1] along them, from the offset of the lane's first row.
        const bool one_matrix = static_cast<uint64_t>(tile0 % p.ne1) + 32 <= static_cast<uint64_t>(p.ne1);
        const auto stride = [&](int s) -> int64_t {
            const DevStep &st = p.chain.steps[s];
            return st.flat123 || one_matrix ? st.nb[1] : -1;
        };
        const auto first = [&](int s) -> int64_t { return row_off(p.chain.steps[s], mbase); };
        // Rows past M read the last row; computed where used, per element.
        const auto row = [&](int e) -> int64_t {
            const int64_t m = opaque(mbase) + tile_row(e);
            return m < p.M ? m : p.M - 1;
        };
        if (GATED) {
            const int64_t f = n0 + 32 * wc + col;
            const int64_t fc = f < p.half ? f : p.half - 1;
            float xv[16], gv[16];
            const float fx = up(fc), fg = up(p.half + fc);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                xv[e] = acc[i][0][e] * fx;
                gv[e] = acc[i][1][e] * fg;
            }
            apply_chain_tile(
                p.chain, xv, full, [&](int s) { return fc * p.chain.steps[s].nb[0] + first(s); }, stride,
                [&](int s, int e) { return fc * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e)); });
            apply_chain_tile(
                p.chain, gv, full, [&](int s) { return (p.half + fc) * p.chain.steps[s].nb[0] + first(s); }, stride,
                [&](int s, int e) {
                    return (p.half + fc) * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e));
                });
            if (f >= p.half) continue;
            float *out = p.y + mbase * p.ldy + f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                if (full || mbase + tile_row(e) < p.M) out[tile_row(e) * p.ldy] = xv[e] * gelu(gv[e]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int64_t n = n0 + wc * 32 * TN + 32 * j + col;
                const int64_t nc = n < p.N ? n : p.N - 1;
                float v[16];
                const float f = up(nc);
#pragma unroll
                for (int e = 0; e < 16; ++e) v[e] = acc[i][j][e] * f;
                float *out = p.y + mbase * p.ldy + nc;
                if (p.from_redirect) {
                    float r[16];
#pragma unroll
                    for (int e = 0; e < 16; ++e) r[e] = full ? out[tile_row(e) * p.ldy] : p.y[row(e) * p.ldy + nc];
#pragma unroll
                    for (int e = 0; e < 16; ++e) v[e] = __fadd_rn(r[e], v[e]);
                }
                apply_chain_tile(
                    p.chain, v, full, [&](int s) { return nc * p.chain.steps[s].nb[0] + first(s); }, stride,
                    [&](int s, int e) { return nc * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e)); });
                if (n >= p.N) continue;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    if (full || mbase + tile_row(e) < p.M) out[tile_row(e) * p.ldy] = v[e];
                }
            }
        }
    }
}

// ------------------------------------------------------------------ MUL_MAT by panels

// MUL_MAT where the output holds many panels of BM tokens by BN features: 64
// by 160 (the UNet's 64 x 64 level, configs[0]), or 64 by 64 where those leave
// too few (the 32 x 32 level).  A workgroup of 4
// waves, BM / 32 along the tokens by 128 / BM along the features, each wave
// 32 tokens by TNW tiles of 16 features as 2 x TNW tiles of
// v_mfma_f32_16x16x32_f16 with W as operand A (features) and x as operand B
// (tokens, split), so that a lane holds 4 consecutive features of one token
// and stores them as one float4.
// K goes in chunks of 64 through two LDS buffers: each chunk of x (64 tokens
// by 64, single precision, rows of 256 bytes) and of W (160 features by 64
// halves, rows of 128 bytes) loaded by whole rows -- every load a full
// 128-byte line -- into registers one chunk ahead, x split into its FP16
// parts once for the workgroup, both written to LDS with each row's 16-byte
// piece p at p ^ ((row >> 1) & 7), so that the 16 rows a fragment read
// takes fall in 16 distinct groups of banks.  Rows past M and features past
// N read the last row and are not stored.  The panels are BM tokens by BN
// features (PanelShape below), K in chunks of kPanelK.
constexpr int kPanelK = 64;

// The panel shapes, by preference: the first that gives 256 panels or more.
struct PanelShape {
    int bm, bn;
};
// (Panels of 32 by 64 for the 16 x 16 level were measured slower there than
// the 64 x 64 core split along K: the UNet step 11.52 -> 11.62 ms.)
constexpr PanelShape kPanelShapes[] = {{64, 160}, {64, 64}};

__device__ __forceinline__ int panel_swizzle(int row) { return (row >> 1) & 7; }

// With `part`, the panels split along K: block b takes split b / panels, of
// split_chunks chunks, and writes its sums, no chain, to part[s][m][n] for
// mul_mat_sum_kernel, as the 64 x 64 core's splits do.
template <bool GENERIC, int BM, int BN>
__global__ __launch_bounds__(256) void mul_mat_panel_kernel(MulMatArgs p, float *__restrict__ part,
                                                            int64_t split_chunks) {
    constexpr int KC = kPanelK;
    constexpr int WR = BM / 32, WC = 4 / WR;        // waves along the tokens, the features
    constexpr int TMW = 2, TNW = BN / (16 * WC);    // tiles of 16 a wave
    constexpr int XQ = BM * (KC / 4) / 256;         // float4 of x a thread a chunk
    constexpr int WQ = BN * (KC / 8) / 256;         // half8 of W a thread a chunk
    static_assert(BM * (KC / 4) % 256 == 0 && BN * (KC / 8) % 256 == 0, "whole pieces a thread");
    static_assert(WR * WC == 4 && TNW * 16 * WC == BN, "the waves tile the panel");
    __shared__ __attribute__((aligned(16))) _Float16 lx[2][2][BM * KC];  // [buffer][hi, lo][token][k]
    __shared__ __attribute__((aligned(16))) _Float16 lw[2][BN * KC];     // [buffer][feature][k]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave / WC, wc = wave % WC;
    const uint32_t b_all = xcd_swizzle(blockIdx.x, gridDim.x);
    const uint32_t panels = static_cast<uint32_t>(((p.M + BM - 1) / BM) * p.col_blocks);
    const uint32_t split = part != nullptr ? b_all / panels : 0;
    const uint32_t b = b_all - split * panels;
    const int64_t m0 = static_cast<int64_t>(b / p.col_blocks) * BM;
    const int64_t n0 = static_cast<int64_t>(b % p.col_blocks) * BN;
    const int64_t chunks_all = p.K / KC;
    const int64_t c_begin = part != nullptr ? static_cast<int64_t>(split) * split_chunks : 0;
    const int64_t chunks =
        part != nullptr ? (c_begin + split_chunks < chunks_all ? c_begin + split_chunks : chunks_all) : chunks_all;
    const float *xs[XQ];
    int xoff[XQ];
#pragma unroll
    for (int u = 0; u < XQ; ++u) {
        const int idx = tid + 256 * u, r = idx >> 4, q = idx & 15;
        const int64_t m = m0 + r < p.M ? m0 + r : p.M - 1;
        xs[u] = p.x + m * p.ldx + 4 * q;
        xoff[u] = r * KC + ((((q >> 1) ^ panel_swizzle(r)) << 3) | ((q & 1) << 2));
    }
    const _Float16 *ws[WQ];
    int woff[WQ];
#pragma unroll
    for (int u = 0; u < WQ; ++u) {
        const int idx = tid + 256 * u, r = idx >> 3, q = idx & 7;
        const int64_t n = n0 + r < p.N ? n0 + r : p.N - 1;
        ws[u] = p.w + n * p.ldw + 8 * q;
        woff[u] = r * KC + ((q ^ panel_swizzle(r)) << 3);
    }
    float4v xr[XQ];
    half8 wg[WQ];
    const auto load = [&](int64_t c) {
#pragma unroll
        for (int u = 0; u < XQ; ++u) xr[u] = *reinterpret_cast<const float4v *>(xs[u] + KC * c);
#pragma unroll
        for (int u = 0; u < WQ; ++u) wg[u] = *reinterpret_cast<const half8 *>(ws[u] + KC * c);
    };
    const auto store = [&](int buf) {
#pragma unroll
        for (int u = 0; u < XQ; ++u) {
            half4 h, l;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                _Float16 a, c;
                split2(xr[u][e], a, c);
                h[e] = a;
                l[e] = c;
            }
            *reinterpret_cast<half4 *>(&lx[buf][0][xoff[u]]) = h;
            *reinterpret_cast<half4 *>(&lx[buf][1][xoff[u]]) = l;
        }
#pragma unroll
        for (int u = 0; u < WQ; ++u) *reinterpret_cast<half8 *>(&lw[buf][woff[u]]) = wg[u];
    };
    const int col = lane & 15, kq = lane >> 4;
    float4v acc[TNW][TMW];
#pragma unroll
    for (int j = 0; j < TNW; ++j)
#pragma unroll
        for (int i = 0; i < TMW; ++i) acc[j][i] = float4v{};
    load(c_begin);
    store(0);
    lds_barrier();
    for (int64_t c = c_begin; c < chunks; ++c) {
        const int buf = static_cast<int>((c - c_begin) & 1);
        if (c + 1 < chunks) load(c + 1);
#pragma unroll
        for (int h = 0; h < KC / 32; ++h) {
            half8 a[TNW], bh[TMW], bl[TMW];
#pragma unroll
            for (int j = 0; j < TNW; ++j) {
                const int r = wc * 16 * TNW + 16 * j + col;
                a[j] = *reinterpret_cast<const half8 *>(&lw[buf][r * KC + (((4 * h + kq) ^ panel_swizzle(r)) << 3)]);
            }
#pragma unroll
            for (int i = 0; i < TMW; ++i) {
                const int r = wr * 16 * TMW + 16 * i + col;
                const int o = r * KC + (((4 * h + kq) ^ panel_swizzle(r)) << 3);
                bh[i] = *reinterpret_cast<const half8 *>(&lx[buf][0][o]);
                bl[i] = *reinterpret_cast<const half8 *>(&lx[buf][1][o]);
            }
            // Every tile's high parts, then every tile's low parts: no MFMA
            // waits on the one just before it.
#pragma unroll
            for (int j = 0; j < TNW; ++j)
#pragma unroll
                for (int i = 0; i < TMW; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], bh[i], acc[j][i], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < TNW; ++j)
#pragma unroll
                for (int i = 0; i < TMW; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], bl[i], acc[j][i], 0, 0, 0);
        }
        if (c + 1 < chunks) store(buf ^ 1);
        lds_barrier();
    }

    // The epilogue: the lane's 2 tokens m and, per tile, 4 features n .. n +
    // 3.  The chain a step at a time over all 10 tiles, every load of a step
    // issued before any is used.  !GENERIC (the host's choice, panel_chain_fast):
    // N whole panels, the output's rows and every operand contiguous along the
    // features and 16-byte aligned at every row, or one number a token -- each
    // read as float4 or once; GENERIC: any operand, element by element where
    // it is neither.
    const uint32_t ne1 = static_cast<uint32_t>(p.ne1), ne2 = static_cast<uint32_t>(p.ne2);
    const bool whole = !GENERIC || n0 + BN <= p.N;
    const bool vy = !GENERIC || (whole && p.ldy % 4 == 0 && (reinterpret_cast<uintptr_t>(p.y) & 15) == 0);
    int64_t mc[TMW];
    uint32_t i1[TMW], i2[TMW], i3[TMW];
#pragma unroll
    for (int i = 0; i < TMW; ++i) {
        const int64_t m = m0 + wr * 16 * TMW + 16 * i + col;
        mc[i] = m < p.M ? m : p.M - 1;
        split_index(static_cast<uint32_t>(mc[i]), ne1, ne2, i1[i], i2[i], i3[i]);
    }
    int64_t nf[TNW];  // the tile's first feature (clamped: never past N - 4 where whole)
#pragma unroll
    for (int j = 0; j < TNW; ++j) nf[j] = n0 + wc * 16 * TNW + 16 * j + 4 * kq;
    float v[TMW][TNW][4];
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[i][j][e] = acc[j][i][e] * kSplitUp;
    if (part != nullptr) {
        // A split's sums, rows of N, a float4 where the four lie inside N.
        float *ps = part + static_cast<int64_t>(split) * p.M * p.N;
        const bool v4 = p.N % 4 == 0;
#pragma unroll
        for (int i = 0; i < TMW; ++i) {
            const int64_t m = m0 + wr * 16 * TMW + 16 * i + col;
            if (m >= p.M) continue;
#pragma unroll
            for (int j = 0; j < TNW; ++j) {
                if (v4 && nf[j] + 3 < p.N) {
                    *reinterpret_cast<float4v *>(ps + m * p.N + nf[j]) =
                        float4v{v[i][j][0], v[i][j][1], v[i][j][2], v[i][j][3]};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (nf[j] + e < p.N) ps[m * p.N + nf[j] + e] = v[i][j][e];
                }
            }
        }
        return;
    }
    // Element e of tile (i, j) of a tensor of the output's rows ld apart.
    const auto at = [&](int i, int j, int e) -> int64_t {
        const int64_t n = nf[j] + e;
        return mc[i] * p.ldy + (n < p.N ? n : p.N - 1);
    };
    if (p.from_redirect) {
        float r[TMW][TNW][4];
#pragma unroll
        for (int i = 0; i < TMW; ++i)
#pragma unroll
            for (int j = 0; j < TNW; ++j) {
                if (vy) {
                    const float4v q = *reinterpret_cast<const float4v *>(p.y + mc[i] * p.ldy + nf[j]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) r[i][j][e] = q[e];
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) r[i][j][e] = p.y[at(i, j, e)];
                }
            }
#pragma unroll
        for (int i = 0; i < TMW; ++i)
#pragma unroll
            for (int j = 0; j < TNW; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) v[i][j][e] = __fadd_rn(r[i][j][e], v[i][j][e]);
    }
#pragma unroll 1
    for (int s = 0; s < p.chain.count; ++s) {
        const DevStep &st = p.chain.steps[s];
        if (st.kind == kSilu) {
#pragma unroll
            for (int i = 0; i < TMW; ++i)
#pragma unroll
                for (int j = 0; j < TNW; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[i][j][e] = silu(v[i][j][e]);
            continue;
        }
        const float *base[TMW];
#pragma unroll
        for (int i = 0; i < TMW; ++i)
            base[i] = st.operand + (st.flat123 ? mc[i] * st.nb[1] : i1[i] * st.nb[1] + i2[i] * st.nb[2] + i3[i] * st.nb[3]);
        const bool rows16 = st.flat123 ? st.nb[1] % 4 == 0 : st.nb[1] % 4 == 0 && st.nb[2] % 4 == 0 && st.nb[3] % 4 == 0;
        const bool vec = !GENERIC || (whole && st.nb[0] == 1 && rows16 && (reinterpret_cast<uintptr_t>(st.operand) & 15) == 0);
        float o[TMW][TNW][4];
        if (st.nb[0] == 0) {
#pragma unroll
            for (int i = 0; i < TMW; ++i) {
                const float bv = *base[i];
#pragma unroll
                for (int j = 0; j < TNW; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[i][j][e] = bv;
            }
        } else if (vec) {
#pragma unroll
            for (int i = 0; i < TMW; ++i)
#pragma unroll
                for (int j = 0; j < TNW; ++j) {
                    const float4v q = *reinterpret_cast<const float4v *>(base[i] + nf[j]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[i][j][e] = q[e];
                }
        } else if (GENERIC) {
#pragma unroll
            for (int i = 0; i < TMW; ++i)
#pragma unroll
                for (int j = 0; j < TNW; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int64_t n = nf[j] + e;
                        o[i][j][e] = base[i][(n < p.N ? n : p.N - 1) * st.nb[0]];
                    }
        }
        if (st.kind == kAdd) {
#pragma unroll
            for (int i = 0; i < TMW; ++i)
#pragma unroll
                for (int j = 0; j < TNW; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[i][j][e] = __fadd_rn(v[i][j][e], o[i][j][e]);
        } else {
#pragma unroll
            for (int i = 0; i < TMW; ++i)
#pragma unroll
                for (int j = 0; j < TNW; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[i][j][e] = __fmul_rn(v[i][j][e], o[i][j][e]);
        }
    }
#pragma unroll
    for (int i = 0; i < TMW; ++i) {
        if (m0 + wr * 16 * TMW + 16 * i + col >= p.M) continue;
#pragma unroll
        for (int j = 0; j < TNW; ++j) {
            if (vy) {
                *reinterpret_cast<float4v *>(p.y + mc[i] * p.ldy + nf[j]) =
                    float4v{v[i][j][0], v[i][j][1], v[i][j][2], v[i][j][3]};
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (nf[j] + e < p.N) p.y[mc[i] * p.ldy + nf[j] + e] = v[i][j][e];
            }
        }
    }
}

// ------------------------------------------------------------------ 1x1 convolution by panels

// The 1x1 convolution (stride 1, no padding) by the MUL_MAT panels' product,
// C[oc][position] = sum_ic W[oc][ic] x[ic][position]: a workgroup's panel is
// 64 positions of one image by 160 output channels, W operand A as MUL_MAT's
// weights (channels), the image's columns operand B (positions, split).  A
// chunk of 64 input channels of x comes in as rows of 64 positions (256
// bytes), a thread 4 channels by 4 positions, transposed in registers and
// written to LDS as [position][channel] with the panels' swizzle; the
// outputs go back through LDS as [oc][position], so that the chain and the
// stores take rows of 64 positions, a float4 a thread.  Channels past OC read
// the last and are not stored.
constexpr int kConvPanelPositions = 64, kConvPanelChannels = 160, kConvStageRow = 68, kConvPanelStages = 2;

// The 16-byte piece p of x's LDS row r at p ^ conv_swizzle(r): 16 consecutive
// rows (an MFMA operand's read) take 8 distinct swizzles among their even
// rows and among their odd ones, and so do the rows 8 m + e of a write.
__device__ __forceinline__ int conv_swizzle(int row) { return ((row >> 1) ^ (row >> 3)) & 7; }

template <int NS>
__global__ __launch_bounds__(512) void conv_panel_kernel(ConvArgs c) {
    constexpr int BM = kConvPanelPositions, BN = kConvPanelChannels, KC = kPanelK;
    constexpr int TNW = 5;                   // a wave's tiles of 16 channels, by one tile of 16 positions
    constexpr int WQ = BN * (KC / 8) / 256;  // half8 of W a thread of the W waves a chunk
    static_assert(BM * KC == 256 * 16 && BN * (KC / 8) % 256 == 0, "whole pieces a thread");
    static_assert(BN * kConvStageRow * 4 <= (2 * 2 * BM * KC + 2 * BN * KC) * 2, "the outputs fit the operands' LDS");
    __shared__ __attribute__((aligned(16))) _Float16 lds[2 * 2 * BM * KC + 2 * BN * KC];
    _Float16 (*lx)[2][BM * KC] = reinterpret_cast<_Float16 (*)[2][BM * KC]>(lds);  // [buffer][hi, lo][position][k]
    _Float16 (*lw)[BN * KC] = reinterpret_cast<_Float16 (*)[BN * KC]>(lds + 2 * 2 * BM * KC);  // [buffer][oc][k]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Waves 0 .. 3 load x, 4 .. 7 W; wave w computes positions 16 (w & 3) ..
    // by channels 80 (w >> 2) ...
    const bool loads_x = wave < 4;
    const int t = tid & 255;
    const int wr = wave & 3, wc = wave >> 2;
    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t pos0 = static_cast<int64_t>(b / c.oc_blocks) * BM;
    const int64_t oc0 = static_cast<int64_t>(b % c.oc_blocks) * BN;
    const int64_t n = pos0 / c.plane, p0 = pos0 - n * c.plane;  // a panel lies in one image
    const int64_t chunks = c.K / KC;
    // x: the thread's 4 positions 4 pq .. and channels 4 kq + u, u = 0 .. 3,
    // its e-th write to LDS position 4 pq + (e ^ (pq & 1)): the 32 lanes of a
    // write then take rows of both parities, which conv_swizzle spreads over
    // all 64 banks.
    const int pq = t & 15, kq = t >> 4, par = pq & 1;
    const float *xs = c.x + n * c.xnb3 + static_cast<int64_t>(4 * kq) * c.xnb2 + p0 + 4 * pq;
    int xoff[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int r = 4 * pq + (e ^ par);
        xoff[e] = r * KC + ((((kq >> 1) ^ conv_swizzle(r)) << 3) | ((kq & 1) << 2));
    }
    const _Float16 *ws[WQ];
    int woff[WQ];
#pragma unroll
    for (int u = 0; u < WQ; ++u) {
        const int idx = t + 256 * u, r = idx >> 3, q = idx & 7;
        const int64_t o = oc0 + r < c.oc ? oc0 + r : c.oc - 1;
        ws[u] = c.w + o * c.ldw + 8 * q;
        woff[u] = r * KC + ((q ^ panel_swizzle(r)) << 3);
    }
    // NS register stages: at the top of chunk t, stage (t + q) % NS holds the
    // loads of chunk t + q; chunks past the last repeat it, so that every load
    // is unconditional.  A wave's stages hold x's or W's pieces, by its kind.
    float4v xr[NS][4];
    half8 wg[NS][WQ];
    const auto load = [&](int st, int64_t ch) {
        const int64_t k = ch < chunks ? ch : chunks - 1;
        if (loads_x) {
#pragma unroll
            for (int u = 0; u < 4; ++u) xr[st][u] = *reinterpret_cast<const float4v *>(xs + (KC * k + u) * c.xnb2);
        } else {
#pragma unroll
            for (int u = 0; u < WQ; ++u) wg[st][u] = *reinterpret_cast<const half8 *>(ws[u] + KC * k);
        }
    };
    const auto store = [&](int st, int buf) {
        if (loads_x) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                half4 h, l;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    _Float16 a, d;
                    split2(par ? xr[st][u][e ^ 1] : xr[st][u][e], a, d);
                    h[u] = a;
                    l[u] = d;
                }
                *reinterpret_cast<half4 *>(&lx[buf][0][xoff[e]]) = h;
                *reinterpret_cast<half4 *>(&lx[buf][1][xoff[e]]) = l;
            }
        } else {
#pragma unroll
            for (int u = 0; u < WQ; ++u) *reinterpret_cast<half8 *>(&lw[buf][woff[u]]) = wg[st][u];
        }
    };
    const int col = lane & 15, kp = lane >> 4;
    float4v acc[TNW];
#pragma unroll
    for (int j = 0; j < TNW; ++j) acc[j] = float4v{};
    const auto compute = [&](int buf) {
#pragma unroll
        for (int h = 0; h < KC / 32; ++h) {
            half8 a[TNW];
#pragma unroll
            for (int j = 0; j < TNW; ++j) {
                const int r = wc * 16 * TNW + 16 * j + col;
                a[j] = *reinterpret_cast<const half8 *>(&lw[buf][r * KC + (((4 * h + kp) ^ panel_swizzle(r)) << 3)]);
            }
            const int r = 16 * wr + col;
            const int o = r * KC + (((4 * h + kp) ^ conv_swizzle(r)) << 3);
            const half8 bh = *reinterpret_cast<const half8 *>(&lx[buf][0][o]);
            const half8 bl = *reinterpret_cast<const half8 *>(&lx[buf][1][o]);
#pragma unroll
            for (int j = 0; j < TNW; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], bh, acc[j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < TNW; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[j], bl, acc[j], 0, 0, 0);
        }
    };
#pragma unroll
    for (int q = 0; q < NS; ++q) load(q, q);
    store(0, 0);
    lds_barrier();
    // Passes of U chunks, U a multiple of NS and of 2, so that stages and
    // buffers are the same at every pass: chunk t's MFMAs from buffer t % 2,
    // chunk t + 1 into the other, the loads of chunk t + NS into the stage
    // chunk t freed.
    constexpr int U = NS % 2 == 0 ? NS : 2 * NS;
    for (int64_t t0 = 0; t0 < chunks; t0 += U) {
#pragma unroll
        for (int q = 0; q < U; ++q) {
            if (t0 + q < chunks) compute(q & 1);
            store((q + 1) % NS, (q + 1) & 1);
            load(q % NS, t0 + q + NS);
            lds_barrier();
        }
    }

    // The outputs into LDS, [oc][position] in rows of kConvStageRow floats
    // (rows 4 apart fall 16 banks apart): the lane's 4 channels 4 kp .. of
    // position col of each tile.
    float *stage = reinterpret_cast<float *>(lds);
#pragma unroll
    for (int j = 0; j < TNW; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
            stage[(wc * 16 * TNW + 16 * j + 4 * kp + e) * kConvStageRow + 16 * wr + col] = acc[j][e] * kSplitUp;
    lds_barrier();
    // A float4 of a row a thread at a time: channel r = f / 16, positions
    // 4 (f % 16) ..; the residual in the output's memory first, then the
    // chain a step at a time, every load of a step before any is used.
    constexpr int RQ = BN * (BM / 4) / 512;
    int64_t oc[RQ], pp[RQ];
    float v[RQ][4];
#pragma unroll
    for (int u = 0; u < RQ; ++u) {
        const int f = tid + 512 * u, r = f >> 4, q = f & 15;
        oc[u] = oc0 + r < c.oc ? oc0 + r : c.oc - 1;
        pp[u] = p0 + 4 * q;
        const float4v t = *reinterpret_cast<const float4v *>(&stage[r * kConvStageRow + 4 * q]);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[u][e] = t[e];
    }
    float *out = c.y + n * c.ynb3;
    if (c.from_redirect) {
        float4v r[RQ];
#pragma unroll
        for (int u = 0; u < RQ; ++u) r[u] = *reinterpret_cast<const float4v *>(out + oc[u] * c.ynb2 + pp[u]);
#pragma unroll
        for (int u = 0; u < RQ; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[u][e] = __fadd_rn(r[u][e], v[u][e]);
    }
#pragma unroll 1
    for (int s = 0; s < c.chain.count; ++s) {
        const DevStep &st = c.chain.steps[s];
        if (st.kind == kSilu) {
#pragma unroll
            for (int u = 0; u < RQ; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) v[u][e] = silu(v[u][e]);
            continue;
        }
        const float *base = st.operand + n * st.nb[3];
        float o[RQ][4];
        if (st.nb[0] == 0 && st.nb[1] == 0) {
            // One number a channel (the bias).
#pragma unroll
            for (int u = 0; u < RQ; ++u) {
                const float q = base[oc[u] * st.nb[2]];
#pragma unroll
                for (int e = 0; e < 4; ++e) o[u][e] = q;
            }
        } else if (st.nb[0] == 1 && st.flat01 && st.nb[2] % 4 == 0 && st.nb[3] % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(st.operand) & 15) == 0) {
#pragma unroll
            for (int u = 0; u < RQ; ++u) {
                const float4v q = *reinterpret_cast<const float4v *>(base + oc[u] * st.nb[2] + pp[u]);
#pragma unroll
                for (int e = 0; e < 4; ++e) o[u][e] = q[e];
            }
        } else {
#pragma unroll
            for (int u = 0; u < RQ; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t p = pp[u] + e, oy = p / c.ow, ox = p - oy * c.ow;
                    o[u][e] = base[oc[u] * st.nb[2] + ox * st.nb[0] + oy * st.nb[1]];
                }
        }
        if (st.kind == kAdd) {
#pragma unroll
            for (int u = 0; u < RQ; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) v[u][e] = __fadd_rn(v[u][e], o[u][e]);
        } else {
#pragma unroll
            for (int u = 0; u < RQ; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) v[u][e] = __fmul_rn(v[u][e], o[u][e]);
        }
    }
#pragma unroll
    for (int u = 0; u < RQ; ++u) {
        if (oc0 + ((tid + 512 * u) >> 4) >= c.oc) continue;
        *reinterpret_cast<float4v *>(out + oc[u] * c.ynb2 + pp[u]) = float4v{v[u][0], v[u][1], v[u][2], v[u][3]};
    }
}

// ------------------------------------------------------------------ MUL_MAT split along K

// Products of few output blocks and long K (the UNet's deepest level, 512
// tokens by 1280 features): partial sums of splits of K in blocks of 64 x 64
// (part[s][m][n]), then added in their order with the chain applied, as the
// single-pass epilogue does.  Both operands as in mul_mat_kernel, whole
// K-steps, rows 16-byte aligned.
template <int NS>
__global__ __launch_bounds__(256) void mul_mat_split_kernel(MulMatArgs p, int64_t split_len,
                                                            float *__restrict__ part) {
    constexpr int BM = 64, BN = 64;
    __shared__ __attribute__((aligned(16))) _Float16 lds[lds_halves<1, 1, kSplitA>()];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave >> 1;
    const int wc = wave & 1;

    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t per_split = ((p.M + BM - 1) / BM) * p.col_blocks;
    const int64_t sp = b / per_split;
    const int64_t rem = b - sp * per_split;
    const int64_t mb = rem / p.col_blocks;  // neighbouring blocks share rows of x
    const int64_t nb = rem - mb * p.col_blocks;
    const int64_t m0 = mb * BM, n0 = nb * BN;
    const int64_t k_begin = sp * split_len;
    const int64_t k_len = p.K - k_begin < split_len ? p.K - k_begin : split_len;

    float16v acc[1][1];
    acc[0][0] = float16v{};
    F32Rows<BM, true, true> xa[NS];
    F16Rows<BN, true, true> wb[NS];
    const auto x_row = [&](int r) -> int64_t { return m0 + r < p.M ? m0 + r : -1; };
    const auto w_row = [&](int r) -> int64_t { return n0 + r < p.N ? n0 + r : -1; };
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        xa[q].init(p.x + k_begin, p.ldx, x_row, k_len, tid);
        wb[q].init(p.w + k_begin, p.ldw, w_row, k_len, tid);
    }
    main_loop<1, 1, kSplitA, NS>(acc, xa, wb, lds, k_len / kBK, tid, lane, wr, wc);

    // x was scaled by 2^-4 in its split.
    const int64_t n = n0 + wc * 32 + (lane & 31);
    if (n >= p.N) return;
    const int64_t mbase = m0 + wr * 32 + 4 * (lane >> 5);
    float *out = part + sp * p.M * p.N + n;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int64_t m = mbase + tile_row(e);
        if (m < p.M) out[m * p.N] = acc[0][0][e] * kSplitUp;
    }
}

__global__ __launch_bounds__(256) void mul_mat_sum_kernel(MulMatArgs p, const float *__restrict__ part,
                                                          int64_t splits) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t plane = p.M * p.N;
    if (t >= plane) return;
    const int64_t m = t / p.N, n = t - m * p.N;
    float v = part[t];
    for (int64_t sp = 1; sp < splits; ++sp) v = __fadd_rn(v, part[sp * plane + t]);
    float *out = p.y + m * p.ldy + n;
    if (p.from_redirect) v = __fadd_rn(*out, v);
    float vv[1] = {v};
    const uint32_t ne1 = static_cast<uint32_t>(p.ne1), ne2 = static_cast<uint32_t>(p.ne2);
    apply_chain_block<1>(p.chain, vv, [&](int s, int) -> int64_t {
        const DevStep &st = p.chain.steps[s];
        if (st.flat123) return n * st.nb[0] + m * st.nb[1];
        uint32_t i1, i2, i3;
        split_index(static_cast<uint32_t>(m), ne1, ne2, i1, i2, i3);
        return n * st.nb[0] + i1 * st.nb[1] + i2 * st.nb[2] + i3 * st.nb[3];
    });
    *out = vv[0];
}

// ------------------------------------------------------------------ direct convolution

// y[n][oc][pos] = sum_k W[oc][k] columns[k][pos], the chain applied; W rows
// K-contiguous FP16 (the kernel as ggml holds it, [OC][IC][KH][KW]).
template <int TM, int TN, bool POINTWISE, bool VECW, bool FULL, int NS, bool K3 = false, int WP = 1,
          int HALF = 0>
__global__ __launch_bounds__(256) void conv_direct_kernel(ConvArgs c) {
    constexpr int BM = 64 * TM;  // output channels
    constexpr int BN = 64 * TN;  // positions
    // WP as mul_mat_kernel's: split single-precision kernels in two planes;
    // HALF, the products of 16 bits: the columns rounded to FP16 (1), or both
    // operands to bfloat16 (2).
    static_assert(!HALF || WP == 1, "products of 16 bits take FP16 kernels");
    constexpr int MODE = HALF == 2 ? kBf16 : HALF ? kSplitNone : WP == 2 ? kSplitBoth : kSplitB;
    __shared__ __attribute__((aligned(16))) _Float16 lds[lds_halves<TM, TN, MODE>()];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave >> 1;
    const int wc = wave & 1;

    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t pb = b / c.oc_blocks;  // neighbouring blocks share positions
    const int64_t ob = b % c.oc_blocks;
    const int64_t oc0 = ob * BM;
    const int64_t p0 = pb * BN;
    const auto w_row = [&](int r) -> int64_t { return oc0 + r < c.oc ? oc0 + r : -1; };

    float16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = float16v{};

    F16Rows<BM, VECW, FULL, WP, false, HALF == 2> wa[NS];
    Columns<BN, POINTWISE, FULL, K3, !HALF, HALF == 2> xb[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        wa[s].init(c.w, c.ldw, w_row, c.K, tid, c.w_plane);
        xb[s].init(c, p0, tid);
    }
    main_loop<TM, TN, MODE, NS>(acc, wa, xb, lds, (c.K + kBK - 1) / kBK, tid, lane, wr, wc);

    // The epilogue: output channels oc down the tile, position lane % 32 across;
    // a tile wholly inside OC addresses its channels as a stride from its first.
    const int col = lane & 31;
    const int64_t lane_row = 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int64_t pos = p0 + wc * 32 * TN + 32 * j + col;
        if (pos >= c.P) continue;
        uint32_t ox, oy, n;
        split_index(static_cast<uint32_t>(pos), static_cast<uint32_t>(c.ow), static_cast<uint32_t>(c.oh), ox, oy, n);
        const int64_t at = static_cast<int64_t>(n) * c.ynb3 + static_cast<int64_t>(oy) * c.ynb1 + ox;
        const int64_t in_image = static_cast<int64_t>(oy) * c.ow + ox;
        const auto xyn = [&](const DevStep &st) -> int64_t {
            const int64_t xy =
                st.flat01 ? in_image * st.nb[0] : static_cast<int64_t>(ox) * st.nb[0] + static_cast<int64_t>(oy) * st.nb[1];
            return xy + static_cast<int64_t>(n) * st.nb[3];
        };
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int64_t tile0 = oc0 + wr * 32 * TM + 32 * i;
            const int64_t obase = tile0 + lane_row;
            const bool full = tile0 + 32 <= c.oc;
            // Channels past OC read the last and are not stored.
            const auto chan = [&](int e) -> int64_t {
                const int64_t oc = opaque(obase) + tile_row(e);
                return oc < c.oc ? oc : c.oc - 1;
            };
            float v[16];
            if (WP == 2) {
#pragma unroll
                for (int e = 0; e < 16; ++e) v[e] = acc[i][j][e] * (kSplitUp * c.w_scale[chan(e)]);
            } else {
#pragma unroll
                for (int e = 0; e < 16; ++e) v[e] = acc[i][j][e] * kSplitUp;
            }
            float *out = c.y + at + obase * c.ynb2;
            if (c.from_redirect) {
                float r[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) r[e] = full ? out[tile_row(e) * c.ynb2] : c.y[at + chan(e) * c.ynb2];
#pragma unroll
                for (int e = 0; e < 16; ++e) v[e] = __fadd_rn(r[e], v[e]);
            }
            apply_chain_tile(
                c.chain, v, full,
                [&](int s) { return xyn(c.chain.steps[s]) + obase * c.chain.steps[s].nb[2]; },
                [&](int s) { return c.chain.steps[s].nb[2]; },
                [&](int s, int e) { return xyn(c.chain.steps[s]) + chan(e) * c.chain.steps[s].nb[2]; });
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                if (full || obase + tile_row(e) < c.oc) out[tile_row(e) * c.ynb2] = v[e];
            }
        }
    }
}

// ------------------------------------------------------------------ convolution by columns

// The direct convolution of kernels other than 1x1 as an explicit im2col and
// a product split along K: the columns gathered once (columns_kernel), the
// split products of the FP16 weights by the split columns into partial sums
// (conv_columns_kernel, as many splits as fill the chip when the output has
// few blocks -- the deep, long-K layers), and the splits added in their
// order with the chain applied (conv_sum_kernel).  K = IC KH KW a multiple
// of the K-step.

// cols[p][k] for positions p and k = (ic, kh, kw), zeros outside the image;
// a thread four consecutive k of one position.
template <bool K3>
__global__ __launch_bounds__(256) void columns_kernel(ConvArgs c, float *__restrict__ cols) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t quads = c.K / 4;
    if (t >= c.P * quads) return;
    const int64_t p = t / quads;
    const uint32_t k0 = static_cast<uint32_t>(t - p * quads) * 4;
    uint32_t ox, oy, n;
    split_index(static_cast<uint32_t>(p), static_cast<uint32_t>(c.ow), static_cast<uint32_t>(c.oh), ox, oy, n);
    const int32_t iy0 = static_cast<int32_t>(oy) * c.s1 - c.p1;
    const int32_t ix0 = static_cast<int32_t>(ox) * c.s0 - c.p0;
    const float *img = c.x + static_cast<int64_t>(n) * c.xnb3;
    const uint32_t taps = K3 ? 9u : static_cast<uint32_t>(c.taps);
    const uint32_t kwidth = K3 ? 3u : static_cast<uint32_t>(c.kw);
    float4 v;
    float *ve = reinterpret_cast<float *>(&v);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t k = k0 + e;
        const uint32_t ic = k / taps;
        const uint32_t tap = k - ic * taps;
        const uint32_t kh = tap / kwidth;
        const uint32_t kw = tap - kh * kwidth;
        const int32_t iy = iy0 + static_cast<int32_t>(kh) * c.d1;
        const int32_t ix = ix0 + static_cast<int32_t>(kw) * c.d0;
        ve[e] = (iy >= 0 && iy < c.ih && ix >= 0 && ix < c.iw)
                    ? img[static_cast<int64_t>(ic) * c.xnb2 + static_cast<int64_t>(iy) * c.xnb1 + ix]
                    : 0.0f;
    }
    *reinterpret_cast<float4 *>(cols + p * c.K + k0) = v;
}

// part[s][oc][p] = 16 sum over split s's k of W[oc][k] cols[p][k]: blocks of
// 64 output channels by 64 positions, the splits of split_len (a multiple of
// the K-step) one after the other in the grid.
template <int NS, int WP = 1, int HALF = 0>
__global__ __launch_bounds__(256) void conv_columns_kernel(ConvArgs c, const float *__restrict__ cols,
                                                           int64_t split_len, int64_t p_blocks,
                                                           float *__restrict__ part) {
    constexpr int BM = 64, BN = 64;
    constexpr int MODE = HALF == 2 ? kBf16 : HALF ? kSplitNone : WP == 2 ? kSplitBoth : kSplitB;
    __shared__ __attribute__((aligned(16))) _Float16 lds[lds_halves<1, 1, MODE>()];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave >> 1;
    const int wc = wave & 1;

    const uint32_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t per_split = c.oc_blocks * p_blocks;
    const int64_t sp = b / per_split;
    const int64_t rem = b - sp * per_split;
    const int64_t pb = rem / c.oc_blocks;  // neighbouring blocks share positions
    const int64_t ob = rem - pb * c.oc_blocks;
    const int64_t oc0 = ob * BM, p0 = pb * BN;
    const int64_t k_begin = sp * split_len;
    const int64_t k_len = c.K - k_begin < split_len ? c.K - k_begin : split_len;

    float16v acc[1][1];
    acc[0][0] = float16v{};
    F16Rows<BM, true, true, WP, false, HALF == 2> wa[NS];
    F32Rows<BN, true, true, !HALF, HALF == 2> xb[NS];
    const auto w_row = [&](int r) -> int64_t { return oc0 + r < c.oc ? oc0 + r : -1; };
    const auto p_row = [&](int r) -> int64_t { return p0 + r < c.P ? p0 + r : -1; };
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        wa[q].init(c.w + k_begin, c.ldw, w_row, k_len, tid, c.w_plane);
        xb[q].init(cols + k_begin, c.K, p_row, k_len, tid);
    }
    main_loop<1, 1, MODE, NS>(acc, wa, xb, lds, k_len / kBK, tid, lane, wr, wc);

    // The columns were scaled by 2^-4 in their split.
    const int64_t pos = p0 + wc * 32 + (lane & 31);
    if (pos >= c.P) return;
    const int64_t obase = oc0 + wr * 32 + 4 * (lane >> 5);
    float *out = part + sp * c.oc * c.P + pos;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const int64_t oc = obase + tile_row(e);
        if (oc < c.oc) out[oc * c.P] = acc[0][0][e] * (WP == 2 ? kSplitUp * c.w_scale[oc] : kSplitUp);
    }
}

// y = the splits' partial sums added in their order, from the redirect's
// values if asked, and the chain (as the direct kernel's epilogue).
__global__ __launch_bounds__(256) void conv_sum_kernel(ConvArgs c, const float *__restrict__ part, int64_t splits) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t plane = c.oc * c.P;
    if (t >= plane) return;
    const int64_t oc = t / c.P, p = t - oc * c.P;
    float v = part[t];
    for (int64_t sp = 1; sp < splits; ++sp) v = __fadd_rn(v, part[sp * plane + t]);
    uint32_t ox, oy, n;
    split_index(static_cast<uint32_t>(p), static_cast<uint32_t>(c.ow), static_cast<uint32_t>(c.oh), ox, oy, n);
    const int64_t at = static_cast<int64_t>(n) * c.ynb3 + oc * c.ynb2 + static_cast<int64_t>(oy) * c.ynb1 + ox;
    if (c.from_redirect) v = __fadd_rn(c.y[at], v);
    float vv[1] = {v};
    const int64_t in_image = static_cast<int64_t>(oy) * c.ow + ox;
    apply_chain_block<1>(c.chain, vv, [&](int s, int) -> int64_t {
        const DevStep &st = c.chain.steps[s];
        const int64_t xy =
            st.flat01 ? in_image * st.nb[0] : static_cast<int64_t>(ox) * st.nb[0] + static_cast<int64_t>(oy) * st.nb[1];
        return xy + static_cast<int64_t>(n) * st.nb[3] + oc * st.nb[2];
    });
    c.y[at] = vv[0];
}

// ------------------------------------------------------------------ Winograd's products

// C[b][m][n] = sum_k A[b][m][k] B[b][n][k] for the batches b: A already split
// into two FP16 planes held in blocks of 32 of K, [k / 32][m][k % 32], or
// (SCALED) single precision K-contiguous rows with their columns scaled and
// split on their way into LDS; B already split into two FP16 planes in
// blocks, [k / 32][n][k % 32]; three MFMAs a product.
template <int TM, int TN, bool FULL, int NS, bool SCALED = false>
__global__ __launch_bounds__(256) void split_batched_kernel(SplitBatchedArgs p) {
    constexpr int BM = 64 * TM;
    constexpr int BN = 64 * TN;
    __shared__ __attribute__((aligned(16))) _Float16 lds[lds_halves<TM, TN, kSplitBoth>()];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave >> 1;
    const int wc = wave & 1;

    const int64_t per_batch = p.m_blocks * p.n_blocks;
    const uint32_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t batch = bid / per_batch;
    const int64_t rem = bid - batch * per_batch;
    const int64_t mb = rem / p.n_blocks;
    const int64_t nb = rem - mb * p.n_blocks;
    const int64_t m0 = mb * BM, n0 = nb * BN;
    const _Float16 *A = p.a + batch * p.a_batch;
    const _Float16 *B = p.b + batch * p.b_batch;
    float *C = p.c + batch * p.c_batch;

    float16v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = float16v{};

    using LA = std::conditional_t<SCALED, ScaledF32Rows<BM, FULL>, F16Rows<BM, true, FULL, 2, true>>;
    LA la[NS];
    F16Rows<BN, true, FULL, 2, true> lb[NS];
    const auto a_row = [&](int r) -> int64_t { return m0 + r < p.M ? m0 + r : -1; };
    const auto b_row = [&](int r) -> int64_t { return n0 + r < p.N ? n0 + r : -1; };
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        if constexpr (SCALED) {
            la[s].init(p.a32 + batch * p.a_batch, p.K, a_row, p.K, tid, p.a_scale);
        } else {
            la[s].init(A, kBK, a_row, p.K, tid, p.a_plane, p.M * kBK);
        }
        lb[s].init(B, kBK, b_row, p.K, tid, p.b_plane, p.N * kBK);
    }
    main_loop<TM, TN, kSplitBoth, NS>(acc, la, lb, lds, (p.K + kBK - 1) / kBK, tid, lane, wr, wc);

    // Both operands were scaled by 2^-4 in the split: the product by 2^-8.
    const int col = lane & 31;
    const int64_t lane_row = 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int64_t n = n0 + wc * 32 * TN + 32 * j + col;
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int64_t tile0 = m0 + wr * 32 * TM + 32 * i;
            const bool full = tile0 + 32 <= p.M;
            float *out = C + (tile0 + lane_row) * p.N + n;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                if (full || tile0 + lane_row + tile_row(e) < p.M) {
                    out[tile_row(e) * p.N] = acc[i][j][e] * (kSplitUp * kSplitUp);
                }
            }
        }
    }
}

// ------------------------------------------------------------------ launchers

template <int TM, int TN, bool GATED>
hipError_t launch_mul_mat_w32(const MulMatArgs &a, dim3 grid, hipStream_t stream) {
    // Split weights: rows 32-aligned and zero past K, so their loads are
    // always whole vectors; x's decide FULL.
    const bool vx = a.ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(a.x) % 16) == 0;
    const dim3 block(256);
    if (vx && a.K % kBK == 0) {
        SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, true, true, true, 2, 2>), grid, block, 0, stream, a);
    } else if (vx) {
        SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, true, true, false, 2, 2>), grid, block, 0, stream, a);
    } else {
        SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, false, true, false, 2, 2>), grid, block, 0, stream, a);
    }
    return hipGetLastError();
}

template <int TM, int TN, bool GATED>
hipError_t launch_mul_mat_t(const MulMatArgs &p, int stages, hipStream_t stream) {
    constexpr int BM = 64 * TM;
    constexpr int BN = 64 * TN;
    MulMatArgs a = p;
    const int64_t cols = GATED ? p.half : p.N;
    a.col_blocks = (cols + (GATED ? BN / 2 : BN) - 1) / (GATED ? BN / 2 : BN);
    const int64_t blocks = ((p.M + BM - 1) / BM) * a.col_blocks;
    const bool vx = p.ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(p.x) % 16) == 0;
    const bool vw = p.ldw % 8 == 0 && (reinterpret_cast<uintptr_t>(p.w) % 16) == 0;
    const bool full = vx && vw && p.K % kBK == 0;
    dim3 grid(static_cast<uint32_t>(blocks)), block(256);
    KernelScope scope(GATED ? "mul_mat_gated" : "mul_mat", stream);
    if (p.w_scale != nullptr) return launch_mul_mat_w32<TM, TN, GATED>(a, grid, stream);
    if (p.half16) {
        // The products of 16 bits, in FP16 (half16 1) or bfloat16 (2).
        const auto half = [&](auto form) {
            constexpr int H = decltype(form)::value;
            if (full) {
                SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, true, true, true, 2, 1, H>), grid, block, 0, stream, a);
            } else if (vx && vw) {
                SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, true, true, false, 2, 1, H>), grid, block, 0, stream, a);
            } else {
                SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, false, false, false, 2, 1, H>), grid, block, 0, stream,
                             a);
            }
        };
        if (p.half16 == 2) {
            half(std::integral_constant<int, 2>{});
        } else {
            half(std::integral_constant<int, 1>{});
        }
        return hipGetLastError();
    }
    if (full && stages == 4) {
        SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, true, true, true, 4>), grid, block, 0, stream, a);
    } else if (full) {
        SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, true, true, true, 2>), grid, block, 0, stream, a);
    } else if (vx && vw) {
        SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, true, true, false, 2>), grid, block, 0, stream, a);
    } else if (vx) {
        SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, true, false, false, 2>), grid, block, 0, stream, a);
    } else if (vw) {
        SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, false, true, false, 2>), grid, block, 0, stream, a);
    } else {
        SDHIP_LAUNCH((mul_mat_kernel<TM, TN, GATED, false, false, false, 2>), grid, block, 0, stream, a);
    }
    return hipGetLastError();
}

template <int TM, int TN, bool POINTWISE>
hipError_t launch_conv_t(const ConvArgs &c, int stages, hipStream_t stream) {
    constexpr int BM = 64 * TM;
    constexpr int BN = 64 * TN;
    ConvArgs a = c;
    a.oc_blocks = (c.oc + BM - 1) / BM;
    const int64_t blocks = ((c.P + BN - 1) / BN) * a.oc_blocks;
    const bool vw = c.ldw % 8 == 0 && (reinterpret_cast<uintptr_t>(c.w) % 16) == 0;
    const bool full = POINTWISE && vw && c.K % kBK == 0;
    dim3 grid(static_cast<uint32_t>(blocks)), block(256);
    KernelScope scope(POINTWISE ? "conv_direct_pointwise" : "conv_direct", stream);
    if (c.half16) {
        // The products of 16 bits, in FP16 (half16 1) or bfloat16 (2).
        const auto half = [&](auto form) {
            constexpr int H = decltype(form)::value;
            if (full) {
                SDHIP_LAUNCH((conv_direct_kernel<TM, TN, POINTWISE, true, POINTWISE, 2, false, 1, H>), grid, block,
                             0, stream, a);
            } else if (vw) {
                SDHIP_LAUNCH((conv_direct_kernel<TM, TN, POINTWISE, true, false, 2, false, 1, H>), grid, block, 0,
                             stream, a);
            } else {
                SDHIP_LAUNCH((conv_direct_kernel<TM, TN, POINTWISE, false, false, 2, false, 1, H>), grid, block, 0,
                             stream, a);
            }
        };
        if (c.half16 == 2) {
            half(std::integral_constant<int, 2>{});
        } else {
            half(std::integral_constant<int, 1>{});
        }
        return hipGetLastError();
    }
    if (c.w_scale != nullptr) {
        // Split kernels: whole vectors always (rows 32-aligned, zeros past K).
        if (full) {
            SDHIP_LAUNCH((conv_direct_kernel<TM, TN, POINTWISE, true, POINTWISE, 2, false, 2>), grid, block, 0,
                         stream, a);
        } else {
            SDHIP_LAUNCH((conv_direct_kernel<TM, TN, POINTWISE, true, false, 2, false, 2>), grid, block, 0,
                         stream, a);
        }
        return hipGetLastError();
    }
    if (full && stages == 4) {
        SDHIP_LAUNCH((conv_direct_kernel<TM, TN, POINTWISE, true, POINTWISE, 4>), grid, block, 0, stream, a);
    } else if (full) {
        SDHIP_LAUNCH((conv_direct_kernel<TM, TN, POINTWISE, true, POINTWISE, 2>), grid, block, 0, stream, a);
    } else if (vw && !POINTWISE && c.kh == 3 && c.kw == 3) {
        SDHIP_LAUNCH((conv_direct_kernel<TM, TN, false, true, false, 2, true>), grid, block, 0, stream, a);
    } else if (vw) {
        SDHIP_LAUNCH((conv_direct_kernel<TM, TN, POINTWISE, true, false, 2>), grid, block, 0, stream, a);
    } else {
        SDHIP_LAUNCH((conv_direct_kernel<TM, TN, POINTWISE, false, false, 2>), grid, block, 0, stream, a);
    }
    return hipGetLastError();
}

template <int TM, int TN>
hipError_t launch_split_t(SplitBatchedArgs p, int stages, hipStream_t stream) {
    p.m_blocks = (p.M + 64 * TM - 1) / (64 * TM);
    p.n_blocks = (p.N + 64 * TN - 1) / (64 * TN);
    dim3 grid(static_cast<uint32_t>(p.batches * p.m_blocks * p.n_blocks)), block(256);
    if (p.a32 != nullptr) {
        if (stages == 4) {
            SDHIP_LAUNCH((split_batched_kernel<TM, TN, true, 4, true>), grid, block, 0, stream, p);
        } else {
            SDHIP_LAUNCH((split_batched_kernel<TM, TN, true, 2, true>), grid, block, 0, stream, p);
        }
    } else if (stages == 4) {
        SDHIP_LAUNCH((split_batched_kernel<TM, TN, true, 4>), grid, block, 0, stream, p);
    } else {
        SDHIP_LAUNCH((split_batched_kernel<TM, TN, true, 2>), grid, block, 0, stream, p);
    }
    return hipGetLastError();
}

// Blocks of 64 TM x 64 TN: the largest tiles that still give each CU two
// blocks or more, down to 64 x 64 -- and 64 rows wherever 128 would leave a
// part of the last block idle (OC = 320 fills 64-row blocks, not 128-row
// ones: a sixth of the MFMAs would be on padding).
template <class Launch>
hipError_t pick_tiles(int64_t rows, int64_t cols, int64_t batches, int forced, Launch launch) {
    const auto blocks = [&](int tm, int tn) {
        return batches * ((rows + 64 * tm - 1) / (64 * tm)) * ((cols + 64 * tn - 1) / (64 * tn));
    };
    const bool rows128 = rows % 128 == 0 || rows % 128 > 64;
    if (forced == 22 || (forced == 0 && rows128 && blocks(2, 2) >= 512)) {
        return launch(std::integral_constant<int, 2>(), std::integral_constant<int, 2>());
    }
    if (forced == 21 || (forced == 0 && rows128 && blocks(2, 1) >= 512)) {
        return launch(std::integral_constant<int, 2>(), std::integral_constant<int, 1>());
    }
    return launch(std::integral_constant<int, 1>(), std::integral_constant<int, 1>());
}

}  // namespace

hipError_t launch_mul_mat(const MulMatArgs &p, GemmShape g, hipStream_t stream) {
    return pick_tiles(p.M, p.N, 1, g.tiles, [&](auto tm, auto tn) {
        return launch_mul_mat_t<decltype(tm)::value, decltype(tn)::value, false>(p, g.stages, stream);
    });
}

hipError_t launch_mul_mat_gated(const MulMatArgs &p, GemmShape g, hipStream_t stream) {
    // Blocks of 64 tokens by 64 features and their 64 gates: the UNet's
    // GEGLU products leave fractions of a round with 128 tokens a block
    // (measured: the step 11.56 -> 11.36 ms).
    return launch_mul_mat_t<1, 2, true>(p, g.stages, stream);
}

hipError_t launch_conv_direct(const ConvArgs &c, GemmShape g, hipStream_t stream) {
    const bool pointwise = c.kw == 1 && c.kh == 1 && c.s0 == 1 && c.s1 == 1 && c.p0 == 0 && c.p1 == 0;
    const int stages = g.stages;
    return pick_tiles(c.oc, c.P, 1, g.tiles, [&](auto tm, auto tn) {
        constexpr int TM = decltype(tm)::value, TN = decltype(tn)::value;
        return pointwise ? launch_conv_t<TM, TN, true>(c, stages, stream)
                         : launch_conv_t<TM, TN, false>(c, stages, stream);
    });
}

namespace {

struct MulMatSplitPlan {
    int64_t blocks, splits, split_len;
};

// Splits of K for about 512 blocks where the output has fewer than 256 of
// 64 x 64, each of 8 K-steps or more (measured at 512 x 1280 x 1280, the
// UNet's deepest level: two splits of 20 steps 19.7 us against 17.3 in one
// pass, while four of 10 took the UNet step 11.67 -> 11.61 ms); one where
// that leaves no room.
MulMatSplitPlan mul_mat_split_plan(const MulMatArgs &p) {
    MulMatSplitPlan l{};
    l.blocks = ((p.M + 63) / 64) * ((p.N + 63) / 64);
    const int64_t steps = p.K / kBK;
    int64_t sp = l.blocks < 256 ? (512 + l.blocks - 1) / l.blocks : 1;
    const int64_t most = steps / 8 > 1 ? steps / 8 : 1;
    sp = sp < most ? sp : most;
    l.split_len = (steps + sp - 1) / sp * kBK;
    l.splits = steps > 0 ? (p.K + l.split_len - 1) / l.split_len : 1;
    return l;
}

}  // namespace

bool mul_mat_split_taken(const MulMatArgs &p) {
    if (p.w_scale != nullptr || p.half16) return false;  // split weights and 16-bit products go in one pass
    const bool aligned = p.ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(p.x) % 16) == 0 && p.ldw % 8 == 0 &&
                         (reinterpret_cast<uintptr_t>(p.w) % 16) == 0;
    return aligned && p.K % kBK == 0 && mul_mat_split_plan(p).splits > 1;
}

size_t mul_mat_split_work_size(const MulMatArgs &p) {
    return static_cast<size_t>(mul_mat_split_plan(p).splits * p.M * p.N * 4);
}

bool conv_panels_taken(const ConvArgs &c, bool enabled) {
    const bool pointwise = c.kw == 1 && c.kh == 1 && c.s0 == 1 && c.s1 == 1 && c.p0 == 0 && c.p1 == 0;
    if (!enabled || !pointwise || c.w_scale != nullptr || c.half16) return false;
    // A panel's 64 positions lie in one image, in consecutive memory of x and
    // of the output; every row 16-byte aligned.
    const bool layout = c.plane % kConvPanelPositions == 0 && c.xnb1 == c.iw && c.ynb1 == c.ow &&
                        c.xnb2 % 4 == 0 && c.xnb3 % 4 == 0 && c.ynb2 % 4 == 0 && c.ynb3 % 4 == 0 &&
                        (reinterpret_cast<uintptr_t>(c.x) & 15) == 0 && (reinterpret_cast<uintptr_t>(c.y) & 15) == 0 &&
                        c.ldw % 8 == 0 && (reinterpret_cast<uintptr_t>(c.w) & 15) == 0;
    // Enough panels for one a CU, as MUL_MAT's.
    const int64_t panels = (c.P / kConvPanelPositions) * ((c.oc + kConvPanelChannels - 1) / kConvPanelChannels);
    return layout && c.K % kPanelK == 0 && panels >= 256;
}

hipError_t launch_conv_panels(const ConvArgs &c, hipStream_t stream) {
    ConvArgs a = c;
    a.oc_blocks = (c.oc + kConvPanelChannels - 1) / kConvPanelChannels;
    const int64_t blocks = (c.P / kConvPanelPositions) * a.oc_blocks;
    KernelScope scope("conv_direct_pointwise", stream);
    SDHIP_LAUNCH(conv_panel_kernel<kConvPanelStages>, dim3(static_cast<uint32_t>(blocks)), dim3(512), 0, stream, a);
    return hipGetLastError();
}

namespace {

// The index into kPanelShapes of the panels MUL_MAT takes, or -1: the first
// shape whose panels are one a CU or more (fewer take the 64 x 64 core and its
// split along K).  mode: the mul_mat_panels tuning (0 none, 1 every shape, 2
// the first only).
int panel_shape(const MulMatArgs &p, int mode) {
    if (mode == 0 || p.w_scale != nullptr || p.half16) return -1;
    const bool aligned = p.ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(p.x) % 16) == 0 && p.ldw % 8 == 0 &&
                         (reinterpret_cast<uintptr_t>(p.w) % 16) == 0;
    if (!aligned || p.K % kPanelK != 0) return -1;
    const int shapes = mode == 1 ? 2 : 1;
    for (int i = 0; i < shapes; ++i) {
        const int64_t panels = ((p.M + kPanelShapes[i].bm - 1) / kPanelShapes[i].bm) *
                               ((p.N + kPanelShapes[i].bn - 1) / kPanelShapes[i].bn);
        if (panels >= 256) return i;
    }
    return -1;
}

}  // namespace

bool mul_mat_panels_taken(const MulMatArgs &p, int mode) { return panel_shape(p, mode) >= 0; }

namespace {

// Whether the panels' fast epilogue takes this output and chain: N whole
// panels, the output's rows and each operand either contiguous along the
// features with rows 16-byte aligned, or one number a token.
bool panel_chain_fast(const MulMatArgs &p, int bn) {
    const auto aligned = [](const void *q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    if (p.N % bn != 0 || p.ldy % 4 != 0 || !aligned(p.y)) return false;
    for (int s = 0; s < p.chain.count; ++s) {
        const DevStep &st = p.chain.steps[s];
        if (st.kind == kSilu || st.nb[0] == 0) continue;
        const bool rows16 = st.flat123 ? st.nb[1] % 4 == 0 : st.nb[1] % 4 == 0 && st.nb[2] % 4 == 0 && st.nb[3] % 4 == 0;
        if (st.nb[0] != 1 || !rows16 || !aligned(st.operand)) return false;
    }
    return true;
}

}  // namespace

namespace {

template <int BM, int BN>
hipError_t launch_panels(const MulMatArgs &p, hipStream_t stream) {
    MulMatArgs a = p;
    a.col_blocks = (p.N + BN - 1) / BN;
    const dim3 grid(static_cast<uint32_t>(((p.M + BM - 1) / BM) * a.col_blocks));
    KernelScope scope("mul_mat", stream);
    if (panel_chain_fast(a, BN)) {
        SDHIP_LAUNCH((mul_mat_panel_kernel<false, BM, BN>), grid, dim3(256), 0, stream, a, nullptr, 0);
    } else {
        SDHIP_LAUNCH((mul_mat_panel_kernel<true, BM, BN>), grid, dim3(256), 0, stream, a, nullptr, 0);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_mul_mat_panels(const MulMatArgs &p, int mode, hipStream_t stream) {
    switch (panel_shape(p, mode)) {
    case 0:
        return launch_panels<64, 160>(p, stream);
    case 1:
        return launch_panels<64, 64>(p, stream);
    default:
        return hipErrorInvalidValue;
    }
}

hipError_t launch_mul_mat_split(const MulMatArgs &p, void *work, GemmShape g, bool panels, hipStream_t stream) {
    const MulMatSplitPlan l = mul_mat_split_plan(p);
    float *part = static_cast<float *>(work);
    MulMatArgs a = p;
    // Panels of 64 x 160 split along K in at most as many splits, where K is
    // whole chunks of the panels' and N takes whole panels, and the splits
    // are 5 chunks or more and the blocks 128 or more: the same partial sums,
    // into the same buffer.  (Measured: 512 x 1280 x 1280 21.1 -> 20.1 us,
    // 512 x 1280 x 5120 37.1 -> 33.7; with splits of 4 chunks, the cross-
    // attention's 154 x 1280 x 768 and 128 x 1280 x 1280, 10.2 -> 12.4 and
    // 11.1 -> 13.4: those keep the 64 x 64 core.)
    const int64_t chunks = p.K / kPanelK;
    const int64_t split_chunks = (chunks + l.splits - 1) / l.splits;
    const int64_t splits = (chunks + split_chunks - 1) / split_chunks;
    const int64_t panel_blocks = ((p.M + 63) / 64) * (p.N / 160) * splits;
    if (panels && p.K % kPanelK == 0 && p.N % 160 == 0 && split_chunks >= 5 && panel_blocks >= 128) {
        a.col_blocks = p.N / 160;
        const int64_t panels = ((p.M + 63) / 64) * a.col_blocks;
        {
            KernelScope scope("mul_mat", stream);
            SDHIP_LAUNCH((mul_mat_panel_kernel<false, 64, 160>), dim3(static_cast<uint32_t>(panels * splits)),
                         dim3(256), 0, stream, a, part, split_chunks);
        }
        KernelScope scope("mul_mat.sum", stream);
        SDHIP_LAUNCH(mul_mat_sum_kernel, dim3(static_cast<uint32_t>((p.M * p.N + 255) / 256)), dim3(256), 0,
                     stream, a, part, splits);
        return hipGetLastError();
    }
    a.col_blocks = (p.N + 63) / 64;
    {
        KernelScope scope("mul_mat", stream);
        const dim3 grid(static_cast<uint32_t>(l.blocks * l.splits));
        if (g.stages == 4) {
            SDHIP_LAUNCH((mul_mat_split_kernel<4>), grid, dim3(256), 0, stream, a, l.split_len, part);
        } else {
            SDHIP_LAUNCH((mul_mat_split_kernel<2>), grid, dim3(256), 0, stream, a, l.split_len, part);
        }
    }
    KernelScope scope("mul_mat.sum", stream);
    SDHIP_LAUNCH(mul_mat_sum_kernel, dim3(static_cast<uint32_t>((p.M * p.N + 255) / 256)), dim3(256), 0, stream,
                 a, part, l.splits);
    return hipGetLastError();
}

namespace {

struct ColumnsPlan {
    int64_t p_blocks, blocks, splits, split_len;
    size_t cols_bytes, total;
};

ColumnsPlan columns_plan(const ConvArgs &c) {
    ColumnsPlan l{};
    l.p_blocks = (c.P + 63) / 64;
    l.blocks = ((c.oc + 63) / 64) * l.p_blocks;
    // Splits for about 512 blocks in all, of four K-steps or more each.
    const int64_t steps = c.K / kBK;
    int64_t sp = (512 + l.blocks - 1) / l.blocks;
    const int64_t most = steps / 4 > 1 ? steps / 4 : 1;
    sp = sp < most ? sp : most;
    l.split_len = (steps + sp - 1) / sp * kBK;
    l.splits = (c.K + l.split_len - 1) / l.split_len;
    l.cols_bytes = static_cast<size_t>((c.P * c.K * 4 + 255) / 256 * 256);
    l.total = l.cols_bytes + static_cast<size_t>(l.splits * c.oc * c.P * 4);
    return l;
}

}  // namespace

bool conv_columns_taken(const ConvArgs &c) {
    const bool pointwise = c.kw == 1 && c.kh == 1 && c.s0 == 1 && c.s1 == 1 && c.p0 == 0 && c.p1 == 0;
    const bool w_aligned = c.w_split || (c.ldw % 8 == 0 && (reinterpret_cast<uintptr_t>(c.w) % 16) == 0);
    // 1x1 kernels too where their direct blocks would leave most CUs idle
    // and K is long (the UNet's 16 x 16 and 8 x 8 levels): the split along K
    // fills the chip, the columns then being x transposed.
    const int64_t direct_blocks = ((c.oc + 63) / 64) * ((c.P + 63) / 64);
    const bool split_pays = direct_blocks < 256 && c.K / kBK >= 16;
    return (!pointwise || split_pays) && c.K % kBK == 0 && w_aligned &&
           c.P * c.K <= (int64_t{1} << 28) && c.P < (int64_t{1} << 31);
}

size_t conv_columns_work_size(const ConvArgs &c) { return columns_plan(c).total; }

hipError_t launch_conv_columns(const ConvArgs &c, void *work, GemmShape g, hipStream_t stream) {
    const ColumnsPlan l = columns_plan(c);
    float *cols = static_cast<float *>(work);
    float *part = reinterpret_cast<float *>(static_cast<char *>(work) + l.cols_bytes);
    {
        KernelScope scope("conv_direct.columns", stream);
        const dim3 grid(static_cast<uint32_t>((c.P * (c.K / 4) + 255) / 256));
        if (c.kh == 3 && c.kw == 3) {
            SDHIP_LAUNCH((columns_kernel<true>), grid, dim3(256), 0, stream, c, cols);
        } else {
            SDHIP_LAUNCH((columns_kernel<false>), grid, dim3(256), 0, stream, c, cols);
        }
    }
    {
        KernelScope scope("conv_direct", stream);
        ConvArgs a = c;
        a.oc_blocks = (c.oc + 63) / 64;
        const dim3 grid(static_cast<uint32_t>(l.blocks * l.splits));
        if (c.w_scale != nullptr) {
            SDHIP_LAUNCH((conv_columns_kernel<2, 2>), grid, dim3(256), 0, stream, a, cols, l.split_len,
                         l.p_blocks, part);
        } else if (c.half16 == 2) {
            SDHIP_LAUNCH((conv_columns_kernel<2, 1, 2>), grid, dim3(256), 0, stream, a, cols, l.split_len,
                         l.p_blocks, part);
        } else if (c.half16) {
            SDHIP_LAUNCH((conv_columns_kernel<2, 1, 1>), grid, dim3(256), 0, stream, a, cols, l.split_len,
                         l.p_blocks, part);
        } else if (g.stages == 4) {
            SDHIP_LAUNCH((conv_columns_kernel<4>), grid, dim3(256), 0, stream, a, cols, l.split_len, l.p_blocks,
                         part);
        } else {
            SDHIP_LAUNCH((conv_columns_kernel<2>), grid, dim3(256), 0, stream, a, cols, l.split_len, l.p_blocks,
                         part);
        }
    }
    KernelScope scope("conv_direct.sum", stream);
    SDHIP_LAUNCH(conv_sum_kernel, dim3(static_cast<uint32_t>((c.oc * c.P + 255) / 256)), dim3(256), 0, stream, c,
                 part, l.splits);
    return hipGetLastError();
}

// ------------------------------------------------------------------ single-precision weights

namespace {

// One block per row: the row's greatest |w|, its exponent, then the row split.
__global__ __launch_bounds__(256) void split_weights_kernel(const float *__restrict__ w, int64_t ld, int64_t k,
                                                            int64_t kw, int64_t rows, _Float16 *__restrict__ hi,
                                                            _Float16 *__restrict__ lo, float *__restrict__ scale) {
    __shared__ float lds_max[4];
    const int64_t row = blockIdx.x;
    const float *src = w + row * ld;
    float m = 0.0f;
    for (int64_t i = threadIdx.x; i < k; i += 256) m = fmaxf(m, fabsf(src[i]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((threadIdx.x & 63) == 0) lds_max[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(lds_max[0], lds_max[1]), fmaxf(lds_max[2], lds_max[3]));
    int e = 0;
    if (m > 0.0f) frexpf(m, &e);  // m < 2^e
    const int s = m > 0.0f ? 15 - e : 0;  // m 2^s in [2^14, 2^15)
    if (threadIdx.x == 0) scale[row] = ldexpf(1.0f, -s);
    for (int64_t i = threadIdx.x; i < kw; i += 256) {
        _Float16 h, l;
        split_scaled(i < k ? ldexpf(src[i], s) : 0.0f, h, l);
        hi[row * kw + i] = h;
        lo[row * kw + i] = l;
    }
}

}  // namespace

size_t split_weights_bytes(int64_t rows, int64_t k) {
    const size_t planes = static_cast<size_t>(2 * rows * split_weights_ld(k) * 2 + 255) / 256 * 256;
    return planes + static_cast<size_t>(rows * 4 + 255) / 256 * 256;
}

hipError_t launch_split_weights(const float *w, int64_t ld, int64_t rows, int64_t k, void *out, hipStream_t stream) {
    const int64_t kw = split_weights_ld(k);
    _Float16 *hi = static_cast<_Float16 *>(out);
    KernelScope scope("split_weights", stream);
    SDHIP_LAUNCH(split_weights_kernel, dim3(static_cast<uint32_t>(rows)), dim3(256), 0, stream, w, ld, k, kw,
                 rows, hi, hi + rows * kw, const_cast<float *>(split_weights_scale(out, rows, k)));
    return hipGetLastError();
}

hipError_t launch_split_batched(const SplitBatchedArgs &p, GemmShape g, hipStream_t stream) {
    // The operands' layout is the caller's own: K padded to whole steps, every
    // row 16-byte aligned.
    const bool a_aligned = p.a32 != nullptr ? (reinterpret_cast<uintptr_t>(p.a32) % 16) == 0 &&
                                                  (reinterpret_cast<uintptr_t>(p.a_scale) % 16) == 0
                                            : (reinterpret_cast<uintptr_t>(p.a) % 16) == 0 && p.a_plane % 8 == 0;
    const bool aligned = a_aligned && (reinterpret_cast<uintptr_t>(p.b) % 16) == 0 && p.a_batch % 8 == 0 &&
                         p.b_batch % 8 == 0 && p.b_plane % 8 == 0;
    if (p.K % kBK != 0 || !aligned) return hipErrorInvalidValue;
    // Both operands split, two planes each: 80 KB of LDS at 128 x 128.
    return pick_tiles(p.M, p.N, p.batches, g.tiles, [&](auto tm, auto tn) {
        return launch_split_t<decltype(tm)::value, decltype(tn)::value>(p, g.stages, stream);
    });
}

}  // namespace sdhip
