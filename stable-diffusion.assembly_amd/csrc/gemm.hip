// The products of FP16 weights by single-precision activations on gfx950's
// FP16 MFMA (v_mfma_f32_32x32x16_f16): MUL_MAT (mul_mat.cc), MUL_MAT with the
// gated GELU after it (mul_mat.cc:889-1058) and the direct convolution
// (conv2d.cc), each with its chain applied while the output tile is in
// registers.
//
// Precision.  The weights are FP16 and so exact as FP16 MFMA operands; each
// activation x is split into two FP16 parts (device.h, split2), and every
// product is taken as w*hi + w*lo, two MFMAs into the same single-precision
// accumulator: 22 bits of x, as the reference's AMX-FP16 form takes it
// (x86_64/amx_fp16.S: the weights exact, x in two FP16 parts), where ggml
// rounds x to FP16 (11 bits).  Measured by the reference's metric, |error| /
// sum |products| against float64, the result is within a few 1e-7.
//
// Shape.  A workgroup of 4 waves computes a block of BM x BN of C = A B^T,
// A and B both K-contiguous rows, in steps of BK = 32 of K: the rows of both
// operands go from global memory into registers, are split (the single-
// precision one) and written to LDS as FP16, double-buffered, and each wave
// computes its TM x TN tiles of 32 x 32 from LDS, 2 K-steps of 16 per BK.
//   MUL_MAT:     A = x (tokens, split), B = W (features):  C[token][feature]
//   convolution: A = W (output channels), B = the image's columns (split),
//                C[channel][position]
// so that the output's contiguous dimension is always C's column, lane % 32
// of the MFMA's result, and a wave's stores are 128-byte rows.

#include "device.h"
#include "kernels.h"
#include "profile.h"

namespace sdhip {

namespace {

constexpr int kBK = 32;
constexpr int kLdk = kBK + 8;  // halves per LDS row: 80 bytes, 16-byte aligned, skewed across banks

// ------------------------------------------------------------------ MFMA core

// acc[i][j] += A rows (32 i ..) x B cols (32 j ..) over one BK step held in
// LDS.  `a_hi/a_lo` and `b_hi/b_lo`: when an operand is not split its lo
// plane is null and one MFMA is made per tile and K-step instead of two.
template <int TM, int TN, bool SPLIT_A>
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
            if (SPLIT_A) {
                al[i] = *reinterpret_cast<const half8 *>(a_lo + (32 * i + r) * kLdk + ks + kh);
            }
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            b[j] = *reinterpret_cast<const half8 *>(b_hi + (32 * j + r) * kLdk + ks + kh);
            if (!SPLIT_A) {
                bl[j] = *reinterpret_cast<const half8 *>(b_lo + (32 * j + r) * kLdk + ks + kh);
            }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
                if (SPLIT_A) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], b[j], acc[i][j], 0, 0, 0);
                } else {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bl[j], acc[i][j], 0, 0, 0);
                }
            }
        }
    }
}

// Row of the MFMA result held in register e (of 16) of a lane, within a 32 x 32
// tile: the column is lane % 32.
__device__ __forceinline__ int acc_row(int e, int lane) { return 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3); }

// ------------------------------------------------------------------ loaders

// BR rows x BK of K-contiguous single-precision rows (row stride ld elements),
// split into hi and lo planes of LDS.  Rows at or past `rows`, and k at or
// past K, are zeros.  VEC: every row start and ld are multiples of 4 floats.
template <int BR, bool VEC>
struct F32RowsTile {
    static constexpr int kQuads = BR * kBK / 4 / 256;  // float4 per thread
    float4 v[kQuads];

    __device__ void load(const float *base, int64_t ld, int64_t row0, int64_t rows, int64_t k0, int64_t K, int tid) {
#pragma unroll
        for (int i = 0; i < kQuads; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / (kBK / 4);
            const int kq = (idx % (kBK / 4)) * 4;
            const int64_t row = row0 + r;
            const int64_t k = k0 + kq;
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row < rows) {
                const float *p = base + row * ld + k;
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
            _Float16 a, b;
            split2(v[i].x, a, b); h[0] = a; l[0] = b;
            split2(v[i].y, a, b); h[1] = a; l[1] = b;
            split2(v[i].z, a, b); h[2] = a; l[2] = b;
            split2(v[i].w, a, b); h[3] = a; l[3] = b;
            *reinterpret_cast<half4 *>(hi + r * kLdk + kq) = h;
            *reinterpret_cast<half4 *>(lo + r * kLdk + kq) = l;
        }
    }
};

// BR rows x BK of K-contiguous FP16 (or single-precision, rounded... no:
// single-precision weights are split like activations, see F32RowsTile) rows
// into one LDS plane.  `row_of(r)` gives the global row of LDS row r, or -1.
template <int BR, bool VEC>
struct F16RowsTile {
    static constexpr int kOcts = BR * kBK / 8 / 256;  // 8 halves per load
    static_assert(kOcts >= 1, "tile too small for 256 threads");
    half8 v[kOcts];

    template <class RowOf>
    __device__ void load(const _Float16 *base, int64_t ld, RowOf row_of, int64_t k0, int64_t K, int tid) {
#pragma unroll
        for (int i = 0; i < kOcts; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / (kBK / 8);
            const int kq = (idx % (kBK / 8)) * 8;
            const int64_t row = row_of(r);
            const int64_t k = k0 + kq;
            half8 x = {};
            if (row >= 0) {
                const _Float16 *p = base + row * ld + k;
                if (VEC && k + 8 <= K) {
                    x = *reinterpret_cast<const half8 *>(p);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        if (k + e < K) x[e] = p[e];
                    }
                }
            }
            v[i] = x;
        }
    }

    __device__ void store(_Float16 *dst, int tid) const {
#pragma unroll
        for (int i = 0; i < kOcts; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / (kBK / 8);
            const int kq = (idx % (kBK / 8)) * 8;
            *reinterpret_cast<half8 *>(dst + r * kLdk + kq) = v[i];
        }
    }
};

// ------------------------------------------------------------------ MUL_MAT

// C[m][n] = sum_k x[m][k] W[n][k] for rows m of x (single precision, split)
// and rows n of W (FP16), the chain applied, into y[m * ldy + n].  With GATED,
// the block's 128 rows of W are 64 features of the first half and the same 64
// of the second (the gate), each wave's two column tiles a pair, and the
// block writes out[m * ldo + j] = P[m][j] GELU(P[m][half + j]).
template <int TM, int TN, bool GATED, bool VECX, bool VECW>
__global__ __launch_bounds__(256) void mul_mat_kernel(MulMatArgs p) {
    constexpr int BM = 64 * TM;
    constexpr int BN = 64 * TN;
    static_assert(!GATED || TN == 2, "the gated form pairs two column tiles");
    __shared__ __attribute__((aligned(16))) _Float16 lds[2][(2 * BM + BN) * kLdk];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave >> 1;  // wave row (0, 1)
    const int wc = wave & 1;   // wave column

    const uint32_t nblocks = gridDim.x;
    const uint32_t b = xcd_swizzle(blockIdx.x, nblocks);
    const int64_t mb = b / p.col_blocks;
    const int64_t nb = b % p.col_blocks;
    const int64_t m0 = mb * BM;
    const int64_t n0 = nb * (GATED ? BN / 2 : BN);

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

    F32RowsTile<BM, VECX> xa;
    F16RowsTile<BN, VECW> wb;
    const int64_t steps = (p.K + kBK - 1) / kBK;
    xa.load(p.x, p.ldx, m0, p.M, 0, p.K, tid);
    wb.load(p.w, p.ldw, w_row, 0, p.K, tid);
    xa.store(lds[0], lds[0] + BM * kLdk, tid);
    wb.store(lds[0] + 2 * BM * kLdk, tid);
    __syncthreads();
    for (int64_t s = 0; s < steps; ++s) {
        const int cur = s & 1;
        if (s + 1 < steps) {
            xa.load(p.x, p.ldx, m0, p.M, (s + 1) * kBK, p.K, tid);
            wb.load(p.w, p.ldw, w_row, (s + 1) * kBK, p.K, tid);
        }
        const _Float16 *base = lds[cur];
        mfma_step<TM, TN, true>(acc, base + (wr * 32 * TM) * kLdk, base + BM * kLdk + (wr * 32 * TM) * kLdk,
                                base + 2 * BM * kLdk + (wc * 32 * TN) * kLdk, nullptr, lane);
        if (s + 1 < steps) {
            xa.store(lds[cur ^ 1], lds[cur ^ 1] + BM * kLdk, tid);
            wb.store(lds[cur ^ 1] + 2 * BM * kLdk, tid);
        }
        __syncthreads();
    }

    // The epilogue: rows m of the tile, column (feature) lane % 32; a tile's
    // 16 values of the lane at a time, their loads before their stores.
    const int col = lane & 31;
    const uint32_t ne1 = static_cast<uint32_t>(p.ne1), ne2 = static_cast<uint32_t>(p.ne2);
    const auto row_off = [&](const DevStep &st, int64_t m) -> int64_t {
        if (st.flat123) return m * st.nb[1];
        uint32_t i1, i2, i3;
        split_index(static_cast<uint32_t>(m), ne1, ne2, i1, i2, i3);
        return i1 * st.nb[1] + i2 * st.nb[2] + i3 * st.nb[3];
    };
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int64_t mbase = m0 + wr * 32 * TM + 32 * i;
        // Rows past M read the last row and are not stored.
        const auto row = [&](int e) -> int64_t {
            const int64_t m = mbase + acc_row(e, lane);
            return m < p.M ? m : p.M - 1;
        };
        if (GATED) {
            const int64_t f = n0 + 32 * wc + col;
            const int64_t fc = f < p.half ? f : p.half - 1;
            float xv[16], gv[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                xv[e] = acc[i][0][e] * kSplitUp;
                gv[e] = acc[i][1][e] * kSplitUp;
            }
            apply_chain_block(p.chain, xv, [&](int s, int e) {
                return fc * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e));
            });
            apply_chain_block(p.chain, gv, [&](int s, int e) {
                return (p.half + fc) * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e));
            });
            if (f >= p.half) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t m = mbase + acc_row(e, lane);
                if (m < p.M) p.y[m * p.ldy + f] = xv[e] * gelu(gv[e]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int64_t n = n0 + wc * 32 * TN + 32 * j + col;
                const int64_t nc = n < p.N ? n : p.N - 1;
                float v[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) v[e] = acc[i][j][e] * kSplitUp;
                if (p.from_redirect) {
                    float r[16];
#pragma unroll
                    for (int e = 0; e < 16; ++e) r[e] = p.y[row(e) * p.ldy + nc];
#pragma unroll
                    for (int e = 0; e < 16; ++e) v[e] = __fadd_rn(r[e], v[e]);
                }
                apply_chain_block(p.chain, v, [&](int s, int e) {
                    return nc * p.chain.steps[s].nb[0] + row_off(p.chain.steps[s], row(e));
                });
                if (n >= p.N) continue;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int64_t m = mbase + acc_row(e, lane);
                    if (m < p.M) p.y[m * p.ldy + n] = v[e];
                }
            }
        }
    }
}

// ------------------------------------------------------------------ direct convolution

// The columns of the image for BN positions p (of all images, n * OH * OW +
// oy * OW + ox) by BK of K = (ic, kh, kw), read from the image where im2col
// would have put them, split, into LDS as [position][k].  A thread takes one
// position and 4 consecutive k: consecutive threads read consecutive
// positions, which are consecutive in a row of the image at stride 1.
template <int BN, bool POINTWISE>
struct ColumnsTile {
    static constexpr int kLoads = BN * kBK / 4 / 256;
    float v[kLoads][4];
    // Per load slot, fixed over K: the image's first element (or -1 past the
    // last position) and the position's first input row and column.
    int64_t base[kLoads];
    int32_t iy0[kLoads], ix0[kLoads];

    __device__ void init(const ConvArgs &c, int64_t p0, int tid) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int idx = tid + 256 * i;
            const int64_t pos = p0 + idx % BN;
            base[i] = -1;
            if (pos >= c.P) continue;
            uint32_t ox, oy, n;
            split_index(static_cast<uint32_t>(pos), static_cast<uint32_t>(c.ow), static_cast<uint32_t>(c.oh), ox, oy,
                        n);
            base[i] = static_cast<int64_t>(n) * c.xnb3;
            if (POINTWISE) {
                base[i] += static_cast<int64_t>(oy) * c.xnb1 + ox;
            } else {
                iy0[i] = static_cast<int32_t>(oy) * c.s1 - c.p1;
                ix0[i] = static_cast<int32_t>(ox) * c.s0 - c.p0;
            }
        }
    }

    __device__ void load(const ConvArgs &c, int64_t k0, int tid) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int idx = tid + 256 * i;
            const int kq = (idx / BN) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[i][e] = 0.0f;
            if (base[i] < 0) continue;
            const float *img = c.x + base[i];
            if (POINTWISE) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int64_t k = k0 + kq + e;
                    if (k < c.K) v[i][e] = img[k * c.xnb2];
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t k = static_cast<uint32_t>(k0 + kq + e);
                    if (k >= c.K) continue;
                    const uint32_t ic = k / static_cast<uint32_t>(c.taps);
                    const uint32_t t = k - ic * static_cast<uint32_t>(c.taps);
                    const uint32_t kh = t / static_cast<uint32_t>(c.kw);
                    const uint32_t kw = t - kh * static_cast<uint32_t>(c.kw);
                    const int32_t iy = iy0[i] + static_cast<int32_t>(kh) * c.d1;
                    const int32_t ix = ix0[i] + static_cast<int32_t>(kw) * c.d0;
                    if (iy >= 0 && iy < c.ih && ix >= 0 && ix < c.iw) {
                        v[i][e] = img[static_cast<int64_t>(ic) * c.xnb2 + static_cast<int64_t>(iy) * c.xnb1 + ix];
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
                split2(v[i][e], a, b);
                h[e] = a;
                l[e] = b;
            }
            *reinterpret_cast<half4 *>(hi + pl * kLdk + kq) = h;
            *reinterpret_cast<half4 *>(lo + pl * kLdk + kq) = l;
        }
    }
};

// y[n][oc][pos] = sum_k W[oc][k] columns[k][pos], the chain applied; W rows
// K-contiguous FP16 (the kernel as ggml holds it, [OC][IC][KH][KW]).
template <int TM, int TN, bool POINTWISE, bool VECW>
__global__ __launch_bounds__(256) void conv_direct_kernel(ConvArgs c) {
    constexpr int BM = 64 * TM;  // output channels
    constexpr int BN = 64 * TN;  // positions
    __shared__ __attribute__((aligned(16))) _Float16 lds[2][(BM + 2 * BN) * kLdk];

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

    F16RowsTile<BM, VECW> wa;
    ColumnsTile<BN, POINTWISE> xb;
    const int64_t steps = (c.K + kBK - 1) / kBK;
    xb.init(c, p0, tid);
    wa.load(c.w, c.K, w_row, 0, c.K, tid);
    xb.load(c, 0, tid);
    wa.store(lds[0], tid);
    xb.store(lds[0] + BM * kLdk, lds[0] + (BM + BN) * kLdk, tid);
    __syncthreads();
    for (int64_t s = 0; s < steps; ++s) {
        const int cur = s & 1;
        if (s + 1 < steps) {
            wa.load(c.w, c.K, w_row, (s + 1) * kBK, c.K, tid);
            xb.load(c, (s + 1) * kBK, tid);
        }
        const _Float16 *base = lds[cur];
        mfma_step<TM, TN, false>(acc, base + (wr * 32 * TM) * kLdk, nullptr, base + (BM + wc * 32 * TN) * kLdk,
                                 base + (BM + BN + wc * 32 * TN) * kLdk, lane);
        if (s + 1 < steps) {
            wa.store(lds[cur ^ 1], tid);
            xb.store(lds[cur ^ 1] + BM * kLdk, lds[cur ^ 1] + (BM + BN) * kLdk, tid);
        }
        __syncthreads();
    }

    const int col = lane & 31;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int64_t pos = p0 + wc * 32 * TN + 32 * j + col;
        if (pos >= c.P) continue;
        uint32_t ox, oy, n;
        split_index(static_cast<uint32_t>(pos), static_cast<uint32_t>(c.ow), static_cast<uint32_t>(c.oh), ox, oy, n);
        const int64_t at = static_cast<int64_t>(n) * c.ynb3 + static_cast<int64_t>(oy) * c.ynb1 + ox;
        const int64_t in_image = static_cast<int64_t>(oy) * c.ow + ox;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int64_t obase = oc0 + wr * 32 * TM + 32 * i;
            // Channels past OC read the last and are not stored.
            const auto chan = [&](int e) -> int64_t {
                const int64_t oc = obase + acc_row(e, lane);
                return oc < c.oc ? oc : c.oc - 1;
            };
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) v[e] = acc[i][j][e] * kSplitUp;
            if (c.from_redirect) {
                float r[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) r[e] = c.y[at + chan(e) * c.ynb2];
#pragma unroll
                for (int e = 0; e < 16; ++e) v[e] = __fadd_rn(r[e], v[e]);
            }
            apply_chain_block(c.chain, v, [&](int s, int e) {
                const DevStep &st = c.chain.steps[s];
                const int64_t xy = st.flat01 ? in_image * st.nb[0]
                                             : static_cast<int64_t>(ox) * st.nb[0] + static_cast<int64_t>(oy) * st.nb[1];
                return xy + chan(e) * st.nb[2] + static_cast<int64_t>(n) * st.nb[3];
            });
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t oc = obase + acc_row(e, lane);
                if (oc < c.oc) c.y[at + oc * c.ynb2] = v[e];
            }
        }
    }
}

template <int TM, int TN, bool GATED>
hipError_t launch_mul_mat_t(const MulMatArgs &p, hipStream_t stream) {
    constexpr int BM = 64 * TM;
    constexpr int BN = 64 * TN;
    MulMatArgs a = p;
    const int64_t cols = GATED ? p.half : p.N;
    a.col_blocks = (cols + (GATED ? BN / 2 : BN) - 1) / (GATED ? BN / 2 : BN);
    const int64_t blocks = ((p.M + BM - 1) / BM) * a.col_blocks;
    const bool vx = p.ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(p.x) % 16) == 0;
    const bool vw = p.ldw % 8 == 0 && (reinterpret_cast<uintptr_t>(p.w) % 16) == 0;
    dim3 grid(static_cast<uint32_t>(blocks)), block(256);
    KernelScope scope(GATED ? "mul_mat_gated" : "mul_mat", stream);
    if (vx && vw) {
        hipLaunchKernelGGL((mul_mat_kernel<TM, TN, GATED, true, true>), grid, block, 0, stream, a);
    } else if (vx) {
        hipLaunchKernelGGL((mul_mat_kernel<TM, TN, GATED, true, false>), grid, block, 0, stream, a);
    } else if (vw) {
        hipLaunchKernelGGL((mul_mat_kernel<TM, TN, GATED, false, true>), grid, block, 0, stream, a);
    } else {
        hipLaunchKernelGGL((mul_mat_kernel<TM, TN, GATED, false, false>), grid, block, 0, stream, a);
    }
    return hipGetLastError();
}

template <int TM, int TN, bool POINTWISE>
hipError_t launch_conv_t(const ConvArgs &c, hipStream_t stream) {
    constexpr int BM = 64 * TM;
    constexpr int BN = 64 * TN;
    ConvArgs a = c;
    a.oc_blocks = (c.oc + BM - 1) / BM;
    const int64_t blocks = ((c.P + BN - 1) / BN) * a.oc_blocks;
    const bool vw = c.K % 8 == 0 && (reinterpret_cast<uintptr_t>(c.w) % 16) == 0;
    dim3 grid(static_cast<uint32_t>(blocks)), block(256);
    KernelScope scope(POINTWISE ? "conv_direct_pointwise" : "conv_direct", stream);
    if (vw) {
        hipLaunchKernelGGL((conv_direct_kernel<TM, TN, POINTWISE, true>), grid, block, 0, stream, a);
    } else {
        hipLaunchKernelGGL((conv_direct_kernel<TM, TN, POINTWISE, false>), grid, block, 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_mul_mat(const MulMatArgs &p, hipStream_t stream) {
    // Blocks of 128 rows; of 128 features where that still gives every CU a
    // block, of 64 otherwise.
    const int64_t rows = (p.M + 127) / 128;
    if (rows * ((p.N + 127) / 128) >= 256) {
        return launch_mul_mat_t<2, 2, false>(p, stream);
    }
    return launch_mul_mat_t<2, 1, false>(p, stream);
}

hipError_t launch_mul_mat_gated(const MulMatArgs &p, hipStream_t stream) {
    return launch_mul_mat_t<2, 2, true>(p, stream);
}

hipError_t launch_conv_direct(const ConvArgs &c, hipStream_t stream) {
    const bool pointwise = c.kw == 1 && c.kh == 1 && c.s0 == 1 && c.s1 == 1 && c.p0 == 0 && c.p1 == 0;
    const int64_t pblocks = (c.P + 127) / 128;
    const bool wide = pblocks * ((c.oc + 127) / 128) >= 256;
    if (pointwise) {
        return wide ? launch_conv_t<2, 2, true>(c, stream) : launch_conv_t<1, 2, true>(c, stream);
    }
    return wide ? launch_conv_t<2, 2, false>(c, stream) : launch_conv_t<1, 2, false>(c, stream);
}

}  // namespace sdhip
