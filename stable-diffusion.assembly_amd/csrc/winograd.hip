// Winograd's minimal filtering F(m x m, 3x3) (Lavin and Gray, 2016), as the
// reference computes 3x3 convolutions at stride 1 (winograd.cc):
//
//     Y = A^T [ sum over ic of (G g G^T) (.) (B^T d B) ] A
//
// F(2x2, 3x3) with the matrices of winograd.cc:19-22 and F(4x4, 3x3) with the
// points 0, 1, -1, 2, -1/2, infinity of winograd.cc:1146-1183, 1259-1264.
//
// On the device, in five launches:
//   0. the scales, exact powers of two: each input channel's e_c, its
//      greatest |x| times the input transform's gain (49 for F(4x4), 4 for
//      F(2x2)) below 2^(17 + e_c); each output channel's a_o, its greatest
//      FP16 weight times the weight transform's gain ((28/15)^2, 1.5^2)
//      below 2^(17 - a_o);
//   1. the weights at every call, U[xi][oc][ic] = (G g G^T)[xi] * 2^(a_o +
//      e_c - E), E the greatest e_c, as two FP16 parts (device.h, split2), hi
//      and lo, each a plane of its own, [xi][part][kp / 32][oc][32], IC
//      padded with zeros to kp, a multiple of 32; or, where the device store keeps them
//      (as the reference's store keeps its transformed weights when its
//      budget allows, winograd.cc:2147-2149, store.h:26-34), U * 2^a_o in
//      single precision, [xi][oc][kp], with a_o, made by the first call;
//   2. the inputs, V[xi][tile][ic] = (B^T d B)[xi] * 2^-e_c, split into two
//      FP16 parts, [xi][part][kp / 32][tile][32]; with kept weights its first
//      block also finds E, each channel's factor 2^(e_c - E) and each
//      output's shift E - a_o (without, 1. and 2. are one launch);
//   3. the alpha^2 products M[xi] = U[xi] V[xi]^T: kept U (its column c times
//      2^(e_c - E)) split into two FP16 parts on its way into LDS, three
//      MFMAs a product (gemm.hip), so that the sums are those of 22-bit
//      operands where FP16 would hold 11 -- the scales keep every part inside
//      FP16's range: |U| 2^(a_o + e_c - E) and |V| 2^-e_c below 2^17;
//   4. the outputs, A^T M A * 2^(E - a_o), with the sum begun from the
//      residual when the chain says so and the chain after, one thread per
//      (oc, tile).
// The scales cancel: sum_c (U 2^(a + e_c - E)) (V 2^-e_c) = 2^(a - E) sum_c U V.
// The weights and the inputs go out through LDS, so that their stores are
// whole rows of IC rather than scattered halves.
//
// With winograd_fp32=1 the products go to the single-precision MFMA instead
// (v_mfma_f32_16x16x4_f32), unscaled: a sixteenth of the rate, for comparison.

#include "host.h"
#include "kernels.h"
#include "profile.h"
#include "winograd.h"

namespace sdhip {

namespace {

// ------------------------------------------------------------------ matrices

__constant__ float kBT2[4][4] = {{1, 0, -1, 0}, {0, 1, 1, 0}, {0, -1, 1, 0}, {0, 1, 0, -1}};
__constant__ float kG2[4][3] = {{1, 0, 0}, {0.5f, 0.5f, 0.5f}, {0.5f, -0.5f, 0.5f}, {0, 0, 1}};
__constant__ float kAT2[2][4] = {{1, 1, 1, 0}, {0, 1, -1, -1}};

__constant__ float kBT4[6][6] = {{1.0f, 1.5f, -2.0f, -1.5f, 1.0f, 0.0f},  {0.0f, -1.0f, -2.5f, -0.5f, 1.0f, 0.0f},
                                 {0.0f, 1.0f, 0.5f, -2.5f, 1.0f, 0.0f},   {0.0f, -0.5f, -1.0f, 0.5f, 1.0f, 0.0f},
                                 {0.0f, 2.0f, -1.0f, -2.0f, 1.0f, 0.0f},  {0.0f, 1.0f, 1.5f, -2.0f, -1.5f, 1.0f}};
__constant__ float kG4[6][3] = {{1.0f, 0.0f, 0.0f},
                                {-1.0f / 3, -1.0f / 3, -1.0f / 3},
                                {1.0f / 3, -1.0f / 3, 1.0f / 3},
                                {1.0f / 15, 2.0f / 15, 4.0f / 15},
                                {-16.0f / 15, 8.0f / 15, -4.0f / 15},
                                {0.0f, 0.0f, 1.0f}};
__constant__ float kAT4[4][6] = {{1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 0.0f},
                                 {0.0f, 1.0f, -1.0f, 2.0f, -0.5f, 0.0f},
                                 {0.0f, 1.0f, 1.0f, 4.0f, 0.25f, 0.0f},
                                 {0.0f, 1.0f, -1.0f, 8.0f, -0.125f, 1.0f}};

template <int M>
struct Mat;
template <>
struct Mat<2> {
    static constexpr int A = 4;
    static constexpr float kGain = 4.0f;       // the largest row sum of |B^T|, squared
    static constexpr float kWeightGain = 2.25f;  // the largest row sum of |G|, squared
    __device__ static float bt(int i, int j) { return kBT2[i][j]; }
    __device__ static float g(int i, int j) { return kG2[i][j]; }
    __device__ static float at(int i, int j) { return kAT2[i][j]; }
};
template <>
struct Mat<4> {
    static constexpr int A = 6;
    static constexpr float kGain = 49.0f;
    static constexpr float kWeightGain = 3.4844445f;  // (28 / 15)^2, rounded up
    __device__ static float bt(int i, int j) { return kBT4[i][j]; }
    __device__ static float g(int i, int j) { return kG4[i][j]; }
    __device__ static float at(int i, int j) { return kAT4[i][j]; }
};

// A row of a tile's outputs as one vector.
template <int M>
struct RowOf;
template <>
struct RowOf<2> {
    using type = float __attribute__((ext_vector_type(2)));
};
template <>
struct RowOf<4> {
    using type = float __attribute__((ext_vector_type(4)));
};

// The exponent k of v = m 2^k, m in [0.5, 1): v < 2^k.
__device__ __forceinline__ int exponent_above(float v) {
    int k = 0;
    frexpf(v, &k);
    return k;
}

constexpr int kTop = 17;  // scaled operands below 2^17: below 2^13 once split2 takes 2^-4
constexpr int kZeroChannel = -126;  // the exponent of an input channel of zeros

__device__ __forceinline__ float block_max(float v, float *scratch) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(scratch[0], scratch[1]), fmaxf(scratch[2], scratch[3]));
}

// ------------------------------------------------------------------ 0. scales

__device__ __forceinline__ float abs_max4(float4v v) {
    return fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
}

// One workgroup per channel: blocks [0, IC) input channel c's greatest |x|
// over every image, eight independent float4 loads in flight per thread
// (across the images) where the rows are contiguous, and its exponent e[c]
// (zero channels: the least, so that they scale to zero); blocks
// [IC, IC + OC) output channel o's greatest FP16 weight, four loads of eight
// in flight per thread, and a[o].
template <int M>
__global__ __launch_bounds__(256) void scales_kernel(WinogradArgs a, int32_t *__restrict__ e,
                                                     int32_t *__restrict__ amax) {
    __shared__ float scratch[4];
    const int64_t w = blockIdx.x;
    const int tid = threadIdx.x;
    float m0 = 0.0f, m1 = 0.0f, m2 = 0.0f, m3 = 0.0f;
    if (w < a.ic) {
        const int64_t plane = a.ih * a.iw;
        const float *p0 = a.x + w * a.xnb2;
        const bool vec = a.xnb1 == a.iw && plane % 4 == 0 && a.xnb3 % 4 == 0 &&
                         (reinterpret_cast<uintptr_t>(p0) & 15) == 0 && a.n * (plane / 4) < (int64_t{1} << 32);
        if (vec) {
            // The channel's planes as one run of n * plane / 4 quads, the
            // image of quad i being i / quads.
            const uint32_t quads = static_cast<uint32_t>(plane / 4);
            const uint32_t total = static_cast<uint32_t>(a.n) * quads;
            for (uint32_t base = tid; base < total; base += 256 * 8) {
                float4v v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const uint32_t i = base + 256 * u;
                    v[u] = float4v{};
                    if (i < total) {
                        const uint32_t n = i / quads;
                        v[u] = reinterpret_cast<const float4v *>(p0 + n * a.xnb3)[i - n * quads];
                    }
                }
#pragma unroll
                for (int u = 0; u < 8; u += 4) {
                    m0 = fmaxf(m0, abs_max4(v[u]));
                    m1 = fmaxf(m1, abs_max4(v[u + 1]));
                    m2 = fmaxf(m2, abs_max4(v[u + 2]));
                    m3 = fmaxf(m3, abs_max4(v[u + 3]));
                }
            }
        } else {
            for (int64_t n = 0; n < a.n; ++n) {
                const float *p = p0 + n * a.xnb3;
                for (int64_t i = tid; i < plane; i += 256) {
                    const int64_t y = i / a.iw;
                    m0 = fmaxf(m0, fabsf(p[y * a.xnb1 + (i - y * a.iw)]));
                }
            }
        }
        const float m = block_max(fmaxf(fmaxf(m0, m1), fmaxf(m2, m3)), scratch);
        if (tid == 0) e[w] = m > 0.0f ? exponent_above(m * Mat<M>::kGain) - kTop : kZeroChannel;
    } else {
        const int64_t o = w - a.ic;
        const int64_t count = a.ic * 9;
        const _Float16 *p = a.w != nullptr ? a.w + o * count : nullptr;
        if (a.w32 != nullptr) {
            // Single-precision kernels.
            const float *q = a.w32 + o * count;
            for (int64_t i = tid; i < count; i += 256) m0 = fmaxf(m0, fabsf(q[i]));
        } else if (count % 8 == 0 && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
            const half8 *q = reinterpret_cast<const half8 *>(p);
            const int64_t octs = count / 8;
            int64_t i = tid;
            for (; i + 768 < octs; i += 1024) {
                const half8 v0 = q[i], v1 = q[i + 256], v2 = q[i + 512], v3 = q[i + 768];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    m0 = fmaxf(m0, fabsf(static_cast<float>(v0[k])));
                    m1 = fmaxf(m1, fabsf(static_cast<float>(v1[k])));
                    m2 = fmaxf(m2, fabsf(static_cast<float>(v2[k])));
                    m3 = fmaxf(m3, fabsf(static_cast<float>(v3[k])));
                }
            }
            for (; i < octs; i += 256) {
                const half8 v = q[i];
#pragma unroll
                for (int k = 0; k < 8; ++k) m0 = fmaxf(m0, fabsf(static_cast<float>(v[k])));
            }
        } else {
            for (int64_t i = tid; i < count; i += 256) m0 = fmaxf(m0, fabsf(static_cast<float>(p[i])));
        }
        const float m = block_max(fmaxf(fmaxf(m0, m1), fmaxf(m2, m3)), scratch);
        if (tid == 0) amax[o] = m > 0.0f ? kTop - exponent_above(m * Mat<M>::kWeightGain) : 0;
    }
}

// ------------------------------------------------------------------ 1. weights

template <class W>
__device__ __forceinline__ void load_g(const W *w, float (&g)[3][3]) {
#pragma unroll
    for (int i = 0; i < 9; ++i) g[i / 3][i % 3] = static_cast<float>(w[i]);
}

// c0 x0 + c1 x1 + c2 x2 with its roundings written out: the first product
// rounded, the other two fused in turn.  Left to the compiler, the sum is
// contracted by where its operands come from (a kernel that converts the FP16
// weights in the same block fuses other pairs than one that converted them
// earlier), and F(4x4)'s G (thirds, fifteenths) rounds differently each way;
// written out, every kernel that transforms weights gets the same bits.
// Where the coefficients are the folded constants of G, a zero one is left
// out (it would add nothing but the sign of a zero).
__device__ __forceinline__ float dot3(float c0, float x0, float c1, float x1, float c2, float x2) {
    float s = 0.0f;
    bool any = false;
    if (c0 != 0.0f) {
        s = c0 * x0;
        any = true;
    }
    if (c1 != 0.0f) {
        s = any ? fmaf(c1, x1, s) : c1 * x1;
        any = true;
    }
    if (c2 != 0.0f) s = any ? fmaf(c2, x2, s) : c2 * x2;
    return s;
}

// sum_i c(i) x(i) over N terms with its roundings written out, as dot3: the
// first term of a nonzero coefficient rounded, the others fused in turn, the
// zero coefficients of the folded tables left out -- the same bits in every
// kernel that transforms the inputs.
template <int N, class C, class X>
__device__ __forceinline__ float dot_n(C c, X x) {
    float s = 0.0f;
    bool any = false;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float ci = c(i);
        if (ci != 0.0f) {
            s = any ? fmaf(ci, x(i), s) : ci * x(i);
            any = true;
        }
    }
    return s;
}

// (G g G^T) of one kernel: G g a column at a time, then (G g) G^T a row at a
// time (winograd.cc:1281-1300).
template <int M>
__device__ __forceinline__ void transform_g(const float (&g)[3][3], float (&u)[Mat<M>::A][Mat<M>::A]) {
    constexpr int A = Mat<M>::A;
    float gg[A][3];
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
            gg[i][j] = dot3(Mat<M>::g(i, 0), g[0][j], Mat<M>::g(i, 1), g[1][j], Mat<M>::g(i, 2), g[2][j]);
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j)
            u[i][j] = dot3(Mat<M>::g(j, 0), gg[i][0], Mat<M>::g(j, 1), gg[i][1], Mat<M>::g(j, 2), gg[i][2]);
}

// A block per 4 output channels by 64 input channels, a thread per kernel:
// E, the greatest e_c (each block reduces e itself), and shift[o] = E - a_o
// for the outputs (blocks of the first channels); U * 2^(a_o + e_c - E) split
// into its two FP16 parts, staged in LDS as [xi][part][o][channel] and
// written out in blocks of 32 channels, u[xi][part][kp / 32][oc][32], zeros
// from IC to kp.
constexpr int kWeightOc = 4, kWeightIc = 64;

// The points of one pass of the transforms' staging in LDS: half of them.
template <int M>
constexpr int kHalfPoints = Mat<M>::A * Mat<M>::A / 2;
static_assert(Mat<2>::A % 2 == 0 && Mat<4>::A % 2 == 0, "the points split into two halves");

// LDS of a block of weights_split: the 4 floats of the reduction, then the
// staged parts of half of the points.
template <int M>
constexpr int kWeightLds = 16 + 2 * kHalfPoints<M> * kWeightOc * kWeightIc * 2;

// Block (bx, by) of weights_split, its LDS at `lds`.
template <int M, class W>
__device__ __forceinline__ void weights_split_block(const W *__restrict__ w, int64_t oc, int64_t ic, int64_t kp,
                                                    const int32_t *__restrict__ e, const int32_t *__restrict__ amax,
                                                    _Float16 *__restrict__ u, int32_t *__restrict__ shift, int64_t bx,
                                                    int64_t by, char *lds) {
    constexpr int A = Mat<M>::A;
    constexpr int H = kHalfPoints<M>;
    float *scratch = reinterpret_cast<float *>(lds);
    auto stage = reinterpret_cast<_Float16(*)[kWeightOc][kWeightIc]>(lds + 16);
    const int tid = threadIdx.x;
    const int64_t o0 = bx * kWeightOc;
    const int64_t c0 = by * kWeightIc;
    const int ol = tid / kWeightIc, cl = tid % kWeightIc;
    const int64_t o = o0 + ol, c = c0 + cl;
    // The thread's kernel and exponents first, so that their loads overlap
    // those of E's reduction.
    const bool live = o < oc && c < ic;
    float g[3][3] = {};
    int ao = 0, ec = 0;
    if (o < oc) ao = amax[o];
    if (live) {
        load_g(w + (o * ic + c) * 9, g);
        ec = e[c];
    }
    int emax = kZeroChannel;
    for (int64_t k = tid; k < ic; k += 256) emax = max(emax, e[k]);
    const int E = static_cast<int>(block_max(static_cast<float>(emax), scratch));
    if (o < oc && by == 0 && cl == 0) shift[o] = E - ao;
    float t[A][A] = {};
    float f = 0.0f;
    if (live) {
        transform_g<M>(g, t);
        f = ldexpf(kSplitDown, ao + ec - E);
    }
    // Half of the points at a time: kRows / 2 x kWeightOc rows of `width`
    // halves (64, or 32 in the last block of channels), 8 at a time.
    const int width = static_cast<int>(kp - c0 < kWeightIc ? kp - c0 : kWeightIc);
    constexpr int kPerRow = kWeightIc / 8;
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1) __syncthreads();  // the first half read out
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const int pt = pass * H + h;
            _Float16 hi, lo;
            split_scaled(t[pt / A][pt % A] * f, hi, lo);
            stage[2 * h][ol][cl] = hi;
            stage[2 * h + 1][ol][cl] = lo;
        }
        __syncthreads();
        for (int q = tid; q < 2 * H * kWeightOc * kPerRow; q += 256) {
            const int row = q / kPerRow;
            const int k = (q % kPerRow) * 8;
            const int r = 2 * H * pass + row / kWeightOc, oo = row % kWeightOc;
            if (k >= width || o0 + oo >= oc) continue;
            const int64_t cc = c0 + k;
            *reinterpret_cast<half8 *>(u + r * oc * kp + (cc >> 5) * oc * 32 + (o0 + oo) * 32 + (cc & 31)) =
                *reinterpret_cast<const half8 *>(&stage[row / kWeightOc][oo][k]);
        }
    }
}

// Unscaled U[xi][oc][ic], one thread per (oc, ic), for the single-precision products.
template <int M, class W>
__global__ __launch_bounds__(256) void weights_kernel(const W *__restrict__ w, float *__restrict__ u, int64_t oc,
                                                      int64_t ic) {
    constexpr int A = Mat<M>::A;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (t >= oc * ic) return;
    float g[3][3], v[A][A];
    load_g(w + t * 9, g);
    transform_g<M>(g, v);
    const int64_t plane = oc * ic;
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j) u[(i * A + j) * plane + t] = v[i][j];
}

// U[xi][oc][kp] * 2^a_o in single precision, zeros from IC to kp, one thread
// per (oc, channel): the transformed weights as the store keeps them, the
// inputs' scales 2^(e_c - E) applied by the products as they read them.
template <int M, class W>
__global__ __launch_bounds__(256) void weights_scaled_kernel(const W *__restrict__ w, int64_t oc, int64_t ic,
                                                             int64_t kp, const int32_t *__restrict__ amax,
                                                             float *__restrict__ u) {
    constexpr int A = Mat<M>::A;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (t >= oc * kp) return;
    const int64_t o = t / kp, c = t - o * kp;
    float v[A][A] = {};
    if (c < ic) {
        float g[3][3];
        load_g(w + (o * ic + c) * 9, g);
        transform_g<M>(g, v);
        const int s = amax[o];
#pragma unroll
        for (int i = 0; i < A; ++i)
#pragma unroll
            for (int j = 0; j < A; ++j) v[i][j] = ldexpf(v[i][j], s);
    }
    const int64_t plane = oc * kp;
#pragma unroll
    for (int i = 0; i < A; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j) u[(i * A + j) * plane + t] = v[i][j];
}

// ------------------------------------------------------------------ 2. inputs

// The alpha x alpha inputs d of a tile, zeros outside the image, one load a
// point.  Every load unconditional, from the nearest point inside the image,
// and the points outside then cleared by masks of all ones or zeros.  The
// masks pass through an empty asm so that the compiler sees no select of a
// load, which it would turn back into a branch around each load.
template <int M>
__device__ __forceinline__ void load_d(const WinogradArgs &a, uint32_t tx, uint32_t ty, uint32_t n, uint32_t c,
                                       float (&d)[Mat<M>::A][Mat<M>::A]) {
    constexpr int A = Mat<M>::A;
    const int64_t y0 = static_cast<int64_t>(ty) * M - a.p1;
    const int64_t x0 = static_cast<int64_t>(tx) * M - a.p0;
    const float *plane = a.x + static_cast<int64_t>(n) * a.xnb3 + static_cast<int64_t>(c) * a.xnb2;
    int64_t xc[A];
    int mask_col[A];
#pragma unroll
    for (int j = 0; j < A; ++j) {
        const int64_t xx = x0 + j;
        mask_col[j] = xx >= 0 && xx < a.iw ? -1 : 0;
        asm("" : "+v"(mask_col[j]));
        xc[j] = xx < 0 ? 0 : (xx < a.iw ? xx : a.iw - 1);
    }
#pragma unroll
    for (int i = 0; i < A; ++i) {
        const int64_t yy = y0 + i;
        int mask_row = yy >= 0 && yy < a.ih ? -1 : 0;
        asm("" : "+v"(mask_row));
        const float *row = plane + (yy < 0 ? 0 : (yy < a.ih ? yy : a.ih - 1)) * a.xnb1;
#pragma unroll
        for (int j = 0; j < A; ++j) {
            d[i][j] = __builtin_bit_cast(float, __builtin_bit_cast(int, row[xc[j]]) & (mask_row & mask_col[j]));
        }
    }
}

// The same for F(4x4) where a.xbytes is set: the image's rows are runs of a
// multiple of 4 floats, 16-byte aligned, the padding on the left is 1 and the
// tiles end inside each row, so that a tile's columns 4 tx - 1 .. 4 tx + 4 are
// one 16-byte load of the middle four and one 4-byte load on each side, all
// at one row offset.  The loads go through a buffer resource over x's
// a.xbytes bytes, whose range check returns zeros: a point outside the image
// (a row above or below it, the column left of the first tile or right of
// the last) is read at an offset past the end instead of being masked.
__device__ __forceinline__ void load_d_quads(const WinogradArgs &a, uint32_t tx, uint32_t ty, uint32_t n, uint32_t c,
                                             float (&d)[6][6]) {
    constexpr uint32_t kPast = 0x80000000u;  // a.xbytes is below 2^31
    const __amdgpu_buffer_rsrc_t x =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(a.x), 0, static_cast<int>(a.xbytes), 0x00020000);
    const uint32_t col = 4 * tx;
    const uint32_t plane = n * static_cast<uint32_t>(a.xnb3) + c * static_cast<uint32_t>(a.xnb2) + col;
    const bool left = col > 0, right = col + 4 < static_cast<uint32_t>(a.iw);
    const int y0 = static_cast<int>(ty) * 4 - a.p1;
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        const int yy = y0 + i;
        const bool inside = yy >= 0 && yy < static_cast<int>(a.ih);
        const uint32_t off = (plane + static_cast<uint32_t>(yy) * static_cast<uint32_t>(a.xnb1)) * 4;
        const uint32_t mid = inside ? off : kPast;
        const float4v q = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(x, mid, 0, 0));
        d[i][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(x, inside && left ? off - 4 : kPast, 0, 0));
        d[i][1] = q[0];
        d[i][2] = q[1];
        d[i][3] = q[2];
        d[i][4] = q[3];
        d[i][5] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(x, inside && right ? off + 16 : kPast, 0, 0));
    }
}

// One row or column of B^T d B: y = B^T t over six points.  F(4x4)'s B^T
// (points 0, 1, -1, 2, -1/2, infinity) by its shared terms, 17 operations
// where the rows' 26 nonzero coefficients would take 26:
//   y0 = (t0 + t4) - 2 t2 + 1.5 (t1 - t3)     y3 = (t4 - t2) - 0.5 (t1 - t3)
//   y1 = (t4 - t1) - 2.5 t2 - 0.5 t3          y4 = (t4 - t2) + 2 (t1 - t3)
//   y2 = (t4 + t1) + 0.5 t2 - 2.5 t3          y5 = (t1 + t5) - 2 t3 + 1.5 (t2 - t4)
__device__ __forceinline__ void bt4(float t0, float t1, float t2, float t3, float t4, float t5, float &y0,
                                    float &y1, float &y2, float &y3, float &y4, float &y5) {
    const float p = t1 - t3, q = t4 - t2;
    y0 = fmaf(1.5f, p, fmaf(-2.0f, t2, t0 + t4));
    y1 = fmaf(-0.5f, t3, fmaf(-2.5f, t2, t4 - t1));
    y2 = fmaf(-2.5f, t3, fmaf(0.5f, t2, t4 + t1));
    y3 = fmaf(-0.5f, p, q);
    y4 = fmaf(2.0f, p, q);
    y5 = fmaf(1.5f, t2 - t4, fmaf(-2.0f, t3, t1 + t5));
}

// (B^T d B) of the alpha x alpha inputs of a tile, zeros outside the image:
// B^T d (a row r of B^T takes its combination of the rows of d), then each of
// those times B.
template <int M>
__device__ __forceinline__ void transform_d(const WinogradArgs &a, uint32_t tile, uint32_t c,
                                            float (&v)[Mat<M>::A][Mat<M>::A]) {
    constexpr int A = Mat<M>::A;
    uint32_t tx, ty, n;
    split_index(tile, static_cast<uint32_t>(a.tw), static_cast<uint32_t>(a.th), tx, ty, n);
    float d[A][A];
    if constexpr (M == 4) {
        if (a.xbytes != 0) {
            load_d_quads(a, tx, ty, n, c, d);
        } else {
            load_d<M>(a, tx, ty, n, c, d);
        }
        float bd[6][6];
#pragma unroll
        for (int j = 0; j < 6; ++j)
            bt4(d[0][j], d[1][j], d[2][j], d[3][j], d[4][j], d[5][j], bd[0][j], bd[1][j], bd[2][j], bd[3][j],
                bd[4][j], bd[5][j]);
#pragma unroll
        for (int r = 0; r < 6; ++r)
            bt4(bd[r][0], bd[r][1], bd[r][2], bd[r][3], bd[r][4], bd[r][5], v[r][0], v[r][1], v[r][2], v[r][3],
                v[r][4], v[r][5]);
    } else {
        load_d<M>(a, tx, ty, n, c, d);
        float bd[A][A];
#pragma unroll
        for (int r = 0; r < A; ++r)
#pragma unroll
            for (int j = 0; j < A; ++j)
                bd[r][j] = dot_n<A>([&](int i) { return Mat<M>::bt(r, i); }, [&](int i) { return d[i][j]; });
#pragma unroll
        for (int r = 0; r < A; ++r)
#pragma unroll
            for (int s = 0; s < A; ++s)
                v[r][s] = dot_n<A>([&](int j) { return Mat<M>::bt(s, j); }, [&](int j) { return bd[r][j]; });
    }
}

// V[xi][tile][ic] * 2^-e_c split into two FP16 parts, in blocks of 32
// channels, v[xi][part][c / 32][tile][c % 32], zeros for the channels from IC
// to kp.  A block takes 8 consecutive tiles by
// 32 channels, one (tile, channel) a thread, consecutive threads consecutive
// tiles (so that the reads of a channel are rows of the image); the results
// are staged in LDS as [xi][part][tile][channel], half of the points at a
// time (so that more blocks fit a CU), and written out as rows of 32
// channels.
constexpr int kInTiles = 8, kInChannels = 32;

// LDS of a block of inputs_split: the staged parts of half of the points,
// [xi][part][tile][channel], rows of a tile 40 halves apart (16-byte aligned).
template <int M>
constexpr int kInputLds = 2 * kHalfPoints<M> * kInTiles * (kInChannels + 8) * 2;

// Block (bx, by) of inputs_split, its LDS at `lds`: V * 2^-e_c split into
// its two FP16 parts (split2, the form the products take; the channel's
// 2^-e_c and the split's 2^-4 one factor), written as
// v[xi][part][c / 32][tile][c % 32].
template <int M>
__device__ __forceinline__ void inputs_split_block(const WinogradArgs &a, int64_t kp, const int32_t *__restrict__ e,
                                                   _Float16 *__restrict__ v, int64_t bx, int64_t by, char *lds) {
    constexpr int A = Mat<M>::A;
    constexpr int H = kHalfPoints<M>;
    auto stage = reinterpret_cast<_Float16(*)[kInTiles][kInChannels + 8]>(lds);
    const int tid = threadIdx.x;
    const int64_t t0 = bx * kInTiles;
    const int64_t c0 = by * kInChannels;
    const int tl = tid % kInTiles, cl = tid / kInTiles;
    const int64_t tile = t0 + tl, c = c0 + cl;
    float x[A][A] = {};
    float f = 0.0f;
    if (c < a.ic && tile < a.tiles) {
        transform_d<M>(a, static_cast<uint32_t>(tile), static_cast<uint32_t>(c), x);
        f = ldexpf(kSplitDown, -e[c]);
    }
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1) __syncthreads();  // the first half read out
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const int pt = pass * H + h;
            _Float16 hi, lo;
            split_scaled(x[pt / A][pt % A] * f, hi, lo);
            stage[2 * h][tl][cl] = hi;
            stage[2 * h + 1][tl][cl] = lo;
        }
        __syncthreads();
        if (a.v_by8) {
            // Runs of 8 channels, [xp][kp / 8][tile][8]: consecutive threads
            // consecutive tiles of one run.
            for (int q = tid; q < 2 * H * kInTiles * (kInChannels / 8); q += 256) {
                const int t = q % kInTiles;
                const int run = (q / kInTiles) % (kInChannels / 8);
                const int xl = q / (kInTiles * (kInChannels / 8));
                if (t0 + t >= a.tiles) continue;
                const int64_t xp = 2 * H * pass + xl;
                *reinterpret_cast<half8 *>(v + ((xp * (kp / 8) + c0 / 8 + run) * a.tiles + t0 + t) * 8) =
                    *reinterpret_cast<const half8 *>(&stage[xl][t][8 * run]);
            }
            continue;
        }
        // 2 H * kInTiles rows of 32 halves, 8 at a time.
        for (int q = tid; q < 2 * H * kInTiles * (kInChannels / 8); q += 256) {
            const int row = q / (kInChannels / 8);
            const int k = (q % (kInChannels / 8)) * 8;
            const int xl = row / kInTiles, t = row % kInTiles;
            if (t0 + t >= a.tiles) continue;
            const int xp = 2 * H * pass + xl;
            *reinterpret_cast<half8 *>(v + xp * a.tiles * kp + c0 * a.tiles + (t0 + t) * kInChannels + k) =
                *reinterpret_cast<const half8 *>(&stage[xl][t][k]);
        }
    }
}

template <int M>
__global__ __launch_bounds__(256) void inputs_split_kernel(WinogradArgs a, int64_t kp, const int32_t *__restrict__ e,
                                                           _Float16 *__restrict__ v, const int32_t *__restrict__ amax,
                                                           float *__restrict__ f, int32_t *__restrict__ shift) {
    __shared__ __attribute__((aligned(16))) char lds[kInputLds<M>];
    if (f != nullptr && blockIdx.x == 0 && blockIdx.y == 0) {
        // With the weights kept: E, the greatest e_c; each channel's scale of
        // the weights 2^(e_c - E) (zero past IC), and each output channel's
        // shift E - a_o.
        float *scratch = reinterpret_cast<float *>(lds);
        int emax = kZeroChannel;
        for (int64_t c = threadIdx.x; c < a.ic; c += 256) emax = max(emax, e[c]);
        const int E = static_cast<int>(block_max(static_cast<float>(emax), scratch));
        for (int64_t c = threadIdx.x; c < kp; c += 256) f[c] = c < a.ic ? ldexpf(1.0f, e[c] - E) : 0.0f;
        for (int64_t o = threadIdx.x; o < a.oc; o += 256) shift[o] = E - amax[o];
        __syncthreads();
    }
    // Neighbouring tiles on one XCD, as in the transforms' launch.
    const uint32_t b = xcd_swizzle(blockIdx.x + blockIdx.y * gridDim.x, gridDim.x * gridDim.y);
    inputs_split_block<M>(a, kp, e, v, b % gridDim.x, b / gridDim.x, lds);
}

// The weights' and the inputs' transforms of a call without kept weights in
// one launch, wblocks of the weights' (wgx of them along OC) and the rest the
// inputs' (igx along the tiles): neither waits for the other, and the
// VALU-heavy weights share the chip with the memory-heavy inputs.
template <int M>
constexpr int kTransformLds = kWeightLds<M> > kInputLds<M> ? kWeightLds<M> : kInputLds<M>;

template <int M>
__global__ __launch_bounds__(256) void transforms_kernel(WinogradArgs a, int64_t kp, const int32_t *__restrict__ e,
                                                         const int32_t *__restrict__ amax, _Float16 *__restrict__ u,
                                                         int32_t *__restrict__ shift, _Float16 *__restrict__ v,
                                                         int64_t wgx, int64_t wblocks, int64_t igx) {
    __shared__ __attribute__((aligned(16))) char lds[kTransformLds<M>];
    // The two kinds alternate while both last, so that every CU gets some of
    // each; the rest of the longer kind follows.  The blocks an XCD takes
    // (every 8th of the launch) are consecutive ones of this order, so that
    // each XCD gets both kinds and the inputs' blocks of one XCD are
    // neighbouring tiles, whose overlapping rows its own L2 then holds.
    const int64_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t iblocks = gridDim.x - wblocks;
    const int64_t both = wblocks < iblocks ? wblocks : iblocks;
    bool weights;
    int64_t q;
    if (b < 2 * both) {
        weights = (b & 1) == 0;
        q = b >> 1;
    } else {
        weights = wblocks > iblocks;
        q = b - both;
    }
    if (weights) {
        if (a.w32 != nullptr) {
            weights_split_block<M>(a.w32, a.oc, a.ic, kp, e, amax, u, shift, q % wgx, q / wgx, lds);
        } else {
            weights_split_block<M>(a.w, a.oc, a.ic, kp, e, amax, u, shift, q % wgx, q / wgx, lds);
        }
    } else {
        inputs_split_block<M>(a, kp, e, v, q % igx, q / igx, lds);
    }
}

// Unscaled V[xi][ic][tile], for the single-precision products: consecutive
// threads consecutive tiles.
template <int M>
__global__ __launch_bounds__(256) void inputs_kernel(WinogradArgs a, float *__restrict__ v) {
    constexpr int A = Mat<M>::A;
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= static_cast<uint32_t>(a.tiles * a.ic)) return;
    const uint32_t c = t / static_cast<uint32_t>(a.tiles);
    const uint32_t tile = t - c * static_cast<uint32_t>(a.tiles);
    float x[A][A];
    transform_d<M>(a, tile, c, x);
    const int64_t plane = a.ic * a.tiles;
#pragma unroll
    for (int r = 0; r < A; ++r)
#pragma unroll
        for (int q = 0; q < A; ++q) v[(r * A + q) * plane + t] = x[r][q];
}

// ------------------------------------------------------------------ 3. single-precision products

// C[b][m][n] = sum_k A[b][m][k] B[b][k][n] for the alpha^2 batches b, A rows
// K-contiguous (U: [oc][ic]), B rows N-contiguous (V: [ic][tile]), on
// v_mfma_f32_16x16x4_f32.  A block of 64 x 128 by 4 waves of 32 x 64 (2 x 4
// tiles of 16 x 16), K in steps of 16 through LDS, double-buffered; LDS holds
// both operands k-major, [k][row] and [k][col], padded so that the four k-rows
// a wave reads at once fall in four distinct sets of banks.
constexpr int kGBM = 64, kGBN = 128, kGBK = 16;
constexpr int kPadA = kGBM + 16, kPadB = kGBN + 16;

__global__ __launch_bounds__(256) void batched_gemm_f32(const float *__restrict__ A, const float *__restrict__ B,
                                                        float *__restrict__ C, int64_t M, int64_t N, int64_t K,
                                                        int64_t m_blocks, int64_t n_blocks) {
    __shared__ float la[2][kGBK * kPadA];
    __shared__ float lb[2][kGBK * kPadB];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave >> 1, wc = wave & 1;

    const int64_t per_batch = m_blocks * n_blocks;
    const int64_t bid = blockIdx.x;
    const int64_t batch = bid / per_batch;
    const int64_t rem = bid - batch * per_batch;
    const int64_t mb = rem / n_blocks;
    const int64_t nb = rem - mb * n_blocks;
    const int64_t m0 = mb * kGBM, n0 = nb * kGBN;
    const float *Ab = A + batch * M * K;
    const float *Bb = B + batch * K * N;
    float *Cb = C + batch * M * N;
    const bool vec_a = (K % 4) == 0;
    const bool vec_b = (N % 4) == 0;

    float4 ra, rb[2];
    const auto load = [&](int64_t k0) {
        {
            const int r = tid / 4, kq = (tid % 4) * 4;
            const int64_t row = m0 + r, k = k0 + kq;
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row < M) {
                const float *p = Ab + row * K + k;
                if (vec_a && k + 4 <= K) {
                    x = *reinterpret_cast<const float4 *>(p);
                } else {
                    if (k + 0 < K) x.x = p[0];
                    if (k + 1 < K) x.y = p[1];
                    if (k + 2 < K) x.z = p[2];
                    if (k + 3 < K) x.w = p[3];
                }
            }
            ra = x;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int kr = idx / 32, nq = (idx % 32) * 4;
            const int64_t k = k0 + kr, col = n0 + nq;
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k < K) {
                const float *p = Bb + k * N + col;
                if (vec_b && col + 4 <= N) {
                    x = *reinterpret_cast<const float4 *>(p);
                } else {
                    if (col + 0 < N) x.x = p[0];
                    if (col + 1 < N) x.y = p[1];
                    if (col + 2 < N) x.z = p[2];
                    if (col + 3 < N) x.w = p[3];
                }
            }
            rb[i] = x;
        }
    };
    const auto store = [&](int buf) {
        const int r = tid / 4, kq = (tid % 4) * 4;
        la[buf][(kq + 0) * kPadA + r] = ra.x;
        la[buf][(kq + 1) * kPadA + r] = ra.y;
        la[buf][(kq + 2) * kPadA + r] = ra.z;
        la[buf][(kq + 3) * kPadA + r] = ra.w;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int kr = idx / 32, nq = (idx % 32) * 4;
            *reinterpret_cast<float4 *>(&lb[buf][kr * kPadB + nq]) = rb[i];
        }
    };

    float4v acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = float4v{};

    const int64_t steps = (K + kGBK - 1) / kGBK;
    load(0);
    store(0);
    __syncthreads();
    const int lr = lane & 15, lk = lane >> 4;
    for (int64_t s = 0; s < steps; ++s) {
        const int cur = s & 1;
        if (s + 1 < steps) load((s + 1) * kGBK);
#pragma unroll
        for (int kk = 0; kk < kGBK; kk += 4) {
            float av[2], bv[4];
#pragma unroll
            for (int i = 0; i < 2; ++i) av[i] = la[cur][(kk + lk) * kPadA + wr * 32 + 16 * i + lr];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = lb[cur][(kk + lk) * kPadB + wc * 64 + 16 * j + lr];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < steps) store(cur ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int64_t row = m0 + wr * 32 + 16 * i + 4 * lk + e;
                const int64_t col = n0 + wc * 64 + 16 * j + lr;
                if (row < M && col < N) Cb[row * N + col] = acc[i][j][e];
            }
}

// ------------------------------------------------------------------ 4. outputs

// Y = A^T M A * 2^shift[oc] of the tile's alpha^2 products, then the sum
// begun from the residual (from_redirect) and the chain, one thread per
// (oc, tile), consecutive threads consecutive tiles.  shift null: no scale.
// The products may come in `splits` parts over the input channels (the small
// images' path), each with its own scale, prod[s][xi][oc][ld] and
// shift[s][oc]; they are added in the order of s.
template <int M, bool PAIRS = false>
__global__ __launch_bounds__(256) void outputs_kernel(WinogradArgs a, const float *__restrict__ prod,
                                                      const int32_t *__restrict__ shift, int64_t splits,
                                                      int64_t ld) {
    constexpr int A = Mat<M>::A;
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= static_cast<uint32_t>(a.tiles * a.oc)) return;
    const uint32_t oc = t / static_cast<uint32_t>(a.tiles);
    const uint32_t tile = t - oc * static_cast<uint32_t>(a.tiles);
    uint32_t tx, ty, n;
    split_index(tile, static_cast<uint32_t>(a.tw), static_cast<uint32_t>(a.th), tx, ty, n);
    if (ld == 0) ld = a.tiles;
    const int64_t plane = a.oc * ld;
    // The splits' sums added in their order; with PAIRS, the loads of two
    // splits at once.
    float m[A][A];
    if constexpr (!PAIRS) {
        for (int64_t sp = 0; sp < splits; ++sp) {
            const int unscale = shift != nullptr ? shift[sp * a.oc + oc] : 0;
            const float *part = prod + sp * A * A * plane + static_cast<int64_t>(oc) * ld + tile;
#pragma unroll
            for (int i = 0; i < A; ++i)
#pragma unroll
                for (int j = 0; j < A; ++j) {
                    const float v = ldexpf(part[(i * A + j) * plane], unscale);
                    m[i][j] = sp == 0 ? v : __fadd_rn(m[i][j], v);
                }
        }
    } else {
        const auto part = [&](int64_t sp, float (&p)[A][A]) {
            const int unscale = shift[sp * a.oc + oc];
            const float *src = prod + sp * A * A * plane + static_cast<int64_t>(oc) * ld + tile;
#pragma unroll
            for (int i = 0; i < A; ++i)
#pragma unroll
                for (int j = 0; j < A; ++j) p[i][j] = ldexpf(src[(i * A + j) * plane], unscale);
        };
        part(0, m);
        int64_t sp = 1;
        for (; sp + 1 < splits; sp += 2) {
            float p0[A][A], p1[A][A];
            part(sp, p0);
            part(sp + 1, p1);
#pragma unroll
            for (int i = 0; i < A; ++i)
#pragma unroll
                for (int j = 0; j < A; ++j) m[i][j] = __fadd_rn(__fadd_rn(m[i][j], p0[i][j]), p1[i][j]);
        }
        if (sp < splits) {
            float p0[A][A];
            part(sp, p0);
#pragma unroll
            for (int i = 0; i < A; ++i)
#pragma unroll
                for (int j = 0; j < A; ++j) m[i][j] = __fadd_rn(m[i][j], p0[i][j]);
        }
    }
    float am[M][A];
#pragma unroll
    for (int i = 0; i < M; ++i)
#pragma unroll
        for (int j = 0; j < A; ++j) {
            float s = 0.0f;
#pragma unroll
            for (int x = 0; x < A; ++x) s += Mat<M>::at(i, x) * m[x][j];
            am[i][j] = s;
        }
    // The tile's M x M outputs, their loads (the residual, the chain's
    // operands) all before their stores.  A tile inside the image whose rows
    // are aligned (`vec`) moves whole rows of M; at the edges, outputs past
    // the image read its last row or column and are not stored.
    float v[M * M];
#pragma unroll
    for (int i = 0; i < M; ++i)
#pragma unroll
        for (int jj = 0; jj < M; ++jj) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < A; ++j) s += am[i][j] * Mat<M>::at(jj, j);
            v[i * M + jj] = s;
        }
    using Row = typename RowOf<M>::type;
    const int64_t y0 = static_cast<int64_t>(ty) * M, x0 = static_cast<int64_t>(tx) * M;
    const bool full = y0 + M <= a.oh && x0 + M <= a.ow;
    const auto yy = [&](int e) -> int64_t {
        const int64_t y = y0 + e / M;
        return y < a.oh ? y : a.oh - 1;
    };
    const auto xx = [&](int e) -> int64_t {
        const int64_t x = x0 + e % M;
        return x < a.ow ? x : a.ow - 1;
    };
    const auto aligned = [&](const void *p, int64_t nb1, int64_t nb2, int64_t nb3) {
        return (reinterpret_cast<uintptr_t>(p) % (4 * M)) == 0 && nb1 % M == 0 && nb2 % M == 0 && nb3 % M == 0;
    };
    float *out = a.y + static_cast<int64_t>(n) * a.ynb3 + static_cast<int64_t>(oc) * a.ynb2;
    const bool vec = full && aligned(a.y, a.ynb1, a.ynb2, a.ynb3);
    if (a.from_redirect) {
        float r[M * M];
        if (vec) {
#pragma unroll
            for (int i = 0; i < M; ++i) {
                const Row q = *reinterpret_cast<const Row *>(out + (y0 + i) * a.ynb1 + x0);
#pragma unroll
                for (int j = 0; j < M; ++j) r[i * M + j] = q[j];
            }
        } else {
#pragma unroll
            for (int e = 0; e < M * M; ++e) r[e] = out[yy(e) * a.ynb1 + xx(e)];
        }
#pragma unroll
        for (int e = 0; e < M * M; ++e) v[e] = __fadd_rn(r[e], v[e]);
    }
#pragma unroll 1
    for (int s = 0; s < a.chain.count; ++s) {
        const DevStep &st = a.chain.steps[s];
        if (st.kind == 2) {
#pragma unroll
            for (int e = 0; e < M * M; ++e) v[e] = silu(v[e]);
            continue;
        }
        const float *base = st.operand + static_cast<int64_t>(oc) * st.nb[2] + static_cast<int64_t>(n) * st.nb[3];
        float o[M * M];
        if (st.nb[0] == 0 && st.nb[1] == 0) {
            const float b = *base;
#pragma unroll
            for (int e = 0; e < M * M; ++e) o[e] = b;
        } else if (full && st.nb[0] == 1 && aligned(st.operand, st.nb[1], st.nb[2], st.nb[3])) {
#pragma unroll
            for (int i = 0; i < M; ++i) {
                const Row q = *reinterpret_cast<const Row *>(base + (y0 + i) * st.nb[1] + x0);
#pragma unroll
                for (int j = 0; j < M; ++j) o[i * M + j] = q[j];
            }
        } else {
#pragma unroll
            for (int e = 0; e < M * M; ++e) o[e] = base[xx(e) * st.nb[0] + yy(e) * st.nb[1]];
        }
        if (st.kind == 0) {
#pragma unroll
            for (int e = 0; e < M * M; ++e) v[e] = __fadd_rn(v[e], o[e]);
        } else {
#pragma unroll
            for (int e = 0; e < M * M; ++e) v[e] = __fmul_rn(v[e], o[e]);
        }
    }
    if (vec) {
#pragma unroll
        for (int i = 0; i < M; ++i) {
            Row q;
#pragma unroll
            for (int j = 0; j < M; ++j) q[j] = v[i * M + j];
            *reinterpret_cast<Row *>(out + (y0 + i) * a.ynb1 + x0) = q;
        }
    } else {
#pragma unroll
        for (int e = 0; e < M * M; ++e) {
            const int64_t y = y0 + e / M;
            const int64_t x = x0 + e % M;
            if (y < a.oh && x < a.ow) out[y * a.ynb1 + x] = v[e];
        }
    }
}

// ------------------------------------------------------------------ small images

// Images of few tiles (the deepest levels of SD's UNet: 16x16 by F(4x4) and
// 8x8 by F(2x2), 32 tiles for two images) take a path of their own, as the
// reference's small path does (winograd.cc:1069-1144): the transformed
// weights are never written out -- at this size they would be 16/9 or 4 times
// the FP16 weights, read back once each -- but made in registers from the
// FP16 kernels, straight into the MFMA's operands.
//
//   inputs:   V[xi][part][c / 32][tile][c % 32] * 2^-e_c as two FP16 planes,
//             tiles padded to tp (16 or 32) with zeros; beside it, in the
//             same launch, each split's exponent a_os of every output
//             channel from its greatest weight (a wave a pair);
//   products: a block of A waves per (16 output channels, split of the input
//             channels), wave i taking row i of U, so that each kernel is read
//             once.  A step is 32 input
//             channels, eight a lane: the lane makes row i of G g of each of
//             its kernels, scaled by 2^(a_os + e_c - E) -- a_os from the
//             split's greatest weight of the output channel, as a_o from the
//             channel's (section 0) -- then each of the row's A numbers of U
//             in turn, split into the operand A of v_mfma_f32_16x16x32_f16,
//             and V's parts of that point are its operand B: the three
//             products of split parts into the tiles' sums.  Each split's sums
//             go to M[s][xi][oc][tp], and its scale shift[s][oc] = E - a_os;
//   outputs:  the splits added in their order (outputs_kernel).
constexpr int kSmallTilesMax = 32;

typedef unsigned short ushort2v __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));

// The blocks from `iblocks` on take the weights' exponents instead, a wave
// per (split, output channel): a_os = kTop - the exponent above the split's
// greatest |weight| of channel o times the weight transform's gain (0 for a
// channel of zeros), read as the 16-byte pieces of its 9 split_len
// consecutive FP16 numbers, whose magnitudes compare as their bits, two to
// a register.
template <int M>
__device__ __forceinline__ void weights_split_max(const WinogradArgs &a, int64_t split_len, int64_t item,
                                                  int32_t *__restrict__ ao) {
    const int lane = threadIdx.x & 63;
    const int64_t sp = item / a.oc, o = item - sp * a.oc;
    const int64_t c_begin = sp * split_len;
    const int64_t c_end = c_begin + split_len < a.ic ? c_begin + split_len : a.ic;
    ushort2v big = {0, 0};
    if (c_begin < c_end) {
        // (o ic + c_begin) is a multiple of 8: the run starts 16-byte aligned
        // and is whole pieces of 8 numbers.
        const int4v *run = reinterpret_cast<const int4v *>(a.w + (o * a.ic + c_begin) * 9);
        const int64_t pieces = (c_end - c_begin) * 9 / 8;
        for (int64_t q = lane; q < pieces; q += 64) {
            const int4v w = run[q];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                big = __builtin_elementwise_max(big, __builtin_bit_cast(ushort2v, w[k] & 0x7fff7fff));
        }
    }
    int bits = big.x > big.y ? big.x : big.y;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) bits = max(bits, __shfl_xor(bits, off, 64));
    if (lane == 0) {
        const float wm = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(bits)));
        ao[item] = wm > 0.0f ? kTop - exponent_above(wm * Mat<M>::kWeightGain) : 0;
    }
}

template <int M>
__global__ __launch_bounds__(256) void inputs_small_kernel(WinogradArgs a, int64_t kp, int64_t tp,
                                                           const int32_t *__restrict__ e, _Float16 *__restrict__ v,
                                                           int64_t iblocks, int64_t split_len, int64_t splits,
                                                           int32_t *__restrict__ ao) {
    constexpr int A = Mat<M>::A;
    if (blockIdx.x >= iblocks) {
        const int64_t item = (static_cast<int64_t>(blockIdx.x) - iblocks) * 4 + (threadIdx.x >> 6);
        if (item < splits * a.oc) weights_split_max<M>(a, split_len, item, ao);
        return;
    }
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= tp * kp) return;
    const int64_t tile = idx / kp, c = idx - tile * kp;
    float x[A][A] = {};
    if (c < a.ic && tile < a.tiles) {
        transform_d<M>(a, static_cast<uint32_t>(tile), static_cast<uint32_t>(c), x);
        const int s = -e[c];
#pragma unroll
        for (int r = 0; r < A; ++r)
#pragma unroll
            for (int q = 0; q < A; ++q) x[r][q] = ldexpf(x[r][q], s);
    }
    // [c / 32][tile][c % 32] in each plane: the 16 tiles by 32 channels a
    // wave of the products reads at once are 1 KB in a row.
    const int64_t plane = tp * kp;
    const int64_t at = ((c >> 5) * tp + tile) * 32 + (c & 31);
#pragma unroll
    for (int r = 0; r < A; ++r)
#pragma unroll
        for (int q = 0; q < A; ++q) {
            _Float16 hi, lo;
            split2(x[r][q], hi, lo);
            const int64_t xi = r * A + q;
            v[(2 * xi) * plane + at] = hi;
            v[(2 * xi + 1) * plane + at] = lo;
        }
}

template <int M, int NT>
__global__ __launch_bounds__(64 * Mat<M>::A) void products_small_kernel(WinogradArgs a, int64_t kp, int64_t split_len,
                                                                        int64_t oc_blocks, const int32_t *__restrict__ e,
                                                                        const _Float16 *__restrict__ v,
                                                                        float *__restrict__ prod,
                                                                        int32_t *__restrict__ shift,
                                                                        const int32_t *__restrict__ ao_split) {
    constexpr int A = Mat<M>::A;
    constexpr int TP = 16 * NT;  // tiles, padded
    const int lane = threadIdx.x & 63;
    const int row = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, kg = lane >> 4;
    // Consecutive blocks on one XCD take one split, whose V its L2 keeps.
    const int64_t b = xcd_swizzle(blockIdx.x, gridDim.x);
    const int64_t sp = b / oc_blocks;
    const int64_t o0 = (b - sp * oc_blocks) * 16;
    const int64_t o = o0 + lr;
    const bool o_in = o < a.oc;
    const int64_t og = o_in ? o : a.oc - 1;
    const int64_t c_begin = sp * split_len;
    const int64_t c_end = c_begin + split_len < kp ? c_begin + split_len : kp;

    int emax = kZeroChannel;
#pragma unroll 4
    for (int64_t c = 4 * lane; c < a.ic; c += 256) {
        const int4v q = *reinterpret_cast<const int4v *>(e + c);
        emax = max(emax, max(max(q[0], q[1]), max(q[2], q[3])));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) emax = max(emax, __shfl_xor(emax, off, 64));

    // The split's exponent of channel o (taken with the inputs' transform).
    const int ao = ao_split[sp * a.oc + og];
    if (row == 0 && kg == 0 && o_in) shift[sp * a.oc + o] = emax - ao;

    // The kernels of a step, 16 output channels by 32 input channels, copied
    // into LDS (two stages) by the block: a channel's 32 kernels are 36
    // pieces of 16 bytes, rows of 37 pieces (odd, so that the 16 rows a read
    // takes fall in distinct banks).  Pieces past the weights' end read their
    // last piece: finite numbers that meet V's zeros, as any past IC do.
    constexpr int kRowPieces = 37;
    constexpr int kCopies = (16 * kRowPieces + 63) / 64;
    __shared__ __attribute__((aligned(16))) char gbuf[2][kCopies * 1024];
    const int64_t w_last = a.oc * a.ic * 9 - 8;
    const auto copy_g = [&](int64_t c0, int stage) {
#pragma unroll
        for (int r = 0; r < (kCopies + A - 1) / A; ++r) {
            const int n = row + r * A;
            if (n >= kCopies) break;
            const int p = n * 64 + lane;
            int orow = p / kRowPieces, k = p - orow * kRowPieces;
            if (orow > 15) orow = 15;
            if (k > 35) k = 35;
            const int64_t oo = o0 + orow < a.oc ? o0 + orow : a.oc - 1;
            int64_t hw = (oo * a.ic + c0) * 9 + 8 * k;
            hw = hw < w_last ? hw : w_last;
            copy_lds(a.w + hw, gbuf[stage] + n * 1024);
        }
    };

    float4v acc[A][NT];
#pragma unroll
    for (int j = 0; j < A; ++j)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[j][t] = float4v{};
    // Row `row` of G, the same for every lane of the wave.
    const float r0 = Mat<M>::g(row, 0), r1 = Mat<M>::g(row, 1), r2 = Mat<M>::g(row, 2);
    const int64_t plane = static_cast<int64_t>(TP) * kp;
    const _Float16 *vrow = v + static_cast<int64_t>(row * A) * 2 * plane;  // the same for the wave
    const uint32_t vlane = static_cast<uint32_t>(lr * 32 + 8 * kg);         // the lane's, in V's planes
    // V's parts of point (row, j) at step c0, operand B; each point's are
    // loaded again for the next step as soon as its MFMAs have them.
    half8 vb[A][NT][2];
    const auto load_v = [&](int j, int64_t c0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                const _Float16 *base = vrow + (2 * j + part) * plane + (c0 >> 5) * (TP * 32) + 16 * t * 32;
                vb[j][t][part] = *reinterpret_cast<const half8 *>(base + vlane);
            }
    };
    // The exponents e_c of the lane's eight channels at step c0.
    int4v e0, e1;
    const auto load_e = [&](int64_t c0) {
        const int64_t c = c0 + 8 * kg;
        const int4v *ep = reinterpret_cast<const int4v *>(e + (c < a.ic ? c : a.ic - 8));
        e0 = ep[0];
        e1 = ep[1];
    };
    copy_g(c_begin, 0);
    load_e(c_begin);
#pragma unroll
    for (int j = 0; j < A; ++j) load_v(j, c_begin);
    int stage = 0;
    for (int64_t c0 = c_begin; c0 < c_end; c0 += 32, stage ^= 1) {
        const int64_t next = c0 + 32 < c_end ? c0 + 32 : c0;  // past the last step: this one again
        // The step's kernels in (copied a step ahead: loads complete in the
        // order they were issued, and the exponents' two and V's 2 NT A
        // loads of the step went out after them); every wave past the step
        // before, whose stage the next step's kernels now overwrite.  The
        // exponents and V are waited for where they are used.
        wait_loads<2 + 2 * NT * A>();
        __syncthreads();
        int4v q[9];
        const char *gl = gbuf[stage] + (lr * kRowPieces + 9 * kg) * 16;
#pragma unroll
        for (int k = 0; k < 9; ++k) q[k] = *reinterpret_cast<const int4v *>(gl + 16 * k);
        if (c0 + 32 < c_end) copy_g(c0 + 32, stage ^ 1);
        const int64_t c = c0 + 8 * kg;
        const bool c_in = c < a.ic;
        // Row `row` of G g of each kernel, times 2^(a_os + e_c - E) and the
        // split's 2^-4 (zero past IC): the power of two goes into the row's
        // coefficients, which changes no rounding, and each term is a fused
        // multiply-add of an FP16 number as it is.
        float gi[8][3];
        const _Float16 *h = reinterpret_cast<const _Float16 *>(q);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const int ec = jj < 4 ? e0[jj] : e1[jj - 4];
            const float f = c_in ? ldexpf(1.0f, ao + ec - emax - 4) : 0.0f;
            const float s0 = r0 * f, s1 = r1 * f, s2 = r2 * f;
#pragma unroll
            for (int bb = 0; bb < 3; ++bb) {
                const float x0 = static_cast<float>(h[9 * jj + bb]);
                const float x1 = static_cast<float>(h[9 * jj + 3 + bb]);
                const float x2 = static_cast<float>(h[9 * jj + 6 + bb]);
                gi[jj][bb] = fmaf(s2, x2, fmaf(s1, x1, fmaf(s0, x0, 0.0f)));
            }
        }
        // The loads of the next step go out where they are written, each
        // point's V as soon as its MFMAs have read it, so that a whole step
        // covers their latency.
        __builtin_amdgcn_sched_barrier(0);
        load_e(next);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < A; ++j) {
            // U split two numbers at a time: the high parts rounded toward
            // zero (the remainder u - hi then exact in single precision), the
            // low parts from the remainders; hi + lo keeps 22 bits of u.
            half8 uh, ul;
#pragma unroll
            for (int jj = 0; jj < 8; jj += 2) {
                const float u0 =
                    dot3(Mat<M>::g(j, 0), gi[jj][0], Mat<M>::g(j, 1), gi[jj][1], Mat<M>::g(j, 2), gi[jj][2]);
                const float u1 = dot3(Mat<M>::g(j, 0), gi[jj + 1][0], Mat<M>::g(j, 1), gi[jj + 1][1],
                                      Mat<M>::g(j, 2), gi[jj + 1][2]);
                const fp16x2 h = __builtin_amdgcn_cvt_pkrtz(u0, u1);
                const fp16x2 l = __builtin_amdgcn_cvt_pkrtz(u0 - static_cast<float>(h[0]), u1 - static_cast<float>(h[1]));
                uh[jj] = h[0];
                uh[jj + 1] = h[1];
                ul[jj] = l[0];
                ul[jj + 1] = l[1];
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                acc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(uh, vb[j][t][0], acc[j][t], 0, 0, 0);
                acc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(uh, vb[j][t][1], acc[j][t], 0, 0, 0);
                acc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ul, vb[j][t][0], acc[j][t], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            load_v(j, next);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // Lane holds the sums of channels o0 + 4 kg + r, tile 16 t + lr; both
    // operands were scaled by 2^-4 in their splits.
    const int64_t oplane = a.oc * TP;
#pragma unroll
    for (int j = 0; j < A; ++j) {
        float *out = prod + (sp * A * A + row * A + j) * oplane;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t oo = o0 + 4 * kg + r;
                if (oo < a.oc) out[oo * TP + 16 * t + lr] = acc[j][t][r] * (kSplitUp * kSplitUp);
            }
    }
}

// ------------------------------------------------------------------ host

struct WorkLayout {
    int64_t kp;                          // IC padded to whole steps of K
    bool small;                          // the small images' path
    int64_t tp, splits, split_len;       // its tiles padded to 16, splits of the input channels
    size_t e, a, shift, f, u, v, m, total;  // byte offsets
};

// The small images' path: F(4x4) or F(2x2) on the reference's small images
// (few tiles in all, winograd.cc:194-196) of at most 32 tiles, FP16 kernels
// whose rows of eight channels are 16-byte aligned; not with winograd_fp32.
bool small_path(const WinogradArgs &a) {
    return !tuning().winograd_fp32 && a.w32 == nullptr && a.tiles <= kSmallTilesMax &&
           a.n * ((a.ow + 1) / 2) * ((a.oh + 1) / 2) <= tuning().winograd_small_tiles && a.ic % 8 == 0 &&
           (reinterpret_cast<uintptr_t>(a.w) & 15) == 0;
}

WorkLayout work_layout(const WinogradArgs &a) {
    const int64_t alpha2 = (a.m + 2) * (a.m + 2);
    WorkLayout l{};
    l.kp = round_up(a.ic, 32);
    size_t at = 0;
    const auto take = [&](int64_t bytes) {
        const size_t here = at;
        at += static_cast<size_t>(round_up(bytes, 256));
        return here;
    };
    l.small = small_path(a);
    if (l.small) {
        // Splits of the input channels: as many as give every CU one block
        // in a single round, two with F(2x2), whose blocks of four waves
        // then hide each other's latency (a round and a fraction leaves most
        // CUs idle through the fraction: measured, 1280 -> 1280 at 8x8 by
        // F(2x2), 80 blocks a split, 3 splits 50.4 us, 4 53.5, 5 50.1, 2
        // 58.7, 6 48.6); winograd_splits: that many instead.  Two steps or
        // more a split.
        l.tp = round_up(a.tiles, 16);
        const int64_t oc_blocks = ceil_div(a.oc, 16);
        const int64_t rounds = a.m == 2 ? 2 : 1;
        int64_t sp = tuning().winograd_splits > 0 ? tuning().winograd_splits : rounds * compute_units() / oc_blocks;
        sp = sp < 1 ? 1 : (sp > l.kp / 64 ? l.kp / 64 : sp);
        sp = sp < 1 ? 1 : sp;
        l.split_len = round_up(ceil_div(l.kp, sp), 32);
        l.splits = ceil_div(l.kp, l.split_len);
        l.e = take(a.ic * 4);
        l.a = take(l.splits * a.oc * 4);
        l.shift = take(l.splits * a.oc * 4);
        l.u = at;
        l.v = take(alpha2 * 2 * l.tp * l.kp * 2);
        l.m = take(l.splits * alpha2 * a.oc * l.tp * 4);
        l.total = at;
        return l;
    }
    // Either form: U as two FP16 planes [xi][part][kp / 32][oc][32] or in single
    // precision [xi][oc][ic] (kept weights live in the store instead); V as
    // two FP16 planes [xi][part][kp / 32][tile][32], or in single precision
    // [xi][ic][tile]; the factors f of kept weights' columns.
    l.e = take(a.ic * 4);
    l.a = take(a.oc * 4);
    l.shift = take(a.oc * 4);
    l.f = take(l.kp * 4);
    l.u = take(alpha2 * a.oc * l.kp * 4);
    l.v = take(alpha2 * l.kp * a.tiles * 4);
    l.m = take(alpha2 * a.oc * a.tiles * 4);
    l.total = at;
    return l;
}

// x's bytes from its first element past its last where F(4x4)'s inputs can
// be read by rows of whole quads (load_d_quads), else 0.
uint32_t quad_rows_bytes(const WinogradArgs &a) {
    if (a.m != 4 || a.p0 != 1 || a.iw % 4 != 0 || a.tw * 4 > a.iw || a.xnb1 % 4 != 0 || a.xnb2 % 4 != 0 ||
        a.xnb3 % 4 != 0 || a.xnb1 < a.iw || (reinterpret_cast<uintptr_t>(a.x) & 15) != 0)
        return 0;
    const int64_t floats = (a.n - 1) * a.xnb3 + (a.ic - 1) * a.xnb2 + (a.ih - 1) * a.xnb1 + a.iw;
    return floats * 4 < (int64_t{1} << 31) - 64 ? static_cast<uint32_t>(floats * 4) : 0;
}

template <int M>
sdhip_status run(const WinogradArgs &in, void *work, hipStream_t stream) {
    constexpr int A = Mat<M>::A;
    WinogradArgs a = in;
    a.xbytes = quad_rows_bytes(a);
    const char *tag = M == 4 ? "winograd4" : "winograd2";
    const WorkLayout l = work_layout(a);
    char *base = static_cast<char *>(work);
    int32_t *e = reinterpret_cast<int32_t *>(base + l.e);
    int32_t *a_oc = reinterpret_cast<int32_t *>(base + l.a);
    int32_t *shift = reinterpret_cast<int32_t *>(base + l.shift);
    float *u = reinterpret_cast<float *>(base + l.u);
    float *v = reinterpret_cast<float *>(base + l.v);
    float *m = reinterpret_cast<float *>(base + l.m);
    const std::string names[] = {std::string(tag) + ".scales",   std::string(tag) + ".weights",
                                 std::string(tag) + ".inputs",   std::string(tag) + ".products",
                                 std::string(tag) + ".outputs",  std::string(tag) + ".transforms"};
    if (tuning().winograd_fp32) {
        const int64_t n_in = a.tiles * a.ic;
        {
            KernelScope scope(names[1].c_str(), stream);
            if (a.w32 != nullptr) {
                SDHIP_LAUNCH((weights_kernel<M, float>), dim3(ceil_div(a.oc * a.ic, 256)), dim3(256), 0, stream,
                             a.w32, u, a.oc, a.ic);
            } else {
                SDHIP_LAUNCH((weights_kernel<M, _Float16>), dim3(ceil_div(a.oc * a.ic, 256)), dim3(256), 0,
                             stream, a.w, u, a.oc, a.ic);
            }
        }
        {
            KernelScope scope(names[2].c_str(), stream);
            SDHIP_LAUNCH((inputs_kernel<M>), dim3(ceil_div(n_in, 256)), dim3(256), 0, stream, a, v);
        }
        {
            KernelScope scope(names[3].c_str(), stream);
            const int64_t mb = ceil_div(a.oc, kGBM), nb = ceil_div(a.tiles, kGBN);
            SDHIP_LAUNCH(batched_gemm_f32, dim3(A * A * mb * nb), dim3(256), 0, stream, u, v, m, a.oc, a.tiles,
                         a.ic, mb, nb);
        }
        KernelScope scope(names[4].c_str(), stream);
        SDHIP_LAUNCH((outputs_kernel<M>), dim3(ceil_div(a.tiles * a.oc, 256)), dim3(256), 0, stream, a, m,
                     nullptr, int64_t{1}, int64_t{0});
        return launched(hipGetLastError(), "winograd");
    }
    if (l.small) {
        {
            KernelScope scope(names[0].c_str(), stream);  // the inputs' exponents only
            SDHIP_LAUNCH((scales_kernel<M>), dim3(static_cast<uint32_t>(a.ic)), dim3(256), 0, stream, a, e,
                         a_oc);
        }
        // Each split's exponents of the weights ([split][oc]) depend on the
        // weights and the splits alone: kept in the store when it has room,
        // as the reference keeps its weights' derived forms (store.cc:64-99),
        // so that later calls read none of the weights for them.
        const int64_t wne[4] = {3, 3, a.ic, a.oc};
        const int64_t wnb[4] = {2, 6, 18, 18 * a.ic};
        const uint64_t variant = static_cast<uint64_t>(M) | (static_cast<uint64_t>(l.splits) << 8) |
                                 (static_cast<uint64_t>(l.split_len) << 32);
        bool ready = false;
        int32_t *ao_kept = static_cast<int32_t *>(
            store_entry(a.w, SDHIP_TYPE_F16, wne, wnb, kStoreWinogradSmall, variant,
                        static_cast<size_t>(a.oc * a.ic * 18), static_cast<size_t>(l.splits * a.oc * 4), stream,
                        ready));
        int32_t *ao = ao_kept != nullptr ? ao_kept : a_oc;
        _Float16 *vh = reinterpret_cast<_Float16 *>(v);
        {
            // The inputs' transform, and beside it, unless kept, each split's
            // exponents of the weights.
            KernelScope scope(names[2].c_str(), stream);
            const int64_t iblocks = ceil_div(l.tp * l.kp, 256);
            const int64_t wblocks = ready ? 0 : ceil_div(l.splits * a.oc, 4);
            SDHIP_LAUNCH((inputs_small_kernel<M>), dim3(static_cast<uint32_t>(iblocks + wblocks)), dim3(256), 0,
                         stream, a, l.kp, l.tp, e, vh, iblocks, l.split_len, l.splits, ao);
            const hipError_t err = hipGetLastError();
            if (err != hipSuccess) return launched(err, "winograd inputs (small images)");
            if (ao_kept != nullptr && !ready) store_publish(ao_kept);
        }
        {
            KernelScope scope(names[3].c_str(), stream);
            const int64_t oc_blocks = ceil_div(a.oc, 16);
            const dim3 grid(static_cast<uint32_t>(oc_blocks * l.splits));
            const dim3 block(64 * A);
            if (l.tp <= 16) {
                SDHIP_LAUNCH((products_small_kernel<M, 1>), grid, block, 0, stream, a, l.kp, l.split_len,
                             oc_blocks, e, vh, m, shift, ao);
            } else {
                SDHIP_LAUNCH((products_small_kernel<M, 2>), grid, block, 0, stream, a, l.kp, l.split_len,
                             oc_blocks, e, vh, m, shift, ao);
            }
        }
        KernelScope scope(names[4].c_str(), stream);
        SDHIP_LAUNCH((outputs_kernel<M, true>), dim3(ceil_div(a.tiles * a.oc, 256)), dim3(256), 0, stream, a, m,
                     shift, l.splits, l.tp);
        return launched(hipGetLastError(), "winograd (small images)");
    }
    // The transformed weights U 2^a_o and their exponents a_o, kept in the
    // store when it has room: they depend on the weights alone, and the
    // inputs' exponents come in as the products read U.  Without the store
    // (the reference keeps no single-precision transformed weights by
    // default, store.h:26-34), U 2^(a_o + e_c - E) is made at every call
    // already split into two FP16 planes, which the products read as they are.
    const int64_t wne[4] = {3, 3, a.ic, a.oc};
    const int64_t wsize = a.w32 != nullptr ? 4 : 2;
    const int64_t wnb[4] = {wsize, 3 * wsize, 9 * wsize, 9 * wsize * a.ic};
    const void *wdata = a.w32 != nullptr ? static_cast<const void *>(a.w32) : static_cast<const void *>(a.w);
    const size_t a_bytes = static_cast<size_t>(round_up(a.oc * 4, 256));
    const size_t u_bytes = static_cast<size_t>(A * A * a.oc * l.kp * 4);
    bool ready = false;
    char *kept = static_cast<char *>(store_entry(wdata, a.w32 != nullptr ? SDHIP_TYPE_F32 : SDHIP_TYPE_F16, wne, wnb,
                                                 kStoreWinograd, M, static_cast<size_t>(a.oc * a.ic * 9 * wsize),
                                                 a_bytes + u_bytes, stream, ready));
    int32_t *a_kept = kept != nullptr ? reinterpret_cast<int32_t *>(kept) : a_oc;
    float *u_kept = kept != nullptr ? reinterpret_cast<float *>(kept + a_bytes) : nullptr;
    float *f = kept != nullptr ? reinterpret_cast<float *>(base + l.f) : nullptr;
    {
        // The inputs' exponents, and the weights' unless kept.
        KernelScope scope(names[0].c_str(), stream);
        const int64_t waves = ready ? a.ic : a.ic + a.oc;
        SDHIP_LAUNCH((scales_kernel<M>), dim3(static_cast<uint32_t>(waves)), dim3(256), 0, stream, a, e,
                     a_kept);
    }
    _Float16 *uh = reinterpret_cast<_Float16 *>(u);
    _Float16 *vh = reinterpret_cast<_Float16 *>(v);
    // The products' operands and core, chosen first: the inputs' transform
    // writes V in the layout the core reads.
    SplitBatchedArgs p{};
    if (kept != nullptr) {
        p.a32 = u_kept;
        p.a_scale = f;
        p.a_batch = a.oc * l.kp;
    } else {
        p.a = uh;
        p.a_plane = a.oc * l.kp;
        p.a_batch = 2 * p.a_plane;
    }
    p.b = vh;
    p.b_plane = a.tiles * l.kp;
    p.b_batch = 2 * p.b_plane;
    p.c = m;
    p.c_batch = a.oc * a.tiles;
    p.M = a.oc;
    p.N = a.tiles;
    p.K = l.kp;
    p.batches = A * A;
    // gemm_core 0 (the default) chooses by the shape: the core whose waves
    // load their own rows of B (gemm_core=3, four stages ahead) for grids of
    // up to twelve workgroups a CU, where it was measured faster (the UNet's
    // and the VAE's 64x64 .. 128x128 maps), the register-staged one (1) for
    // larger.  Core 3 reads V in runs of 8 channels, so that a lane's 16
    // bytes of a row are next to its neighbours'.
    int core = tuning().gemm_core;
    int stages = tuning().gemm_stages;
    if (core == 0) {
        const int64_t blocks3 = p.batches * ceil_div(p.M, 64) * ceil_div(p.N, 128);
        core = split_batched3_takes(p) && blocks3 <= 12 * 256 ? 3 : 1;
        if (core == 3) stages = 4;
    }
    a.v_by8 = core == 3 && split_batched3_takes(p) ? 1 : 0;
    if (kept == nullptr) {
        // Both transforms in one launch.
        KernelScope scope(names[5].c_str(), stream);
        const int64_t wgx = ceil_div(a.oc, kWeightOc), wblocks = wgx * ceil_div(l.kp, kWeightIc);
        const int64_t igx = ceil_div(a.tiles, kInTiles), iblocks = igx * (l.kp / kInChannels);
        SDHIP_LAUNCH((transforms_kernel<M>), dim3(static_cast<uint32_t>(wblocks + iblocks)), dim3(256), 0,
                     stream, a, l.kp, e, a_oc, uh, shift, vh, wgx, wblocks, igx);
    } else if (!ready) {
        KernelScope scope(names[1].c_str(), stream);
        const dim3 grid(static_cast<uint32_t>(ceil_div(a.oc * l.kp, 256)));
        if (a.w32 != nullptr) {
            SDHIP_LAUNCH((weights_scaled_kernel<M, float>), grid, dim3(256), 0, stream, a.w32, a.oc, a.ic, l.kp,
                         a_kept, u_kept);
        } else {
            SDHIP_LAUNCH((weights_scaled_kernel<M, _Float16>), grid, dim3(256), 0, stream, a.w, a.oc, a.ic, l.kp,
                         a_kept, u_kept);
        }
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return launched(err, "winograd weights");
        store_publish(kept);
    }
    if (kept != nullptr) {
        KernelScope scope(names[2].c_str(), stream);
        SDHIP_LAUNCH((inputs_split_kernel<M>), dim3(ceil_div(a.tiles, kInTiles), l.kp / kInChannels), dim3(256), 0,
                     stream, a, l.kp, e, vh, a_kept, f, shift);
    }
    {
        KernelScope scope(names[3].c_str(), stream);
        const hipError_t err = core == 3 && split_batched3_takes(p)
                                   ? launch_split_batched3(p, tuning().gemm_tiles, stages, stream)
                                   : launch_split_batched(p, gemm_shape(), stream);
        if (err != hipSuccess) return launched(err, "winograd products");
    }
    KernelScope scope(names[4].c_str(), stream);
    SDHIP_LAUNCH((outputs_kernel<M>), dim3(ceil_div(a.tiles * a.oc, 256)), dim3(256), 0, stream, a, m, shift,
                 int64_t{1}, int64_t{0});
    return launched(hipGetLastError(), "winograd");
}

}  // namespace

size_t winograd_work_size(const WinogradArgs &a) { return work_layout(a).total; }

sdhip_status winograd(const WinogradArgs &a, void *work, hipStream_t stream) {
    return a.m == 4 ? run<4>(a, work, stream) : run<2>(a, work, stream);
}

}  // namespace sdhip
