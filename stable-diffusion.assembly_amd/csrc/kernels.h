// The launchers of the library's kernels and the argument blocks they take,
// shared by the host code (api.cpp) and the kernels (*.hip).  Strides here
// are in elements, not bytes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device.h"

namespace sdhip {

// MUL_MAT: y[m][n] = sum_k x[m][k] w[n][k]; m over M = ne1 * ne2 * ne3 rows.
struct MulMatArgs {
    const float *x;
    int64_t ldx;
    const _Float16 *w;
    int64_t ldw;
    // Single-precision weights, split (split_weights): w the hi plane, the lo
    // plane w_plane halves after it, rows ldw (a multiple of 32) apart, zeros
    // past K; row n scaled by 1 / w_scale[n], a power of two, which the
    // epilogue undoes.  Null w_scale: FP16 weights as they are.
    int64_t w_plane;
    const float *w_scale;
    // The single-precision weights as the caller holds them (rows ldw32
    // floats apart), for the bits mode's quantizer; null for FP16 weights.
    const float *w32;
    int64_t ldw32;
    // The products of 16 bits (bits=16): x rounded to FP16 (1), or x and
    // the FP16 weights to bfloat16 (2), one MFMA a product.
    int32_t half16;
    float *y;  // the output, or the redirect, or the gated output
    int64_t ldy;
    int64_t M, N, K;
    int64_t ne1, ne2;  // the output's rows and matrices, for the chain's coordinates
    int64_t half;      // gated: N / 2
    int64_t col_blocks;
    int32_t from_redirect;
    DevChain chain;
};

// The shape of a product's launch: `stages`, the K steps its loads run ahead
// of its MFMAs (2 or 4; the gemm_stages tuning); `tiles`, its block of
// 64 TM x 64 TN given as TM TN (11, 21, 22), or 0 to choose by the size (the
// gemm_tiles tuning).
struct GemmShape {
    int stages;
    int tiles;
};

hipError_t launch_mul_mat(const MulMatArgs &p, GemmShape g, hipStream_t stream);
// MUL_MAT by panels of 64 tokens by 160 features, or 64 by 64 where those
// leave too few (FP16 weights, K a multiple of 64, rows 16-byte aligned),
// where the output holds 256 of them or more; `mode` is the mul_mat_panels
// tuning (0 none, 1 either shape, 2 the 64 by 160 only).
bool mul_mat_panels_taken(const MulMatArgs &p, int mode);
hipError_t launch_mul_mat_panels(const MulMatArgs &p, int mode, hipStream_t stream);
hipError_t launch_mul_mat_gated(const MulMatArgs &p, GemmShape g, hipStream_t stream);

// Single-precision weights [rows][k] (rows ld apart) split into two FP16
// planes for the products (gemm.hip): each row scaled by 2^s, s bringing its
// greatest |w| into [2^14, 2^15) (0 for a row of zeros), hi = fp16(w 2^s),
// lo = fp16(w 2^s - hi), rows kw (K rounded up to 32) halves apart and zeros
// past K, lo kw * rows halves after hi; scale[row] = 2^-s.  22 bits of each
// weight, as the activations' split keeps 22 of theirs.
size_t split_weights_bytes(int64_t rows, int64_t k);
hipError_t launch_split_weights(const float *w, int64_t ld, int64_t rows, int64_t k, void *out, hipStream_t stream);
// Where launch_split_weights puts the planes and the scales in `out`.
inline int64_t split_weights_ld(int64_t k) { return (k + 31) / 32 * 32; }
inline const _Float16 *split_weights_hi(const void *out) { return static_cast<const _Float16 *>(out); }
inline const float *split_weights_scale(const void *out, int64_t rows, int64_t k) {
    const size_t planes = static_cast<size_t>(2 * rows * split_weights_ld(k) * 2 + 255) / 256 * 256;
    return reinterpret_cast<const float *>(static_cast<const char *>(out) + planes);
}

// The direct convolution: y[n][oc][oy][ox] = sum over (ic, kh, kw).
struct ConvArgs {
    const float *x;  // [N][IC][IH][IW], strides xnb1..3
    int64_t xnb1, xnb2, xnb3;
    int64_t iw, ih, ic, n;
    const _Float16 *w;  // [OC][IC * KH * KW], rows ldw apart
    int64_t ldw;
    // Single-precision kernels, split as MulMatArgs's weights (w_split: the
    // call splits them, into rows ldw = K rounded up to 32 apart); null
    // w_scale: FP16 kernels as they are.
    int32_t w_split;
    int64_t w_plane;
    const float *w_scale;
    const float *w32;  // the kernel in single precision, for the bits mode's quantizer; null for FP16
    int32_t half16;    // the products of 16 bits (bits=16): the columns rounded to FP16 (1) or both operands to bfloat16 (2)
    int64_t kw, kh, oc;
    float *y;  // [N][OC][OH][OW], strides ynb1..3
    int64_t ynb1, ynb2, ynb3;
    int64_t ow, oh;
    int32_t s0, s1, p0, p1, d0, d1;
    int64_t K;      // ic * kh * kw
    int64_t taps;   // kh * kw
    int64_t plane;  // oh * ow
    int64_t P;      // n * plane
    int64_t oc_blocks;
    int32_t from_redirect;
    DevChain chain;
};

hipError_t launch_conv_direct(const ConvArgs &c, GemmShape g, hipStream_t stream);
// The 1x1 convolution by panels of 64 positions by 160 output channels
// (FP16 kernels, IC a multiple of 64, positions of an image a multiple of 64
// and contiguous in x and the output, rows 16-byte aligned), where the output
// holds enough of them and `enabled` (the conv_panels tuning).
bool conv_panels_taken(const ConvArgs &c, bool enabled);
hipError_t launch_conv_panels(const ConvArgs &c, hipStream_t stream);

// MUL_MAT split along K (gemm.hip): taken for products of fewer than 256
// output blocks of 64 x 64 whose K (a multiple of 32) gives two splits of 8
// K-steps or more, x and W rows 16-byte aligned; its work buffer holds the
// splits' partial sums.
bool mul_mat_split_taken(const MulMatArgs &p);
size_t mul_mat_split_work_size(const MulMatArgs &p);
// panels: the 64 x 160 panels split along K where K and N take them (the
// mul_mat_panels tuning), else the 64 x 64 core's splits.
hipError_t launch_mul_mat_split(const MulMatArgs &p, void *work, GemmShape g, bool panels, hipStream_t stream);

// The direct convolution by columns (gemm.hip): taken for kernels other than
// 1x1 whose K = IC KH KW is a multiple of 32 and whose FP16 weights are
// 16-byte aligned, columns of at most 2^28 numbers; its work buffer holds the
// columns and the splits' partial sums.
bool conv_columns_taken(const ConvArgs &c);
size_t conv_columns_work_size(const ConvArgs &c);
hipError_t launch_conv_columns(const ConvArgs &c, void *work, GemmShape g, hipStream_t stream);

// Batched products c[b][m][n] = sum_k a[b][m][k] b[b][n][k]: a already split
// into two FP16 planes (hi, and lo `a_plane` elements after it), each in
// blocks of 32 of K, [k / 32][m][k % 32], or single precision with a scale
// per column (a32, a_scale), K-contiguous rows of K elements; b already split
// into two FP16 planes (b_plane apart) in blocks, [k / 32][n][k % 32]; c's
// rows N apart.  Strides between batches in elements.  The caller pads: K a
// multiple of 32, a (or a32, a_scale) and b 16-byte aligned, a_batch,
// a_plane, b_batch and b_plane multiples of 8; hipErrorInvalidValue
// otherwise.
struct SplitBatchedArgs {
    const _Float16 *a;
    const _Float16 *b;  // B already split: hi, and lo `b_plane` elements after it
    float *c;
    int64_t a_batch, a_plane, b_batch, b_plane, c_batch;
    int64_t M, N, K, batches;
    int64_t m_blocks, n_blocks;
    // Instead of a: A in single precision (a32, batches a_batch apart), each
    // column k multiplied by a_scale[k] before the split.
    const float *a32;
    const float *a_scale;
};

hipError_t launch_split_batched(const SplitBatchedArgs &p, GemmShape g, hipStream_t stream);

// The same products by waves that load their own rows of B straight into
// their registers (gemm3.hip): B as two FP16 planes in runs of 8 of K, A as
// two FP16 planes or in single precision (a32, split on its way into LDS), K
// a multiple of 32, every plane and batch 16-byte aligned.  `tiles` 22, 41,
// 12 (not with a32) or 0 (64 x 128 blocks).
bool split_batched3_takes(const SplitBatchedArgs &p);
hipError_t launch_split_batched3(const SplitBatchedArgs &p, int tiles, int stages, hipStream_t stream);

}  // namespace sdhip
