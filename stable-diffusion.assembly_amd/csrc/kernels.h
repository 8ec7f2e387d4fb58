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
hipError_t launch_mul_mat_gated(const MulMatArgs &p, GemmShape g, hipStream_t stream);

// The direct convolution: y[n][oc][oy][ox] = sum over (ic, kh, kw).
struct ConvArgs {
    const float *x;  // [N][IC][IH][IW], strides xnb1..3
    int64_t xnb1, xnb2, xnb3;
    int64_t iw, ih, ic, n;
    const _Float16 *w;  // [OC][IC * KH * KW], contiguous
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

// MUL_MAT split along K (gemm.hip): taken for products of fewer than 256
// output blocks of 64 x 64 whose K (a multiple of 32) gives two splits of 32
// K-steps or more, x and W rows 16-byte aligned; its work buffer holds the
// splits' partial sums.
bool mul_mat_split_taken(const MulMatArgs &p);
size_t mul_mat_split_work_size(const MulMatArgs &p);
hipError_t launch_mul_mat_split(const MulMatArgs &p, void *work, GemmShape g, hipStream_t stream);

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

}  // namespace sdhip
