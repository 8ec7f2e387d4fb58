/*
 * The oracle: a CPU restatement, in plain C, of what the reference computes on
 * the path this library takes over.  TEST INFRASTRUCTURE ONLY -- the tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, as the
 * checker and as the CPU baseline; the library (libsdhip.so) never does.
 *
 * Two kinds of function:
 *   oracle_exact_*  float64 recomputations of an output and of the sum of the
 *                   magnitudes of the products it adds, as the reference's
 *                   tests compute them (tests/ops_test.cc:154-211, and the
 *                   exact() closures at 402-424, 450-462, 517-553, 745-767);
 *                   the metric is |y - exact| / magnitude.
 *   oracle_*        single-precision restatements of the reference's own
 *                   numerics, where the result must match bit for bit or
 *                   nearly (norm.cc, quant.cc, scalar_math.h, fusion.cc), and
 *                   of its algorithms where they serve as the CPU baseline
 *                   (port.c: the packed GEMM, Winograd, attention).
 *
 * Layouts are C arrays, outermost first, with the strides named.  FP16
 * operands are passed widened to float (exactly).  Each function cites the
 * reference file:line it follows.  Every function here is pinned by a check
 * in tests/test_oracle.py (closed forms, identities, brute force, invariants).
 */
#ifndef SDHIP_ORACLE_H
#define SDHIP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar math (sources/scalar_math.h:34-63) */
float oracle_exponential(float x);
float oracle_silu(float x);
float oracle_gelu(float x);
/* SiLU of n numbers in place. */
void oracle_silu_array(float *x, int64_t n);
/* exponential() and GELU of n numbers, into y. */
void oracle_exponential_array(const float *x, float *y, int64_t n);
void oracle_gelu_array(const float *x, float *y, int64_t n);
/* out = x * GELU(gate) of n numbers (fusion.cc:290-310). */
void oracle_gated_gelu_array(const float *x, const float *gate, float *out, int64_t n);

/* ---- float64 references (tests/ops_test.cc) */

/* y[m*N + n] = sum_k w[n*ldw + k] x[m*ldx + k]; mag the sum of |products|
 * (ops_test.cc:450-462). */
void oracle_exact_mul_mat(const float *w, int64_t ldw, const float *x, int64_t ldx, int64_t M, int64_t N,
                          int64_t K, double *y, double *mag);

/* x [n][ic][ih][iw], w [oc][ic][kh][kw] contiguous; y, mag [n][oc][oh][ow]
 * (ops_test.cc:402-424). */
void oracle_exact_conv2d(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w, int64_t oc,
                         int64_t kh, int64_t kw, int s0, int s1, int p0, int p1, int d0, int d1, int64_t oh,
                         int64_t ow, double *y, double *mag);

/* The same at `count` outputs only, their flat indices into y's layout. */
void oracle_exact_conv2d_at(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w,
                            int64_t oc, int64_t kh, int64_t kw, int s0, int s1, int p0, int p1, int d0, int d1,
                            int64_t oh, int64_t ow, const int64_t *index, int64_t count, double *y, double *mag);

/* q [b][lq][h][d], k [b][lk][hk][d], v [b][lk][hk][dv]; y, mag
 * [b][lq][h][dv]: the textbook softmax in double (ops_test.cc:517-553). */
void oracle_exact_attention(const float *q, const float *k, const float *v, int64_t d, int64_t dv, int64_t lq,
                            int64_t lk, int64_t h, int64_t hk, int64_t b, float scale, double *y, double *mag);

/* The same for `count` queries only, each (bi * h + hi) * lq + i; y, mag
 * [count][dv]. */
void oracle_exact_attention_at(const float *q, const float *k, const float *v, int64_t d, int64_t dv, int64_t lq,
                               int64_t lk, int64_t h, int64_t hk, int64_t b, float scale, const int64_t *query,
                               int64_t count, double *y, double *mag);

/* The gated GELU after a linear layer with bias (ops_test.cc:745-767):
 * w [2 half][K], x [M][K], bias [2 half]; y, mag [M][half]. */
void oracle_exact_gated(const float *w, const float *x, const float *bias, int64_t M, int64_t half, int64_t K,
                        double *y, double *mag);

/* ---- single-precision restatements */

/* The chain (fusion.cc:77-99): steps applied in order to out[] of extents
 * ne[4] (contiguous), kinds 0 add, 1 mul, 2 silu; operand s has element
 * strides nb[s*4 + k] (0 where broadcast). */
void oracle_apply_chain(float *out, const int64_t ne[4], int count, const int *kinds, const float *const *operands,
                        const int64_t *nb);

/* GROUP_NORM (norm.cc:100-140), x, y contiguous [ne3][ne2][ne1][ne0]. */
void oracle_group_norm(const float *x, float *y, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, int groups,
                       float eps);
/* NORM over rows of ne0 (norm.cc:148-175), contiguous. */
void oracle_norm(const float *x, float *y, int64_t ne0, int64_t rows, float eps);

/* ---- bits mode (sources/quant.h, quant.cc) */

/* A row's group of inputs, n <= group of them, into `group` bytes
 * (quant.cc:282-315): the scale and offset returned. */
void oracle_quantize_input_row(const float *x, int64_t n, int64_t group, int levels, uint8_t *dst, float *scale,
                               float *offset);

/* Rows of k weights (stride ld) into q [rows][groups * group] (signed bytes),
 * scale, offset and the integer sum of each (row, group) [rows][groups]
 * (quant.cc:204-243). */
void oracle_quantize_weights(const float *w, int64_t ld, int64_t rows, int64_t k, int64_t group, int weight_max,
                             int weight_groups, int8_t *q, float *scale, float *offset, int32_t *sums);

/* The quantized MUL_MAT (mul_mat.cc:498-569 with qgemm, quant.cc:113-164):
 * y[m*N + n] = init (the residual, from_redirect; or 0) + per group g in order
 * t = fma(sa*sb, S, t); t = fma(-oa, ob, t), S the exact integer sum.
 * Also returns, if not null, the quantized inputs xq [M][groups*group], their
 * scales and offsets [M][groups], and the weights' (as
 * oracle_quantize_weights). */
void oracle_quantized_mul_mat(const float *w, const float *x, int64_t M, int64_t N, int64_t K, int64_t group,
                              int input_levels, int weight_max, int weight_groups, const float *init, float *y,
                              uint8_t *xq, float *xscale, float *xoffset, int8_t *wq, float *wscale, float *woffset,
                              int32_t *wsums);

/* The quantized product of operands already quantized (quant.cc:113-164):
 * y[m*N + n] = init (or 0) + per group g in order t = fma(xs*ws, S, t);
 * t = fma(-xo, wo, t); operands [rows][groups*group]. */
void oracle_qgemm(const uint8_t *xq, const float *xs, const float *xo, const int8_t *wq, const float *ws,
                  const float *wo, int64_t M, int64_t N, int64_t groups, int64_t group, const float *init, float *y);

/* The quantized direct convolution (conv2d.cc:338-483): the columns of each
 * output position (k = ic KH KW + kh KW + kw, zeros outside the image)
 * quantized as the linear layers' inputs per (position, group), the kernels
 * as their weights per (output channel, group) or per whole row, the
 * products summed as qgemm, begun from init (the residual's own layout,
 * [n][oc][oh][ow], with from_redirect) or 0.  x [n][ic][ih][iw], w
 * [oc][ic][kh][kw]; y [n][oc][oh][ow]. */
void oracle_quantized_conv2d(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w, int64_t oc,
                             int64_t kh, int64_t kw, int s0, int s1, int p0, int p1, int d0, int d1, int64_t oh,
                             int64_t ow, int64_t group, int input_levels, int weight_max, int weight_groups,
                             const float *init, float *y);

/* A mistake planted in the two quantized convolutions below, for tests that
 * show their checks see one: 0 none, 1 the direct convolution's columns and
 * kernels in tap-major order, 2 Winograd's weights per every input channel
 * instead of per stretch, 3 per stretch of one group. */
void oracle_set_plant(int mode);

/* Winograd F(2x2, 3x3) with quantized products (winograd.cc:1826-2103), the
 * form every Winograd convolution takes in the bits mode: the reference's
 * transforms in its order of single-precision operations, the points'
 * operands quantized per (tile, group) and per (output channel, group) -- or
 * per stretch of `stretch` input channels with weight_groups = 0 -- their
 * products as qgemm, the outputs' transform, added to y with from_redirect. */
void oracle_quantized_winograd2(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w,
                                int64_t oc, int p0, int p1, int64_t oh, int64_t ow, int64_t group, int input_levels,
                                int weight_max, int weight_groups, int64_t stretch, int from_redirect, float *y);

/* Self-attention with quantized products (attention.cc:612-824): keys
 * signed, one group over the head's d dimensions (group 4 ceil(d / 4)),
 * queries unsigned with a zero point likewise, the softmax scale folded into
 * their scales and offsets; the scores' maximum per query; then stretches of
 * key_block keys: the exponentials of the stretch (exponential() for its
 * multiples of 8 keys, expf for the rest, attention.cc:288-301), their sum in
 * double in key order, each query's quantized unsigned per `group` keys; the
 * values signed per (dimension, group of keys); the output summed group by
 * group as quant.cc:150-155 does and multiplied by float(1 / sum).
 * q [b][lq][h][d], k [b][lk][hk][d], v [b][lk][hk][dv]; y [b][lq][h][dv]. */
void oracle_quantized_attention(const float *q, const float *k, const float *v, int64_t d, int64_t dv, int64_t lq,
                                int64_t lk, int64_t h, int64_t hk, int64_t b, float scale, int64_t group,
                                int input_levels, int weight_max, int64_t key_block, float *y);

/* ---- CPU-baseline restatements (port.c), threads OpenMP threads; built
 * for AVX-512 with VNNI: call oracle_port_available() first. */

/* 1 if this host runs port.c's code (AVX-512 F/BW/DQ/VL and VNNI). */
int oracle_port_available(void);

/* Winograd F(4x4, 3x3) of winograd.cc:1548-1613 with bias and residual:
 * x [n][ic][ih][iw], w [oc][ic][3][3] widened, y [n][oc][oh][ow]. */
void oracle_port_winograd4(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w, int64_t oc,
                           int p0, int p1, const float *bias, const float *residual, float *y, int threads);
/* Winograd F(2x2, 3x3), the same arguments. */
void oracle_port_winograd2(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w, int64_t oc,
                           int p0, int p1, const float *bias, const float *residual, float *y, int threads);
/* CONV_2D directly: x [n][ic][ih][iw], w [oc][ic][kh][kw], strides s0 (x),
 * s1 (y), pads p0, p1; bias [oc] and residual (as y) may be NULL. */
void oracle_port_conv2d(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w, int64_t oc,
                        int64_t kh, int64_t kw, int s0, int s1, int p0, int p1, const float *bias,
                        const float *residual, float *y, int threads);

/* MUL_MAT in single precision: y[m][n] = sum_k x[m][k] w[n][k] (+ bias[n]). */
void oracle_port_mul_mat(const float *w, const float *x, const float *bias, int64_t M, int64_t N, int64_t K, float *y,
                         int threads);

/* GROUP_NORM with gamma, beta (NULL: 1, 0) and SiLU; x, y [n][c][hw]. */
void oracle_port_group_norm(const float *x, float *y, int64_t n, int64_t c, int64_t hw, int groups, float eps,
                            const float *gamma, const float *beta, int silu, int threads);
/* NORM over rows of len, with gamma, beta. */
void oracle_port_norm(const float *x, float *y, int64_t rows, int64_t len, float eps, const float *gamma,
                      const float *beta, int threads);

/* FLASH_ATTN_EXT in single precision: q [b][lq][h][d], k [b][lk][h][d],
 * v [b][lk][h][dv], y [b][lq][h][dv]. */
void oracle_port_attention(const float *q, const float *k, const float *v, int64_t b, int64_t lq, int64_t lk,
                           int64_t h, int64_t d, int64_t dv, float scale, float *y, int threads);

/* The bits mode's MUL_MAT: weights quantized by oracle_quantize_weights and
 * packed once (oracle_port_qweights_bytes of memory), inputs quantized per
 * call; y [M][N] (+ bias); with `gated`, out [M][N / 2] = y[:, :N/2]
 * GELU(y[:, N/2:]).  Per group in the order of oracle_qgemm, so that y is
 * oracle_qgemm's bits (plus the bias). */
size_t oracle_port_qweights_bytes(int64_t N, int64_t groups, int64_t group);
void oracle_port_pack_qweights(const int8_t *wq, const float *ws, const float *wo, int64_t N, int64_t groups,
                               int64_t group, void *packed);
void oracle_port_quantized_linear(const float *x, int64_t M, int64_t K, const void *packed, int64_t N, int64_t group,
                                  int levels, const float *bias, float *y, int gated, float *out, int threads);

/* out [M][N / 2] = y[:, :N/2] GELU(y[:, N/2:]), the GEGLU of a product. */
void oracle_port_gated(const float *y, int64_t M, int64_t N, float *out, int threads);

/* The host's single-precision FMA rate on `threads` threads, GFLOP/s. */
/* The bits mode's self-attention (attention.cc:612-824) on AVX512-VNNI: the
 * oracle's algorithm, 16 keys or dimensions a vector (its exponentials by the
 * port's own polynomial, not bit for bit). */
void oracle_port_quantized_attention(const float *q, const float *k, const float *v, int64_t b, int64_t lq,
                                     int64_t lk, int64_t h, int64_t hk, int64_t d, int64_t dv, float scale,
                                     int64_t group, int levels, int wmax, int64_t key_block, float *y, int threads);
double oracle_port_fma_peak(int threads, double seconds);

#ifdef __cplusplus
}
#endif

#endif
