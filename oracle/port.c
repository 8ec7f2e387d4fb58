/*
 * CPU restatements of the reference's algorithms, in single precision (and
 * the bits mode's integer products), for bench.py's cpu_baseline leg: the
 * host-CPU figure beside each GPU one.  TEST INFRASTRUCTURE (oracle.h): the
 * library never calls these.
 *
 * They follow the reference's CPU design -- weights transformed or packed,
 * operands packed into panels, a register-tiled micro-kernel of FMAs
 * (gemm.cc / microkernel.cc: packed panels and a 6 x 16 tile of AVX2; here
 * 6 x 64 of AVX-512), Winograd's transforms around batched products per block
 * of tiles (winograd.cc:1548-1613), attention by blocks of queries with the
 * softmax between two products (attention.cc), the bits mode's products of
 * unsigned inputs by signed weights summed exactly per group (quant.cc:113-164,
 * here by AVX512-VNNI) -- with OpenMP threads in place of ggml's pool.  They
 * are this repository's code, not the reference's hand-written x86 kernels,
 * which cannot be built here (the reference needs ggml and C++26).
 *
 * Built for AVX-512 with VNNI (x86-64-v4); oracle_port_available() (oracle.c,
 * built without those) says whether this host runs them.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

typedef float v16 __attribute__((vector_size(64)));
typedef float v16u __attribute__((vector_size(64), aligned(4)));
typedef int32_t i16v __attribute__((vector_size(64)));

/* The micro-kernel's tile (MR rows by NR columns, NR = 4 vectors), the depth
 * of a packed step (a B micro-panel of KC x NR floats stays in L1), the rows
 * of a packed A block, and a parallel item's rows and panels. */
enum { MR = 6, NR = 64, KC = 128, MC = 96, MB = 48, NG = 2 };

static int64_t min64(int64_t a, int64_t b) { return a < b ? a : b; }
static int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

static void *alloc64(size_t bytes) {
    void *p = NULL;
    if (posix_memalign(&p, 64, bytes ? bytes : 64) != 0) abort();
    return p;
}

/* Buffers kept from one call to the next (slot per use; per thread for the
 * buffers of a thread's own), so that a timed call does not pay the first
 * touch of fresh pages -- the reference's pool keeps its buffers likewise.
 * The contents are not kept: each call writes what it reads. */
static void *kept(int slot, size_t bytes) {
    static void *buffers[8];
    static size_t sizes[8];
    if (sizes[slot] < bytes) {
        free(buffers[slot]);
        buffers[slot] = alloc64(bytes);
        sizes[slot] = bytes;
    }
    return buffers[slot];
}

static void *kept_local(int slot, size_t bytes) {
    static __thread void *buffers[6];
    static __thread size_t sizes[6];
    if (sizes[slot] < bytes) {
        free(buffers[slot]);
        buffers[slot] = alloc64(bytes);
        sizes[slot] = bytes;
    }
    return buffers[slot];
}

/* ------------------------------------------------------------ packing */

/* Rows [0, rows) and depth [0, kc) of A, element (i, k) at a[i sai + k sak],
 * into micro-panels of MR rows: ap[(i / MR) kc MR + k MR + i % MR], zero rows
 * past `rows`. */
static void pack_a(const float *a, int64_t sai, int64_t sak, int64_t rows, int64_t kc, float *ap) {
    for (int64_t ib = 0; ib < rows; ib += MR) {
        const int64_t r = min64(MR, rows - ib);
        float *dst = ap + ib * kc;
        if (sak == 1) {
            for (int64_t i = 0; i < MR; ++i) {
                const float *src = a + (ib + i) * sai;
                if (i < r) {
                    for (int64_t k = 0; k < kc; ++k) dst[k * MR + i] = src[k];
                } else {
                    for (int64_t k = 0; k < kc; ++k) dst[k * MR + i] = 0.0f;
                }
            }
        } else {
            for (int64_t k = 0; k < kc; ++k)
                for (int64_t i = 0; i < MR; ++i) dst[k * MR + i] = i < r ? a[(ib + i) * sai + k * sak] : 0.0f;
        }
    }
}

/* Panels [p0, p1) of B (K x N, element (k, n) at b[k rbs + n cbs]) over all of
 * K: panel p is [K][NR] at bp + p K NR, zero columns past N. */
static void pack_b(const float *b, int64_t rbs, int64_t cbs, int64_t K, int64_t N, int64_t p0, int64_t p1,
                   float *bp) {
    for (int64_t p = p0; p < p1; ++p) {
        float *dst = bp + p * K * NR;
        const int64_t n0 = p * NR, cols = min64(NR, N - n0);
        if (cbs == 1) {
            for (int64_t k = 0; k < K; ++k) {
                memcpy(dst + k * NR, b + k * rbs + n0, (size_t)cols * sizeof(float));
                for (int64_t j = cols; j < NR; ++j) dst[k * NR + j] = 0.0f;
            }
        } else {
            for (int64_t j = 0; j < NR; ++j) {
                if (j < cols) {
                    const float *src = b + (n0 + j) * cbs;
                    for (int64_t k = 0; k < K; ++k) dst[k * NR + j] = src[k * rbs];
                } else {
                    for (int64_t k = 0; k < K; ++k) dst[k * NR + j] = 0.0f;
                }
            }
        }
    }
}

static size_t packed_b_floats(int64_t K, int64_t N) { return (size_t)(cdiv(N, NR) * K * NR); }

/* ------------------------------------------------------------ the products */

/* The rows [0, rows) and columns [0, cols) of an MR x NR tile into C, by
 * masked vectors. */
static inline void store_partial(v16 acc[MR][4], float *c, int64_t ldc, int64_t rows, int64_t cols, int accumulate) {
    for (int64_t i = 0; i < rows; ++i)
        for (int j = 0; j < 4; ++j) {
            const int64_t live = cols - 16 * j;
            if (live <= 0) break;
            const __mmask16 mask = live >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << live) - 1u);
            float *d = c + i * ldc + 16 * j;
            __m512 v = (__m512)acc[i][j];
            if (accumulate) v = _mm512_add_ps(_mm512_maskz_loadu_ps(mask, d), v);
            _mm512_mask_storeu_ps(d, mask, v);
        }
}

/* C[0..rows)[0..cols) = (or += with accumulate) the MR x NR tile of a packed
 * A micro-panel by a packed B micro-panel over kc. */
static inline void micro(int64_t kc, const float *restrict a, const float *restrict b, float *restrict c, int64_t ldc,
                         int64_t rows, int64_t cols, int accumulate) {
    v16 acc[MR][4];
#pragma GCC unroll 6
    for (int i = 0; i < MR; ++i)
#pragma GCC unroll 4
        for (int j = 0; j < 4; ++j) acc[i][j] = (v16){0};
    for (int64_t k = 0; k < kc; ++k) {
        const v16 *bk = (const v16 *)(b + k * NR);
        const v16 b0 = bk[0], b1 = bk[1], b2 = bk[2], b3 = bk[3];
#pragma GCC unroll 6
        for (int i = 0; i < MR; ++i) {
            const v16 av = (v16)_mm512_set1_ps(a[k * MR + i]);
            acc[i][0] += av * b0;
            acc[i][1] += av * b1;
            acc[i][2] += av * b2;
            acc[i][3] += av * b3;
        }
    }
    if (rows == MR && cols == NR) {
#pragma GCC unroll 6
        for (int i = 0; i < MR; ++i)
#pragma GCC unroll 4
            for (int j = 0; j < 4; ++j) {
                v16u *d = (v16u *)(c + i * ldc + 16 * j);
                *d = accumulate ? *d + acc[i][j] : acc[i][j];
            }
        return;
    }
    store_partial(acc, c, ldc, rows, cols, accumulate);
}

/* C (M x N, row stride ldc) = A B, or += with accumulate, on this thread, for
 * B's panels [p0, p1): A element (i, k) at a[i sai + k sak]; bp packed by
 * pack_b over K; ab holds MC x KC floats. */
static void gemm1(int64_t M, int64_t N, int64_t K, const float *a, int64_t sai, int64_t sak, const float *bp,
                  int64_t p0, int64_t p1, float *c, int64_t ldc, int accumulate, float *ab) {
    for (int64_t k0 = 0; k0 < K; k0 += KC) {
        const int64_t kc = min64(KC, K - k0);
        for (int64_t i0 = 0; i0 < M; i0 += MC) {
            const int64_t mc = min64(MC, M - i0);
            pack_a(a + i0 * sai + k0 * sak, sai, sak, mc, kc, ab);
            for (int64_t p = p0; p < p1; ++p) {
                const float *b = bp + (p * K + k0) * NR;
                const int64_t cols = min64(NR, N - p * NR);
                for (int64_t ib = 0; ib < mc; ib += MR)
                    micro(kc, ab + ib * kc, b, c + (i0 + ib) * ldc + p * NR, ldc, min64(MR, mc - ib), cols,
                          accumulate || k0 > 0);
            }
        }
    }
}

/* As micro, with A's rows read in place (row i at a + i lda, rows past
 * `rows` reading the last) rather than packed. */
static inline void micro_rows(int64_t kc, const float *a, int64_t lda, const float *restrict b, float *restrict c,
                              int64_t ldc, int64_t rows, int64_t cols, int accumulate) {
    const float *ar[MR];
    for (int i = 0; i < MR; ++i) ar[i] = a + (i < rows ? i : rows - 1) * lda;
    v16 acc[MR][4];
#pragma GCC unroll 6
    for (int i = 0; i < MR; ++i)
#pragma GCC unroll 4
        for (int j = 0; j < 4; ++j) acc[i][j] = (v16){0};
    for (int64_t k = 0; k < kc; ++k) {
        const v16 *bk = (const v16 *)(b + k * NR);
        const v16 b0 = bk[0], b1 = bk[1], b2 = bk[2], b3 = bk[3];
#pragma GCC unroll 6
        for (int i = 0; i < MR; ++i) {
            const v16 av = (v16)_mm512_set1_ps(ar[i][k]);
            acc[i][0] += av * b0;
            acc[i][1] += av * b1;
            acc[i][2] += av * b2;
            acc[i][3] += av * b3;
        }
    }
    store_partial(acc, c, ldc, rows, cols, accumulate);
}

/* C (M x N) = A B on this thread with A's rows (stride lda) read in place:
 * for operands already in cache, where packing A would cost more than it
 * saves (attention's probabilities by the values). */
static void gemm_rows(int64_t M, int64_t N, int64_t K, const float *a, int64_t lda, const float *bp, float *c,
                      int64_t ldc) {
    const int64_t panels = cdiv(N, NR);
    for (int64_t k0 = 0; k0 < K; k0 += KC) {
        const int64_t kc = min64(KC, K - k0);
        for (int64_t p = 0; p < panels; ++p) {
            const float *b = bp + (p * K + k0) * NR;
            const int64_t cols = min64(NR, N - p * NR);
            for (int64_t i = 0; i < M; i += MR)
                micro_rows(kc, a + i * lda + k0, lda, b, c + i * ldc + p * NR, ldc, min64(MR, M - i), cols, k0 > 0);
        }
    }
}

/* gemm1 over `threads` threads, by items of MB rows and NG panels. */
static void par_gemm(int64_t M, int64_t N, int64_t K, const float *a, int64_t sai, int64_t sak, const float *bp,
                     float *c, int64_t ldc, int accumulate, int threads) {
    const int64_t mb = cdiv(M, MB), panels = cdiv(N, NR), ng = cdiv(panels, NG);
#pragma omp parallel num_threads(threads)
    {
        float *ab = (float *)kept_local(0, MC * KC * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (int64_t item = 0; item < mb * ng; ++item) {
            const int64_t i0 = (item / ng) * MB, g = item % ng;
            gemm1(min64(MB, M - i0), N, K, a + i0 * sai, sai, sak, bp, g * NG, min64(panels, g * NG + NG),
                  c + i0 * ldc, ldc, accumulate, ab);
        }
    }
}

/* B packed in parallel (pack_b over all panels). */
static float *par_pack_b(const float *b, int64_t rbs, int64_t cbs, int64_t K, int64_t N, int threads) {
    float *bp = (float *)kept(0, packed_b_floats(K, N) * sizeof(float));
    const int64_t panels = cdiv(N, NR);
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t p = 0; p < panels; ++p) pack_b(b, rbs, cbs, K, N, p, p + 1, bp);
    return bp;
}

/* ------------------------------------------------------------ MUL_MAT */

/* MUL_MAT in single precision (mul_mat.cc's packed path): the weights packed
 * once into panels, then the products by items of rows and panels; y[m][n] =
 * sum_k x[m][k] w[n][k] (+ bias[n]). */
void oracle_port_mul_mat(const float *w, const float *x, const float *bias, int64_t M, int64_t N, int64_t K, float *y,
                         int threads) {
    float *bp = par_pack_b(w, 1, K, K, N, threads);
    par_gemm(M, N, K, x, K, 1, bp, y, N, 0, threads);
    if (bias) {
#pragma omp parallel for num_threads(threads) schedule(static)
        for (int64_t m = 0; m < M; ++m)
            for (int64_t n = 0; n < N; ++n) y[m * N + n] += bias[n];
    }
}

/* ------------------------------------------------------------ direct convolution */

/* Panels [p0, p1) of one image's columns (k = c KH KW + dy KW + dx, n = the
 * output position), packed as pack_b packs, zeros outside the image. */
static void pack_columns(const float *x, int64_t ih, int64_t iw, int64_t kh, int64_t kw, int s0, int s1, int p0,
                         int p1, int64_t ow, int64_t K, int64_t P, int64_t q0, int64_t q1, float *bp) {
    for (int64_t p = q0; p < q1; ++p) {
        float *dst = bp + p * K * NR;
        const int64_t n0 = p * NR, cols = min64(NR, P - n0);
        for (int64_t k = 0; k < K; ++k) {
            const int64_t c = k / (kh * kw), dy = (k / kw) % kh, dx = k % kw;
            const float *plane = x + c * ih * iw;
            for (int64_t j = 0; j < NR; ++j) {
                float v = 0.0f;
                if (j < cols) {
                    const int64_t pos = n0 + j, oy = pos / ow, ox = pos % ow;
                    const int64_t yy = oy * s1 - p1 + dy, xx = ox * s0 - p0 + dx;
                    if (yy >= 0 && yy < ih && xx >= 0 && xx < iw) v = plane[yy * iw + xx];
                }
                dst[k * NR + j] = v;
            }
        }
    }
}

/* CONV_2D directly (conv2d.cc's path): per image, the columns packed into
 * panels (the image itself for a 1x1 kernel of stride 1), the kernel as the
 * rows; then the bias and the residual.  x [n][ic][ih][iw], w [oc][ic][kh][kw]
 * widened, y [n][oc][oh][ow]. */
void oracle_port_conv2d(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w, int64_t oc,
                        int64_t kh, int64_t kw, int s0, int s1, int p0, int p1, const float *bias,
                        const float *residual, float *y, int threads) {
    const int64_t oh = (ih + 2 * p1 - kh) / s1 + 1, ow = (iw + 2 * p0 - kw) / s0 + 1;
    const int64_t P = oh * ow, K = ic * kh * kw, panels = cdiv(P, NR);
    const int plain = kh == 1 && kw == 1 && s0 == 1 && s1 == 1 && p0 == 0 && p1 == 0;
    float *bp = (float *)kept(0, packed_b_floats(K, P) * sizeof(float));
    for (int64_t b = 0; b < n; ++b) {
        const float *img = x + b * ic * ih * iw;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
        for (int64_t p = 0; p < panels; ++p) {
            if (plain)
                pack_b(img, P, 1, K, P, p, p + 1, bp);
            else
                pack_columns(img, ih, iw, kh, kw, s0, s1, p0, p1, ow, K, P, p, p + 1, bp);
        }
        float *out = y + b * oc * P;
        par_gemm(oc, P, K, w, K, 1, bp, out, P, 0, threads);
        if (bias || residual) {
            const float *res = residual ? residual + b * oc * P : NULL;
#pragma omp parallel for num_threads(threads) schedule(static)
            for (int64_t o = 0; o < oc; ++o)
                for (int64_t q = 0; q < P; ++q) {
                    float s = out[o * P + q];
                    if (bias) s += bias[o];
                    if (res) s += res[o * P + q];
                    out[o * P + q] = s;
                }
        }
    }
}

/* ------------------------------------------------------------ Winograd F(4x4, 3x3) */

/* F(4x4, 3x3) matrices of winograd.cc:1155-1183, 1259-1264 (the points 0,
 * +-1, 2, -1/2 and infinity). */
static const float BT4[6][6] = {{1.0f, 1.5f, -2.0f, -1.5f, 1.0f, 0.0f},  {0.0f, -1.0f, -2.5f, -0.5f, 1.0f, 0.0f},
                                {0.0f, 1.0f, 0.5f, -2.5f, 1.0f, 0.0f},   {0.0f, -0.5f, -1.0f, 0.5f, 1.0f, 0.0f},
                                {0.0f, 2.0f, -1.0f, -2.0f, 1.0f, 0.0f},  {0.0f, 1.0f, 1.5f, -2.0f, -1.5f, 1.0f}};
static const float G4[6][3] = {{1.0f, 0.0f, 0.0f},
                               {-1.0f / 3, -1.0f / 3, -1.0f / 3},
                               {1.0f / 3, -1.0f / 3, 1.0f / 3},
                               {1.0f / 15, 2.0f / 15, 4.0f / 15},
                               {-16.0f / 15, 8.0f / 15, -4.0f / 15},
                               {0.0f, 0.0f, 1.0f}};
static const float AT4[4][6] = {{1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 0.0f},
                                {0.0f, 1.0f, -1.0f, 2.0f, -0.5f, 0.0f},
                                {0.0f, 1.0f, 1.0f, 4.0f, 0.25f, 0.0f},
                                {0.0f, 1.0f, -1.0f, 8.0f, -0.125f, 1.0f}};

/* F(2x2, 3x3): inputs B^T d B, weights G g G^T, outputs A^T m A. */
static const float BT2[4][4] = {{1, 0, -1, 0}, {0, 1, 1, 0}, {0, -1, 1, 0}, {0, 1, 0, -1}};
static const float G2[4][3] = {{1, 0, 0}, {0.5f, 0.5f, 0.5f}, {0.5f, -0.5f, 0.5f}, {0, 0, 1}};
static const float AT2[2][4] = {{1, 1, 1, 0}, {0, 1, -1, -1}};

/* ---- the transforms, 16 channels a vector */

/* B^T d B of 16 channels at once (d, out [A A] vectors; A = 6 for F(4x4), 4
 * for F(2x2)); the matrices' zeros skipped. */
static inline void input_vec(const v16 *d, int A, const float *bt, v16 *out) {
    v16 t[36];
#pragma GCC unroll 6
    for (int r = 0; r < A; ++r)
#pragma GCC unroll 6
        for (int j = 0; j < A; ++j) {
            v16 acc = (v16){0};
#pragma GCC unroll 6
            for (int i = 0; i < A; ++i)
                if (bt[r * A + i] != 0.0f) acc += bt[r * A + i] * d[i * A + j];
            t[r * A + j] = acc;
        }
#pragma GCC unroll 6
    for (int r = 0; r < A; ++r)
#pragma GCC unroll 6
        for (int c = 0; c < A; ++c) {
            v16 acc = (v16){0};
#pragma GCC unroll 6
            for (int j = 0; j < A; ++j)
                if (bt[c * A + j] != 0.0f) acc += t[r * A + j] * bt[c * A + j];
            out[r * A + c] = acc;
        }
}

/* G g G^T of 16 kernels at once (g [9] vectors, out [A A]). */
static inline void weight_vec(const v16 *g, int A, const float *gm, v16 *out) {
    v16 gg[18];
#pragma GCC unroll 6
    for (int i = 0; i < A; ++i)
#pragma GCC unroll 3
        for (int j = 0; j < 3; ++j) {
            v16 acc = (v16){0};
#pragma GCC unroll 3
            for (int e = 0; e < 3; ++e)
                if (gm[i * 3 + e] != 0.0f) acc += gm[i * 3 + e] * g[e * 3 + j];
            gg[i * 3 + j] = acc;
        }
#pragma GCC unroll 6
    for (int i = 0; i < A; ++i)
#pragma GCC unroll 6
        for (int j = 0; j < A; ++j) {
            v16 acc = (v16){0};
#pragma GCC unroll 3
            for (int e = 0; e < 3; ++e)
                if (gm[j * 3 + e] != 0.0f) acc += gg[i * 3 + e] * gm[j * 3 + e];
            out[i * A + j] = acc;
        }
}

/* The 3 x 3 kernels of 16 output channels [o0, o0 + 16) (those past oc
 * zero) at input channel c, as 9 vectors over the channels. */
static inline void gather_kernels(const float *w, int64_t oc, int64_t ic, int64_t o0, int64_t c, v16 *g) {
    const int32_t stride = (int32_t)(ic * 9);
    const __m512i index = _mm512_mullo_epi32(_mm512_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15),
                                             _mm512_set1_epi32(stride));
    const int64_t live = oc - o0;
    const __mmask16 mask = live >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << (live > 0 ? live : 0)) - 1u);
    const float *base = w + (o0 * ic + c) * 9;
    for (int e = 0; e < 9; ++e)
        g[e] = (v16)_mm512_mask_i32gather_ps(_mm512_setzero_ps(), mask, index, base + e, 4);
}

/* The weights transformed into packed panels, one set per transform point:
 * element (k = c, n = o) of point xi at u + xi panels ic NR, as pack_b lays
 * B out; 16 output channels a vector. */
static float *packed_weights(const float *w, int64_t oc, int64_t ic, int A, const float *gm, int threads) {
    const int64_t panels = cdiv(oc, NR), per = panels * ic * NR;
    float *u = (float *)kept(0, (size_t)(A * A * per) * sizeof(float));
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t pc = 0; pc < panels * ic; ++pc) {
        const int64_t p = pc / ic, c = pc % ic;
        for (int64_t j = 0; j < NR; j += 16) {
            v16 g[9], t[36];
            gather_kernels(w, oc, ic, p * NR + j, c, g);
            weight_vec(g, A, gm, t);
            for (int xi = 0; xi < A * A; ++xi) *(v16 *)(u + xi * per + (p * ic + c) * NR + j) = t[xi];
        }
    }
    return u;
}

/* The outputs of one tile, channels [o0, o0 + cnt): A^T m A + bias
 * (+ residual), m[xi][o] with stride ms between transform points; channels
 * innermost so that the arithmetic goes by vectors. */
static void output_tile(const float *m, int64_t ms, int A, int T, const float *at, int64_t o0, int64_t cnt,
                        int64_t oc, int64_t b, int64_t ty, int64_t tx, int64_t oh, int64_t ow, const float *bias,
                        const float *residual, float *y, float *am) {
    for (int i = 0; i < T; ++i)
        for (int j = 0; j < A; ++j) {
            float *dst = am + (i * A + j) * cnt;
            for (int64_t o = 0; o < cnt; ++o) dst[o] = 0.0f;
            for (int k = 0; k < A; ++k) {
                const float f = at[i * A + k];
                if (f == 0.0f) continue;
                const float *src = m + (k * A + j) * ms;
                for (int64_t o = 0; o < cnt; ++o) dst[o] += f * src[o];
            }
        }
    for (int i = 0; i < T; ++i) {
        const int64_t yy = ty * T + i;
        if (yy >= oh) continue;
        for (int jj = 0; jj < T; ++jj) {
            const int64_t xx = tx * T + jj;
            if (xx >= ow) continue;
            for (int64_t o = 0; o < cnt; ++o) {
                float s = 0.0f;
                for (int j = 0; j < A; ++j) s += am[(i * A + j) * cnt + o] * at[jj * A + j];
                const int64_t at_ = ((b * oc + o0 + o) * oh + yy) * ow + xx;
                if (bias) s += bias[o0 + o];
                if (residual) s += residual[at_];
                y[at_] = s;
            }
        }
    }
}

/* Rows [y0, y0 + rows) and columns [x0, x0 + cols) of every channel of one
 * image, zero outside it and for channels ic..icp, into buf[row][col][icp]
 * (channels last, icp a multiple of 16), 16 channels a gather. */
static void channels_last(const float *img, int64_t ic, int64_t ih, int64_t iw, int64_t y0, int64_t rows, int64_t x0,
                          int64_t cols, int64_t icp, float *buf) {
    const int64_t plane = ih * iw;
    const __m512i index = _mm512_mullo_epi32(_mm512_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15),
                                             _mm512_set1_epi32((int32_t)plane));
    for (int64_t c0 = 0; c0 < icp; c0 += 16) {
        const int64_t live = ic - c0;
        const __mmask16 mask = live >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << (live > 0 ? live : 0)) - 1u);
        for (int64_t i = 0; i < rows; ++i) {
            const int64_t yy = y0 + i;
            for (int64_t x = 0; x < cols; ++x) {
                const int64_t xx = x0 + x;
                __m512 val = _mm512_setzero_ps();
                if (yy >= 0 && yy < ih && xx >= 0 && xx < iw && mask)
                    val = _mm512_mask_i32gather_ps(val, mask, index, img + c0 * plane + yy * iw + xx, 4);
                _mm512_store_ps(buf + (i * cols + x) * icp + c0, val);
            }
        }
    }
}

/* The outputs of a strip of nt F(4x4) tiles (row of tiles ty, from tile
 * tx0): per tile A^T m A of 16 channels a vector, scattered into
 * obuf[o][4][4 nt] (channels first); then each channel's rows written whole
 * with the bias and the residual.  m[xi][l][o], points ms apart. */
static void output_strip4(const float *m, int64_t ms, int64_t nt, int64_t oc, int64_t b, int64_t ty, int64_t tx0,
                          int64_t oh, int64_t ow, const float *bias, const float *residual, float *y, float *obuf) {
    const int64_t W = 4 * nt;
    const __m512i index = _mm512_mullo_epi32(_mm512_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15),
                                             _mm512_set1_epi32((int32_t)(4 * W)));
    for (int64_t l = 0; l < nt; ++l)
        for (int64_t o0 = 0; o0 < oc; o0 += 16) {
            const int64_t live = oc - o0;
            const __mmask16 mask = live >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << live) - 1u);
            v16 mv[36], am[24];
            for (int xi = 0; xi < 36; ++xi) mv[xi] = (v16)_mm512_maskz_loadu_ps(mask, m + xi * ms + l * oc + o0);
#pragma GCC unroll 4
            for (int i = 0; i < 4; ++i)
#pragma GCC unroll 6
                for (int j = 0; j < 6; ++j) {
                    v16 acc = (v16){0};
#pragma GCC unroll 6
                    for (int k = 0; k < 6; ++k)
                        if (AT4[i][k] != 0.0f) acc += AT4[i][k] * mv[k * 6 + j];
                    am[i * 6 + j] = acc;
                }
#pragma GCC unroll 4
            for (int i = 0; i < 4; ++i)
#pragma GCC unroll 4
                for (int jj = 0; jj < 4; ++jj) {
                    v16 acc = (v16){0};
#pragma GCC unroll 6
                    for (int j = 0; j < 6; ++j)
                        if (AT4[jj][j] != 0.0f) acc += am[i * 6 + j] * AT4[jj][j];
                    _mm512_mask_i32scatter_ps(obuf + (o0 * 4 + i) * W + 4 * l + jj, mask, index, (__m512)acc, 4);
                }
        }
    const int64_t cnt = min64(W, ow - tx0 * 4);
    for (int64_t o = 0; o < oc; ++o)
        for (int64_t i = 0; i < 4; ++i) {
            const int64_t yy = ty * 4 + i;
            if (yy >= oh) continue;
            const int64_t at = ((b * oc + o) * oh + yy) * ow + tx0 * 4;
            const float *src = obuf + (o * 4 + i) * W;
            const float bo = bias ? bias[o] : 0.0f;
            float *dst = y + at;
            if (residual) {
                const float *res = residual + at;
                for (int64_t x = 0; x < cnt; ++x) dst[x] = src[x] + bo + res[x];
            } else {
                for (int64_t x = 0; x < cnt; ++x) dst[x] = src[x] + bo;
            }
        }
}

enum { TS = 16 };  /* tiles of a strip: a block of the F(4x4) port */

/* The large-image F(4x4, 3x3) of winograd.cc:1548-1613: the weights
 * transformed once into packed panels; then per (image, strip of TS tiles
 * along a row of tiles) a thread lays the strip's input rows out channels
 * last, transforms them 16 channels a vector into V[xi][tile][icp], makes the
 * 36 products V_xi U_xi with the packed kernel, and transforms them into the
 * outputs with the bias and the residual (the chain of configs[1]).
 * x [n][ic][ih][iw], w [oc][ic][3][3] widened, y [n][oc][oh][ow]. */
void oracle_port_winograd4(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w, int64_t oc,
                           int p0, int p1, const float *bias, const float *residual, float *y, int threads) {
    const int64_t oh = ih + 2 * p1 - 2, ow = iw + 2 * p0 - 2;
    const int64_t tw = cdiv(ow, 4), th = cdiv(oh, 4), icp = cdiv(ic, 16) * 16;
    const int64_t panels = cdiv(oc, NR), per = panels * ic * NR, strips = cdiv(tw, TS);
    float *u = packed_weights(w, oc, ic, 6, &G4[0][0], threads);
#pragma omp parallel num_threads(threads)
    {
        const int64_t wmax = 4 * TS + 2;
        float *buf = (float *)kept_local(0, (size_t)(6 * wmax * icp) * sizeof(float));
        float *v = (float *)kept_local(1, (size_t)(36 * TS * icp) * sizeof(float));
        float *m = (float *)kept_local(2, (size_t)(36 * TS * oc) * sizeof(float));
        float *obuf = (float *)kept_local(3, (size_t)(16 * TS * (oc + 16)) * sizeof(float));
        float *ab = (float *)kept_local(4, MC * KC * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (int64_t item = 0; item < n * th * strips; ++item) {
            const int64_t b = item / (th * strips), ty = (item / strips) % th, tx0 = (item % strips) * TS;
            const int64_t nt = min64(TS, tw - tx0), cols = 4 * nt + 2;
            channels_last(x + b * ic * ih * iw, ic, ih, iw, ty * 4 - p1, 6, tx0 * 4 - p0, cols, icp, buf);
            for (int64_t l = 0; l < nt; ++l)
                for (int64_t c0 = 0; c0 < icp; c0 += 16) {
                    v16 d[36], t[36];
                    for (int i = 0; i < 6; ++i)
                        for (int j = 0; j < 6; ++j)
                            d[i * 6 + j] = *(const v16 *)(buf + (i * cols + 4 * l + j) * icp + c0);
                    input_vec(d, 6, &BT4[0][0], t);
                    for (int xi = 0; xi < 36; ++xi) *(v16 *)(v + (xi * TS + l) * icp + c0) = t[xi];
                }
            for (int xi = 0; xi < 36; ++xi)
                gemm1(nt, oc, ic, v + xi * TS * icp, icp, 1, u + xi * per, 0, panels, m + xi * TS * oc, oc, 0, ab);
            output_strip4(m, TS * oc, nt, oc, b, ty, tx0, oh, ow, bias, residual, y, obuf);
        }
    }
}

/* ------------------------------------------------------------ Winograd F(2x2, 3x3) */

/* F(2x2, 3x3) (winograd.cc's small-image form, 2107-2123): the inputs of all
 * tiles transformed once, 16 channels a vector, into V[xi][tile][icp]; then
 * per (panel of NR output channels, stretch of input channels, block of
 * tiles) a thread transforms its weights (16 output channels a vector) into
 * packed panels a KC of channels at a time and makes the 16 products,
 * partial over its stretch; the stretches' partial products are summed in
 * the output transform, with the bias (and the residual). */
void oracle_port_winograd2(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w, int64_t oc,
                           int p0, int p1, const float *bias, const float *residual, float *y, int threads) {
    const int64_t oh = ih + 2 * p1 - 2, ow = iw + 2 * p0 - 2;
    const int64_t tw = cdiv(ow, 2), th = cdiv(oh, 2), per_image = tw * th, T = n * per_image;
    const int64_t panels = cdiv(oc, NR), icp = cdiv(ic, 16) * 16;
    const int64_t tb = min64(T, 96), tblocks = cdiv(T, tb);
    int64_t splits = ic / 256;
    splits = splits < 1 ? 1 : splits > 4 ? 4 : splits;
    const int64_t stretch = cdiv(cdiv(ic, splits), KC) * KC;
    splits = cdiv(ic, stretch);
    float *v = (float *)kept(0, (size_t)(16 * T * icp) * sizeof(float));
    /* the inputs, a row of tiles at a time, laid out channels last */
#pragma omp parallel num_threads(threads)
    {
        const int64_t cols = 2 * tw + 2;
        float *buf = (float *)kept_local(0, (size_t)(4 * cols * icp) * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (int64_t row = 0; row < n * th; ++row) {
            const int64_t b = row / th, ty = row % th;
            channels_last(x + b * ic * ih * iw, ic, ih, iw, ty * 2 - p1, 4, -p0, cols, icp, buf);
            for (int64_t tx = 0; tx < tw; ++tx)
                for (int64_t c0 = 0; c0 < icp; c0 += 16) {
                    v16 d[16], t[16];
                    for (int i = 0; i < 4; ++i)
                        for (int j = 0; j < 4; ++j)
                            d[i * 4 + j] = *(const v16 *)(buf + (i * cols + 2 * tx + j) * icp + c0);
                    input_vec(d, 4, &BT2[0][0], t);
                    const int64_t tile = b * per_image + ty * tw + tx;
                    for (int xi = 0; xi < 16; ++xi) *(v16 *)(v + (xi * T + tile) * icp + c0) = t[xi];
                }
        }
    }
    /* partial products [split][xi][tile][panels * NR] */
    const int64_t ldm = panels * NR;
    float *m = (float *)kept(1, (size_t)(splits * 16 * T * ldm) * sizeof(float));
    const int64_t items = panels * splits * tblocks;
#pragma omp parallel num_threads(threads)
    {
        float *u = (float *)kept_local(1, (size_t)(16 * KC * NR) * sizeof(float));
        float *ab = (float *)kept_local(2, MC * KC * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (int64_t item = 0; item < items; ++item) {
            const int64_t p = item % panels, s = (item / panels) % splits, tbk = item / (panels * splits);
            const int64_t c_begin = s * stretch, c_end = min64(ic, c_begin + stretch);
            const int64_t t0 = tbk * tb, nt = min64(tb, T - t0);
            for (int64_t c0 = c_begin; c0 < c_end; c0 += KC) {
                const int64_t kc = min64(KC, c_end - c0);
                for (int64_t c = 0; c < kc; ++c)
                    for (int64_t j = 0; j < NR; j += 16) {
                        v16 g[9], t[16];
                        gather_kernels(w, oc, ic, p * NR + j, c0 + c, g);
                        weight_vec(g, 4, &G2[0][0], t);
                        for (int xi = 0; xi < 16; ++xi) *(v16 *)(u + (xi * kc + c) * NR + j) = t[xi];
                    }
                for (int xi = 0; xi < 16; ++xi)
                    gemm1(nt, NR, kc, v + (xi * T + t0) * icp + c0, icp, 1, u + xi * kc * NR, 0, 1,
                          m + ((s * 16 + xi) * T + t0) * ldm + p * NR, ldm, c0 > c_begin, ab);
            }
        }
    }
    /* the stretches summed into the first, then A^T m A */
#pragma omp parallel num_threads(threads)
    {
        float *am = (float *)kept_local(3, (size_t)(8 * NR) * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (int64_t item = 0; item < T * panels; ++item) {
            const int64_t t = item / panels, p = item % panels;
            const int64_t o0 = p * NR, cnt = min64(NR, oc - o0);
            for (int64_t s = 1; s < splits; ++s)
                for (int xi = 0; xi < 16; ++xi) {
                    float *dst = m + (xi * T + t) * ldm + o0;
                    const float *src = m + ((s * 16 + xi) * T + t) * ldm + o0;
                    for (int64_t o = 0; o < cnt; ++o) dst[o] += src[o];
                }
            const int64_t b = t / per_image, l = t % per_image;
            output_tile(m + t * ldm + o0, T * ldm, 4, 2, &AT2[0][0], o0, cnt, oc, b, l / tw, l % tw, oh, ow, bias,
                        residual, y, am);
        }
    }
}

/* ------------------------------------------------------------ norms */

/* GROUP_NORM (norm.cc:100-140: the mean, then the mean square of the centred
 * values, both summed in double) with the affine step and SiLU after it, per
 * (image, group) on a thread.  x, y [n][c][hw]. */
void oracle_port_group_norm(const float *x, float *y, int64_t n, int64_t c, int64_t hw, int groups, float eps,
                            const float *gamma, const float *beta, int silu, int threads) {
    const int64_t cg = c / groups;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t item = 0; item < n * groups; ++item) {
        const int64_t len = cg * hw;
        const float *src = x + item * len;
        float *dst = y + item * len;
        double sum = 0.0;
        for (int64_t e = 0; e < len; ++e) sum += src[e];
        const float mean = (float)(sum / (double)len);
        double sq = 0.0;
        for (int64_t e = 0; e < len; ++e) {
            const float d = src[e] - mean;
            sq += (double)(d * d);
        }
        const float inv = 1.0f / sqrtf((float)(sq / (double)len) + eps);
        for (int64_t ch = 0; ch < cg; ++ch) {
            const int64_t channel = (item % groups) * cg + ch;
            const float g = gamma ? gamma[channel] : 1.0f, bb = beta ? beta[channel] : 0.0f;
            for (int64_t e = 0; e < hw; ++e) {
                float v = (src[ch * hw + e] - mean) * inv * g + bb;
                if (silu) v = v / (1.0f + expf(-v));
                dst[ch * hw + e] = v;
            }
        }
    }
}

/* NORM over rows of `len` (norm.cc:148-175) with the affine step. */
void oracle_port_norm(const float *x, float *y, int64_t rows, int64_t len, float eps, const float *gamma,
                      const float *beta, int threads) {
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float *src = x + r * len;
        float *dst = y + r * len;
        double sum = 0.0;
        for (int64_t e = 0; e < len; ++e) sum += src[e];
        const float mean = (float)(sum / (double)len);
        double sq = 0.0;
        for (int64_t e = 0; e < len; ++e) {
            const float d = src[e] - mean;
            sq += (double)(d * d);
        }
        const float inv = 1.0f / sqrtf((float)(sq / (double)len) + eps);
        for (int64_t e = 0; e < len; ++e)
            dst[e] = (src[e] - mean) * inv * (gamma ? gamma[e] : 1.0f) + (beta ? beta[e] : 0.0f);
    }
}

/* ------------------------------------------------------------ attention */

/* e^x of 16 numbers: x = n ln2 + r, |r| <= ln2 / 2 (ln 2 split in two parts
 * so that n ln2 is exact), e^r by its Taylor polynomial to r^7 (relative
 * error below 2e-8 on that range), 2^n by the exponent bits. */
static inline v16 exp16(v16 x) {
    x = (v16)_mm512_min_ps(_mm512_max_ps((__m512)x, _mm512_set1_ps(-87.0f)), _mm512_set1_ps(88.0f));
    const v16 nf = (v16)_mm512_roundscale_ps((__m512)(x * 1.44269504088896341f), _MM_FROUND_TO_NEAREST_INT);
    v16 r = x - nf * 0.693145751953125f;
    r = r - nf * 1.428606765330187e-06f;
    v16 p = (v16){0} + (1.0f / 5040);
    p = p * r + (1.0f / 720);
    p = p * r + (1.0f / 120);
    p = p * r + (1.0f / 24);
    p = p * r + (1.0f / 6);
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    const i16v bits = (__builtin_convertvector(nf, i16v) + 127) << 23;
    return p * (v16)bits;
}

enum { QB = 48 };  /* queries of a block */

/* FLASH_ATTN_EXT in single precision (attention.cc, without a mask): per
 * (image, head) the keys packed as the columns of K^T and the values as B
 * panels; per block of QB queries S = Q K^T by the packed kernel, the
 * softmax (the row's maximum, e^(scale s - max), the sum in double), O = P V
 * by the packed kernel, divided by the sum.  q [b][lq][h][d], k [b][lk][h][d],
 * v [b][lk][h][dv], y [b][lq][h][dv]. */
void oracle_port_attention(const float *q, const float *k, const float *v, int64_t b, int64_t lq, int64_t lk,
                           int64_t h, int64_t d, int64_t dv, float scale, float *y, int threads) {
    const size_t kp_per = packed_b_floats(d, lk), vp_per = packed_b_floats(lk, dv);
    float *kp = (float *)kept(0, (size_t)(b * h) * kp_per * sizeof(float));
    float *vp = (float *)kept(1, (size_t)(b * h) * vp_per * sizeof(float));
    const int64_t kpanels = cdiv(lk, NR), vpanels = cdiv(dv, NR);
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t item = 0; item < b * h * (kpanels + vpanels); ++item) {
        const int64_t bh = item / (kpanels + vpanels), p = item % (kpanels + vpanels);
        const int64_t bi = bh / h, hh = bh % h;
        if (p < kpanels)
            pack_b(k + (bi * lk * h + hh) * d, 1, h * d, d, lk, p, p + 1, kp + bh * kp_per);
        else
            pack_b(v + (bi * lk * h + hh) * dv, h * dv, 1, lk, dv, p - kpanels, p - kpanels + 1, vp + bh * vp_per);
    }
    const int64_t qblocks = cdiv(lq, QB);
    const int64_t lks = cdiv(lk, 16) * 16;
#pragma omp parallel num_threads(threads)
    {
        float *s = (float *)kept_local(0, (size_t)(QB * lks) * sizeof(float));
        float *o = (float *)kept_local(1, (size_t)(QB * dv) * sizeof(float));
        float *ab = (float *)kept_local(2, MC * KC * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (int64_t item = 0; item < b * h * qblocks; ++item) {
            const int64_t bh = item / qblocks, q0 = (item % qblocks) * QB;
            const int64_t bi = bh / h, hh = bh % h, rows = min64(QB, lq - q0);
            const float *qb = q + ((bi * lq + q0) * h + hh) * d;
            gemm1(rows, lk, d, qb, h * d, 1, kp + bh * kp_per, 0, kpanels, s, lks, 0, ab);
            double sums[QB];
            for (int64_t r = 0; r < rows; ++r) {
                float *row = s + r * lks;
                for (int64_t e = lk; e < lks; ++e) row[e] = -INFINITY;
                __m512 mv = _mm512_set1_ps(-INFINITY);
                for (int64_t e = 0; e < lks; e += 16) mv = _mm512_max_ps(mv, _mm512_loadu_ps(row + e));
                const float mx = _mm512_reduce_max_ps(mv);
                const float m = mx * scale;
                __m512d sum0 = _mm512_setzero_pd(), sum1 = _mm512_setzero_pd();
                for (int64_t e = 0; e < lks; e += 16) {
                    const __mmask16 live = lk - e >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << (lk - e)) - 1u);
                    v16 z;
                    memcpy(&z, row + e, sizeof z);
                    z = (v16)_mm512_maskz_mov_ps(live, (__m512)exp16(z * scale - m));
                    memcpy(row + e, &z, sizeof z);
                    /* the sum in double, in 16 running parts */
                    sum0 = _mm512_add_pd(sum0, _mm512_cvtps_pd(_mm512_castps512_ps256((__m512)z)));
                    sum1 = _mm512_add_pd(sum1, _mm512_cvtps_pd(_mm256_castpd_ps(_mm512_extractf64x4_pd(_mm512_castps_pd((__m512)z), 1))));
                }
                sums[r] = _mm512_reduce_add_pd(_mm512_add_pd(sum0, sum1));
            }
            gemm_rows(rows, dv, lk, s, lks, vp + bh * vp_per, o, dv);
            for (int64_t r = 0; r < rows; ++r) {
                const float inv = (float)(1.0 / sums[r]);
                float *dst = y + ((bi * lq + q0 + r) * h + hh) * dv;
                for (int64_t e = 0; e < dv; ++e) dst[e] = o[r * dv + e] * inv;
            }
        }
    }
}

/* ------------------------------------------------------------ the bits mode */

enum { QR = 6, QN = 32 };  /* the integer kernel's rows and columns */

/* The quantized weights (oracle_quantize_weights' [n][groups * group] bytes,
 * scales and offsets [n][groups]) packed for the integer kernel: panels of QN
 * columns, each a [k / 4][QN][4] run of bytes, and the scales and offsets as
 * [panel][group][QN].  The reference keeps its quantized layouts from one
 * call to the next (store.cc:64-99); so do the callers of this. */
size_t oracle_port_qweights_bytes(int64_t N, int64_t groups, int64_t group) {
    const int64_t panels = cdiv(N, QN);
    return (size_t)(panels * groups * group * QN) + 2 * (size_t)(panels * groups * QN) * sizeof(float);
}

void oracle_port_pack_qweights(const int8_t *wq, const float *ws, const float *wo, int64_t N, int64_t groups,
                               int64_t group, void *packed) {
    const int64_t kp = groups * group, panels = cdiv(N, QN);
    int8_t *bq = (int8_t *)packed;
    float *sb = (float *)(bq + panels * kp * QN);
    float *ob = sb + panels * groups * QN;
    for (int64_t p = 0; p < panels; ++p)
        for (int64_t j = 0; j < QN; ++j) {
            const int64_t n = p * QN + j;
            for (int64_t k = 0; k < kp; ++k)
                bq[((p * (kp / 4) + k / 4) * QN + j) * 4 + k % 4] = n < N ? wq[n * kp + k] : 0;
            for (int64_t g = 0; g < groups; ++g) {
                sb[(p * groups + g) * QN + j] = n < N ? ws[n * groups + g] : 0.0f;
                ob[(p * groups + g) * QN + j] = n < N ? wo[n * groups + g] : 0.0f;
            }
        }
}

/* A row's group of inputs quantized unsigned with a zero point, as
 * quant.cc:282-315 quantizes them (oracle_quantize_input_row's steps). */
static void quantize_group(const float *x, int64_t cnt, int64_t group, int levels, uint8_t *dst, float *scale,
                           float *offset) {
    float least = 0.0f, greatest = 0.0f;
    for (int64_t e = 0; e < cnt; ++e) {
        least = fminf(least, x[e]);
        greatest = fmaxf(greatest, x[e]);
    }
    const float s = (greatest - least) / (float)levels;
    const float inverse = s > 0.0f ? 1.0f / s : 0.0f;
    const float zero = nearbyintf(-least * inverse);
    const float top = (float)levels;
    for (int64_t e = 0; e < cnt; ++e) {
        float qv = nearbyintf(x[e] * inverse) + zero;
        qv = qv < 0.0f ? 0.0f : qv > top ? top : qv;
        dst[e] = (uint8_t)qv;
    }
    for (int64_t e = cnt; e < group; ++e) dst[e] = (uint8_t)zero;
    *scale = s;
    *offset = s * zero;
}

/* quantize_group 16 numbers a vector: the least and greatest with 0 between
 * them, the scale and its inverse, each byte rint(x inverse) + zero clamped
 * to [0, levels] (round to nearest even, as nearbyintf), the tail the zero
 * point. */
static void quantize16(const float *x, int64_t cnt, int64_t group, int levels, uint8_t *dst, float *scale,
                       float *offset) {
    __m512 lo = _mm512_setzero_ps(), hi = _mm512_setzero_ps();
    for (int64_t e = 0; e < cnt; e += 16) {
        const __mmask16 live = cnt - e >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << (cnt - e)) - 1u);
        const __m512 v = _mm512_maskz_loadu_ps(live, x + e);
        lo = _mm512_min_ps(lo, v);
        hi = _mm512_max_ps(hi, v);
    }
    const float least = _mm512_reduce_min_ps(lo), greatest = _mm512_reduce_max_ps(hi);
    const float s = (greatest - least) / (float)levels;
    const float inverse = s > 0.0f ? 1.0f / s : 0.0f;
    const float zero = nearbyintf(-least * inverse);
    const __m512 inv = _mm512_set1_ps(inverse), z = _mm512_set1_ps(zero), top = _mm512_set1_ps((float)levels);
    for (int64_t e = 0; e < group; e += 16) {
        const __mmask16 live = cnt - e >= 16 ? (__mmask16)0xffff
                               : cnt > e     ? (__mmask16)((1u << (cnt - e)) - 1u)
                                             : (__mmask16)0;
        const __m512 v = _mm512_maskz_loadu_ps(live, x + e);
        __m512 qv = _mm512_add_ps(_mm512_roundscale_ps(_mm512_mul_ps(v, inv), _MM_FROUND_TO_NEAREST_INT), z);
        qv = _mm512_min_ps(_mm512_max_ps(qv, _mm512_setzero_ps()), top);
        qv = _mm512_mask_mov_ps(z, live, qv);
        const __mmask16 keep = group - e >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << (group - e)) - 1u);
        _mm_mask_storeu_epi8(dst + e, keep, _mm512_cvtusepi32_epi8(_mm512_cvtps_epu32(qv)));
    }
    *scale = s;
    *offset = s * zero;
}

/* One QR x QN tile of the quantized product: per group the exact integer sum
 * S (AVX512-VNNI, unsigned inputs by signed weights), then t = fma(sa sb, S,
 * t), t = fma(-oa, ob, t) in the order of quant.cc:113-164. */
static void qmicro(const uint8_t *xq, int64_t kp, const float *sa, const float *oa, int64_t groups, int64_t group,
                   const int8_t *bq, const float *sb, const float *ob, int64_t rows, int64_t cols, float *y,
                   int64_t ldy) {
    __m512 t[QR][2];
    for (int i = 0; i < QR; ++i) t[i][0] = t[i][1] = _mm512_setzero_ps();
    for (int64_t g = 0; g < groups; ++g) {
        __m512i acc[QR][2];
        for (int i = 0; i < QR; ++i) acc[i][0] = acc[i][1] = _mm512_setzero_si512();
        for (int64_t k4 = 0; k4 < group / 4; ++k4) {
            const int8_t *bk = bq + ((g * group / 4 + k4) * QN) * 4;
            const __m512i b0 = _mm512_loadu_si512((const void *)bk);
            const __m512i b1 = _mm512_loadu_si512((const void *)(bk + 64));
#pragma GCC unroll 6
            for (int i = 0; i < QR; ++i) {
                int32_t four;
                memcpy(&four, xq + (i < rows ? i : 0) * kp + g * group + 4 * k4, 4);
                const __m512i a = _mm512_set1_epi32(four);
                acc[i][0] = _mm512_dpbusd_epi32(acc[i][0], a, b0);
                acc[i][1] = _mm512_dpbusd_epi32(acc[i][1], a, b1);
            }
        }
        const __m512 sb0 = _mm512_loadu_ps(sb + g * QN), sb1 = _mm512_loadu_ps(sb + g * QN + 16);
        const __m512 ob0 = _mm512_loadu_ps(ob + g * QN), ob1 = _mm512_loadu_ps(ob + g * QN + 16);
#pragma GCC unroll 6
        for (int i = 0; i < QR; ++i) {
            const int64_t r = i < rows ? i : 0;
            const __m512 a = _mm512_set1_ps(sa[r * groups + g]);
            const __m512 o = _mm512_set1_ps(-oa[r * groups + g]);
            t[i][0] = _mm512_fmadd_ps(_mm512_mul_ps(a, sb0), _mm512_cvtepi32_ps(acc[i][0]), t[i][0]);
            t[i][1] = _mm512_fmadd_ps(_mm512_mul_ps(a, sb1), _mm512_cvtepi32_ps(acc[i][1]), t[i][1]);
            t[i][0] = _mm512_fmadd_ps(o, ob0, t[i][0]);
            t[i][1] = _mm512_fmadd_ps(o, ob1, t[i][1]);
        }
    }
    float out[QR][QN] __attribute__((aligned(64)));
    for (int i = 0; i < QR; ++i) {
        _mm512_store_ps(&out[i][0], t[i][0]);
        _mm512_store_ps(&out[i][16], t[i][1]);
    }
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t j = 0; j < cols; ++j) y[i * ldy + j] = out[i][j];
}

/* The bits mode's MUL_MAT (mul_mat.cc:498-569): the inputs quantized per
 * (row, group), the product with weights packed by oracle_port_pack_qweights,
 * y[m][n] = the quantized sum (+ bias[n]).  With `gated`, N is two halves and
 * out[m][j] = y[m][j] GELU(y[m][N / 2 + j]) (y then the caller's scratch of
 * M x N).  x [M][K]; levels as the oracle's (255 for 8 bits). */
void oracle_port_quantized_linear(const float *x, int64_t M, int64_t K, const void *packed, int64_t N, int64_t group,
                                  int levels, const float *bias, float *y, int gated, float *out, int threads) {
    const int64_t groups = cdiv(K, group), kp = groups * group, panels = cdiv(N, QN);
    const int8_t *bq = (const int8_t *)packed;
    const float *sb = (const float *)(bq + panels * kp * QN);
    const float *ob = sb + panels * groups * QN;
    uint8_t *xq = (uint8_t *)kept(0, (size_t)(M * kp));
    float *sa = (float *)kept(1, (size_t)(M * groups) * sizeof(float));
    float *oa = (float *)kept(2, (size_t)(M * groups) * sizeof(float));
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t g = 0; g < groups; ++g)
            quantize_group(x + m * K + g * group, min64(group, K - g * group), group, levels, xq + m * kp + g * group,
                           &sa[m * groups + g], &oa[m * groups + g]);
    const int64_t rb = cdiv(M, 4 * QR);
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t item = 0; item < rb * panels; ++item) {
        const int64_t p = item % panels, m0 = (item / panels) * 4 * QR;
        const int64_t cols = min64(QN, N - p * QN);
        for (int64_t i = m0; i < min64(M, m0 + 4 * QR); i += QR) {
            const int64_t rows = min64(QR, M - i);
            qmicro(xq + i * kp, kp, sa + i * groups, oa + i * groups, groups, group, bq + p * kp * QN,
                   sb + p * groups * QN, ob + p * groups * QN, rows, cols, y + i * N + p * QN, N);
        }
    }
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        float *row = y + m * N;
        if (bias)
            for (int64_t n = 0; n < N; ++n) row[n] += bias[n];
    }
    if (gated) oracle_port_gated(y, M, N, out, threads);
}

/* The bits mode's self-attention (attention.cc:612-824) on AVX512-VNNI, in
 * the reference's algorithm: per (image, key head) the keys quantized signed,
 * one group over the head's dimensions, packed [key tile of 16][gd / 4][16][4];
 * the values signed per (dimension, group of `group` keys), packed per group
 * [dim panel of 16][group / 4][16][4]; per query its bytes unsigned with a
 * zero point over the dimensions, the softmax's scale folded into its scale
 * and offset (754-764); its scores, the integer sums of 16 keys a vector
 * (vpdpbusd), scaled back as quant.cc:150-155 does; their maximum; then per
 * stretch of key_block keys the exponentials (the polynomial of exp16 for the
 * stretch's multiples of 8 keys, expf for the rest), summed in double, and per
 * group of keys quantized unsigned with a zero point, their product with the
 * values 16 dimensions a vector, dequantised in the reference's order; the
 * output times float(1 / sum).  q [b][lq][h][d], k [b][lk][hk][d],
 * v [b][lk][hk][dv], y [b][lq][h][dv]. */
void oracle_port_quantized_attention(const float *q, const float *k, const float *v, int64_t b, int64_t lq,
                                     int64_t lk, int64_t h, int64_t hk, int64_t d, int64_t dv, float scale,
                                     int64_t group, int levels, int wmax, int64_t key_block, float *y, int threads) {
    const int64_t gd = cdiv(d, 4) * 4, lkt = cdiv(lk, 16), groups = cdiv(lk, group), dvt = cdiv(dv, 16);
    const int64_t heads = b * hk;
    const size_t kbytes = (size_t)(lkt * gd * 16), vbytes = (size_t)(groups * dvt * group * 16);
    int8_t *kq = (int8_t *)kept(0, (size_t)heads * kbytes);
    float *ks = (float *)kept(1, (size_t)(heads * lkt * 16) * sizeof(float));
    float *ko = (float *)kept(2, (size_t)(heads * lkt * 16) * sizeof(float));
    int8_t *vq = (int8_t *)kept(3, (size_t)heads * vbytes);
    float *vs = (float *)kept(4, (size_t)(heads * groups * dvt * 16) * sizeof(float));
    float *vo = (float *)kept(5, (size_t)(heads * groups * dvt * 16) * sizeof(float));
    const float wm = (float)wmax;
    /* The keys and the values of each head, quantized and packed. */
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t item = 0; item < heads * (lkt + groups * dvt); ++item) {
        const int64_t head = item / (lkt + groups * dvt), u = item % (lkt + groups * dvt);
        const int64_t bi = head / hk, kh = head % hk;
        if (u < lkt) {
            for (int64_t jj = 0; jj < 16; ++jj) {
                const int64_t j = u * 16 + jj;
                const float *row = k + ((bi * lk + (j < lk ? j : 0)) * hk + kh) * d;
                float m = 0.0f;
                if (j < lk)
                    for (int64_t e = 0; e < d; ++e) m = fmaxf(m, fabsf(row[e]));
                const float sc = m / wm, inv = sc > 0.0f ? 1.0f / sc : 0.0f;
                int32_t sum = 0;
                for (int64_t e = 0; e < gd; ++e) {
                    float qv = j < lk && e < d ? nearbyintf(row[e] * inv) : 0.0f;
                    qv = qv < -wm ? -wm : qv > wm ? wm : qv;
                    kq[(size_t)head * kbytes + ((u * (gd / 4) + e / 4) * 16 + jj) * 4 + e % 4] = (int8_t)qv;
                    sum += (int32_t)qv;
                }
                ks[head * lkt * 16 + j] = sc;
                ko[head * lkt * 16 + j] = sc * (float)sum;
            }
        } else {
            const int64_t g = (u - lkt) / dvt, pnl = (u - lkt) % dvt;
            for (int64_t cc = 0; cc < 16; ++cc) {
                const int64_t c = pnl * 16 + cc;
                float m = 0.0f;
                for (int64_t w = 0; w < group && c < dv; ++w) {
                    const int64_t j = g * group + w;
                    if (j < lk) m = fmaxf(m, fabsf(v[((bi * lk + j) * hk + kh) * dv + c]));
                }
                const float sc = m / wm, inv = sc > 0.0f ? 1.0f / sc : 0.0f;
                int32_t sum = 0;
                int8_t *dst = vq + (size_t)head * vbytes + (size_t)((g * dvt + pnl) * group * 16);
                for (int64_t w = 0; w < group; ++w) {
                    const int64_t j = g * group + w;
                    float qv = c < dv && j < lk ? nearbyintf(v[((bi * lk + j) * hk + kh) * dv + c] * inv) : 0.0f;
                    qv = qv < -wm ? -wm : qv > wm ? wm : qv;
                    dst[((w / 4) * 16 + cc) * 4 + w % 4] = (int8_t)qv;
                    sum += (int32_t)qv;
                }
                vs[((head * groups + g) * dvt + pnl) * 16 + cc] = sc;
                vo[((head * groups + g) * dvt + pnl) * 16 + cc] = sc * (float)sum;
            }
        }
    }
    enum { AQ = 4 };  /* queries a thread takes at once: each key and value load serves all of them */
    const int64_t qblocks = cdiv(lq, AQ);
#pragma omp parallel num_threads(threads)
    {
        float *sc = (float *)kept_local(0, (size_t)(AQ * lkt * 16) * sizeof(float));
        uint8_t *qq = (uint8_t *)kept_local(1, (size_t)(AQ * gd));
        uint8_t *eq = (uint8_t *)kept_local(2, (size_t)(AQ * group));
        float *t = (float *)kept_local(3, (size_t)(AQ * dvt * 16) * sizeof(float));
#pragma omp for schedule(dynamic, 2)
        for (int64_t item = 0; item < b * h * qblocks; ++item) {
            const int64_t i0 = (item % qblocks) * AQ, bh = item / qblocks, bi = bh / h, hh = bh % h;
            const int64_t rows = min64(AQ, lq - i0);
            const int64_t head = bi * hk + hh / (h / hk);
            float qs[AQ], qo[AQ], mx[AQ];
            double total[AQ];
            for (int r = 0; r < AQ; ++r) {
                const int64_t i = i0 + (r < rows ? r : 0);
                quantize16(q + ((bi * lq + i) * h + hh) * d, d, gd, levels, qq + r * gd, &qs[r], &qo[r]);
                qs[r] *= scale;
                qo[r] *= scale;
            }
            /* The scores, 16 keys a vector, AQ queries a key load. */
            const int8_t *kh_q = kq + (size_t)head * kbytes;
            __m512 top[AQ];
            for (int r = 0; r < AQ; ++r) top[r] = _mm512_set1_ps(-INFINITY);
            for (int64_t u = 0; u < lkt; ++u) {
                __m512i acc[AQ];
                for (int r = 0; r < AQ; ++r) acc[r] = _mm512_setzero_si512();
                for (int64_t e4 = 0; e4 < gd / 4; ++e4) {
                    const __m512i kv = _mm512_loadu_si512((const void *)(kh_q + (u * (gd / 4) + e4) * 64));
                    for (int r = 0; r < AQ; ++r) {
                        int32_t four;
                        memcpy(&four, qq + r * gd + 4 * e4, 4);
                        acc[r] = _mm512_dpbusd_epi32(acc[r], _mm512_set1_epi32(four), kv);
                    }
                }
                const __m512 s4 = _mm512_loadu_ps(ks + head * lkt * 16 + u * 16);
                const __m512 o4 = _mm512_sub_ps(_mm512_setzero_ps(), _mm512_loadu_ps(ko + head * lkt * 16 + u * 16));
                const __mmask16 live = lk - u * 16 >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << (lk - u * 16)) - 1u);
                for (int r = 0; r < AQ; ++r) {
                    __m512 x = _mm512_fmadd_ps(_mm512_mul_ps(s4, _mm512_set1_ps(qs[r])), _mm512_cvtepi32_ps(acc[r]),
                                               _mm512_setzero_ps());
                    x = _mm512_fmadd_ps(o4, _mm512_set1_ps(qo[r]), x);
                    _mm512_storeu_ps(sc + r * lkt * 16 + u * 16, x);
                    top[r] = _mm512_mask_max_ps(top[r], live, top[r], x);
                }
            }
            for (int r = 0; r < AQ; ++r) {
                mx[r] = _mm512_reduce_max_ps(top[r]);
                total[r] = 0.0;
            }
            for (int64_t c = 0; c < AQ * dvt * 16; ++c) t[c] = 0.0f;
            for (int64_t j0 = 0; j0 < lk; j0 += key_block) {
                const int64_t j1 = min64(j0 + key_block, lk), whole = j0 + (j1 - j0) / 8 * 8;
                for (int r = 0; r < AQ; ++r) {
                    float *row = sc + r * lkt * 16;
                    __m512d sum0 = _mm512_setzero_pd(), sum1 = _mm512_setzero_pd();
                    int64_t j = j0;
                    for (; j < whole; j += 16) {
                        /* the polynomial for the stretch's multiples of 8 keys */
                        const __mmask16 live = whole - j >= 16 ? (__mmask16)0xffff
                                                               : (__mmask16)((1u << (whole - j)) - 1u);
                        v16 z = (v16)_mm512_maskz_loadu_ps(live, row + j);
                        z = (v16)_mm512_maskz_mov_ps(live, (__m512)exp16(z - mx[r]));
                        _mm512_mask_storeu_ps(row + j, live, (__m512)z);
                        sum0 = _mm512_add_pd(sum0, _mm512_cvtps_pd(_mm512_castps512_ps256((__m512)z)));
                        sum1 = _mm512_add_pd(sum1, _mm512_cvtps_pd(_mm256_castpd_ps(
                                                       _mm512_extractf64x4_pd(_mm512_castps_pd((__m512)z), 1))));
                    }
                    double tail = 0.0;
                    for (j = whole; j < j1; ++j) {
                        row[j] = expf(row[j] - mx[r]);
                        tail += (double)row[j];
                    }
                    total[r] += _mm512_reduce_add_pd(_mm512_add_pd(sum0, sum1)) + tail;
                }
                for (int64_t g0 = j0; g0 < j1; g0 += group) {
                    float es[AQ], eo[AQ];
                    for (int r = 0; r < AQ; ++r)
                        quantize16(sc + r * lkt * 16 + g0, min64(group, j1 - g0), group, levels, eq + r * group, &es[r],
                                   &eo[r]);
                    const int64_t g = g0 / group;
                    const int8_t *vg = vq + (size_t)head * vbytes + (size_t)(g * dvt * group * 16);
                    for (int64_t pnl = 0; pnl < dvt; ++pnl) {
                        __m512i acc[AQ];
                        for (int r = 0; r < AQ; ++r) acc[r] = _mm512_setzero_si512();
                        const int8_t *vp = vg + pnl * group * 16;
                        for (int64_t w4 = 0; w4 < group / 4; ++w4) {
                            const __m512i vv = _mm512_loadu_si512((const void *)(vp + w4 * 64));
                            for (int r = 0; r < AQ; ++r) {
                                int32_t four;
                                memcpy(&four, eq + r * group + 4 * w4, 4);
                                acc[r] = _mm512_dpbusd_epi32(acc[r], _mm512_set1_epi32(four), vv);
                            }
                        }
                        const __m512 vs4 = _mm512_loadu_ps(vs + ((head * groups + g) * dvt + pnl) * 16);
                        const __m512 vo4 =
                            _mm512_sub_ps(_mm512_setzero_ps(), _mm512_loadu_ps(vo + ((head * groups + g) * dvt + pnl) * 16));
                        for (int r = 0; r < AQ; ++r) {
                            float *tr = t + (r * dvt + pnl) * 16;
                            __m512 tt = _mm512_loadu_ps(tr);
                            tt = _mm512_fmadd_ps(_mm512_mul_ps(vs4, _mm512_set1_ps(es[r])), _mm512_cvtepi32_ps(acc[r]), tt);
                            tt = _mm512_fmadd_ps(vo4, _mm512_set1_ps(eo[r]), tt);
                            _mm512_storeu_ps(tr, tt);
                        }
                    }
                }
            }
            for (int64_t r = 0; r < rows; ++r) {
                const float inv = (float)(1.0 / total[r]);
                float *dst = y + ((bi * lq + i0 + r) * h + hh) * dv;
                for (int64_t c = 0; c < dv; ++c) dst[c] = t[r * dvt * 16 + c] * inv;
            }
        }
    }
}

/* The GEGLU after a product (fusion.cc:347-394): out[m][j] = y[m][j]
 * GELU(y[m][N / 2 + j]), GELU(g) = g / (1 + e^(-k g (1 + 0.044715 g^2))),
 * k = 2 sqrt(2 / pi); 16 numbers a vector. */
void oracle_port_gated(const float *y, int64_t M, int64_t N, float *out, int threads) {
    const int64_t half = N / 2;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        const float *row = y + m * N;
        float *dst = out + m * half;
        for (int64_t j = 0; j < half; j += 16) {
            const __mmask16 live = half - j >= 16 ? (__mmask16)0xffff : (__mmask16)((1u << (half - j)) - 1u);
            const v16 a = (v16)_mm512_maskz_loadu_ps(live, row + j);
            const v16 g = (v16)_mm512_maskz_loadu_ps(live, row + half + j);
            const v16 e = exp16(g * (1.0f + 0.044715f * g * g) * -1.5957691216057308f);
            _mm512_mask_storeu_ps(dst + j, live, (__m512)(a * (g / (1.0f + e))));
        }
    }
}

/* ------------------------------------------------------------ the host's peak */

/* The host's single-precision FMA rate on `threads` threads, GFLOP/s: each
 * thread runs 16 independent chains of 16-lane FMAs for about `seconds`
 * (2 FLOPs a lane an FMA) -- the peak the reference's figures are quoted
 * against (README.md:36, tools/bench.cc's FMA peak). */
double oracle_port_fma_peak(int threads, double seconds) {
    double total = 0.0;
    const double t0 = omp_get_wtime();
#pragma omp parallel num_threads(threads) reduction(+ : total)
    {
        v16 a[16];
        for (int i = 0; i < 16; ++i) a[i] = (v16){0} + (float)(i + 1) * 1e-3f;
        const v16 mul = (v16){0} + 0.999999f, add = (v16){0} + 1e-7f;
        int64_t iters = 0;
        while (omp_get_wtime() - t0 < seconds) {
            for (int r = 0; r < 1024; ++r) {
#pragma GCC unroll 16
                for (int i = 0; i < 16; ++i) a[i] = a[i] * mul + add;
            }
            iters += 1024;
        }
        float s = 0.0f;
        for (int i = 0; i < 16; ++i) s += a[i][0];
        volatile float sink = s;  /* the chains' results are used */
        (void)sink;
        total += (double)iters * 16 * 16 * 2;
    }
    const double dt = omp_get_wtime() - t0;
    return total / dt / 1e9;
}
