/*
 * CPU restatements of the reference's algorithms, in single precision, for
 * bench.py's cpu_baseline leg and as a second check of the float64 oracle.
 * TEST INFRASTRUCTURE (oracle.h): the library never calls these.
 *
 * They follow the reference's blocking in spirit -- weights transformed or
 * packed once, then blocks of outputs each thread computes whole from a tile
 * of registers -- in C that gcc vectorises (-O3 -mavx2 -mfma), with OpenMP
 * threads in place of ggml's pool.  They are not the reference's hand-written
 * x86 kernels, which cannot be built here (the reference needs ggml and C++26).
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* F(4x4, 3x3) matrices of winograd.cc:1155-1183, 1259-1264. */
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

enum { TILES = 16, OCS = 6 };

/* B^T d B of the 6 x 6 inputs of every tile of a block, channel c, into
 * v[xi][c][TILES]. */
static void inputs4(const float *plane, int64_t ih, int64_t iw, int64_t tw, int p0, int p1, int64_t t0, int64_t nt,
                    int64_t ic, int64_t c, float *v) {
    for (int64_t l = 0; l < nt; ++l) {
        const int64_t tile = t0 + l;
        const int64_t y0 = (tile / tw) * 4 - p1, x0 = (tile % tw) * 4 - p0;
        float d[6][6], bd[6][6];
        for (int i = 0; i < 6; ++i)
            for (int j = 0; j < 6; ++j) {
                const int64_t yy = y0 + i, xx = x0 + j;
                d[i][j] = (yy >= 0 && yy < ih && xx >= 0 && xx < iw) ? plane[yy * iw + xx] : 0.0f;
            }
        for (int r = 0; r < 6; ++r)
            for (int j = 0; j < 6; ++j) {
                float s = 0.0f;
                for (int i = 0; i < 6; ++i) s += BT4[r][i] * d[i][j];
                bd[r][j] = s;
            }
        for (int r = 0; r < 6; ++r)
            for (int s = 0; s < 6; ++s) {
                float acc = 0.0f;
                for (int j = 0; j < 6; ++j) acc += bd[r][j] * BT4[s][j];
                v[((r * 6 + s) * ic + c) * TILES + l] = acc;
            }
    }
}

/* Y = A^T M A of a block's tiles of output channel o, m [xi][TILES], with
 * the bias and the residual added. */
static void outputs4(const float *m, float *y, int64_t b, int64_t o, int64_t oc, int64_t t0, int64_t nt, int64_t tw,
                     int64_t oh, int64_t ow, const float *bias, const float *residual) {
    for (int64_t l = 0; l < nt; ++l) {
        const int64_t tile = t0 + l;
        const int64_t ty = tile / tw, tx = tile % tw;
        float am[4][6];
        for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 6; ++j) {
                float s = 0.0f;
                for (int k = 0; k < 6; ++k) s += AT4[i][k] * m[(k * 6 + j) * TILES + l];
                am[i][j] = s;
            }
        for (int i = 0; i < 4; ++i) {
            const int64_t yy = ty * 4 + i;
            if (yy >= oh) continue;
            for (int jj = 0; jj < 4; ++jj) {
                const int64_t xx = tx * 4 + jj;
                if (xx >= ow) continue;
                float s = 0.0f;
                for (int j = 0; j < 6; ++j) s += am[i][j] * AT4[jj][j];
                const int64_t at = ((b * oc + o) * oh + yy) * ow + xx;
                if (bias) s = s + bias[o];
                if (residual) s = s + residual[at];
                y[at] = s;
            }
        }
    }
}

/* The large-image F(4x4, 3x3) of winograd.cc:1548-1613: the weights
 * transformed once into U[xi][oc][ic]; then per (image, block of 16 tiles) a
 * thread transforms the block's inputs into V[xi][ic][16], makes the 36
 * products for OCS output channels at a time from a tile of registers, and
 * transforms them into the outputs, adding the bias and the residual (the
 * chain of cfg2).  x [n][ic][ih][iw], w [oc][ic][3][3] widened,
 * y [n][oc][oh][ow], oh = ih + 2 p1 - 2. */
void oracle_port_winograd4(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w, int64_t oc,
                           int p0, int p1, const float *bias, const float *residual, float *y, int threads) {
    const int64_t oh = ih + 2 * p1 - 2, ow = iw + 2 * p0 - 2;
    const int64_t tw = (ow + 3) / 4, th = (oh + 3) / 4, per_image = tw * th;
    const int64_t plane_u = oc * ic;
    float *u = (float *)malloc((size_t)(36 * plane_u) * sizeof(float));
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t t = 0; t < plane_u; ++t) {
        const float *g = w + t * 9;
        float gg[6][3];
        for (int i = 0; i < 6; ++i)
            for (int j = 0; j < 3; ++j) gg[i][j] = G4[i][0] * g[j] + G4[i][1] * g[3 + j] + G4[i][2] * g[6 + j];
        for (int i = 0; i < 6; ++i)
            for (int j = 0; j < 6; ++j)
                u[(i * 6 + j) * plane_u + t] = gg[i][0] * G4[j][0] + gg[i][1] * G4[j][1] + gg[i][2] * G4[j][2];
    }
    const int64_t blocks = (per_image + TILES - 1) / TILES;
#pragma omp parallel num_threads(threads)
    {
        float *v = (float *)malloc((size_t)(36 * ic * TILES) * sizeof(float));
        float *m = (float *)malloc((size_t)(OCS * 36 * TILES) * sizeof(float));
#pragma omp for schedule(dynamic, 1)
        for (int64_t item = 0; item < n * blocks; ++item) {
            const int64_t b = item / blocks;
            const int64_t t0 = (item % blocks) * TILES;
            const int64_t nt = per_image - t0 < TILES ? per_image - t0 : TILES;
            memset(v, 0, (size_t)(36 * ic * TILES) * sizeof(float));
            for (int64_t c = 0; c < ic; ++c) inputs4(x + (b * ic + c) * ih * iw, ih, iw, tw, p0, p1, t0, nt, ic, c, v);
            for (int64_t o0 = 0; o0 < oc; o0 += OCS) {
                const int64_t ocs = oc - o0 < OCS ? oc - o0 : OCS;
                for (int xi = 0; xi < 36; ++xi) {
                    float acc[OCS][TILES];
                    memset(acc, 0, sizeof acc);
                    const float *vx = v + (int64_t)xi * ic * TILES;
                    const float *ux = u + xi * plane_u + o0 * ic;
                    for (int64_t c = 0; c < ic; ++c) {
                        const float *vr = vx + c * TILES;
                        for (int r = 0; r < OCS; ++r) {
                            const float uv = r < ocs ? ux[r * ic + c] : 0.0f;
                            for (int l = 0; l < TILES; ++l) acc[r][l] += uv * vr[l];
                        }
                    }
                    for (int r = 0; r < ocs; ++r) memcpy(m + ((int64_t)r * 36 + xi) * TILES, acc[r], sizeof acc[r]);
                }
                for (int64_t r = 0; r < ocs; ++r)
                    outputs4(m + r * 36 * TILES, y, b, o0 + r, oc, t0, nt, tw, oh, ow, bias, residual);
            }
        }
        free(v);
        free(m);
    }
    free(u);
}

/* MUL_MAT in single precision with the weights packed once (mul_mat.cc:306-366
 * in spirit): y[m][n] = sum_k x[m][k] w[n][k] (+ bias[n]); rows in blocks of 4,
 * the weights transposed to [K][N] so that a row's columns go by in vectors. */
void oracle_port_mul_mat(const float *w, const float *x, const float *bias, int64_t M, int64_t N, int64_t K, float *y,
                         int threads) {
    float *wt = (float *)malloc((size_t)(K * N) * sizeof(float));
#pragma omp parallel for num_threads(threads)
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) wt[k * N + n] = w[n * K + k];
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t m0 = 0; m0 < M; m0 += 4) {
        const int64_t rows = M - m0 < 4 ? M - m0 : 4;
        for (int64_t r = 0; r < rows; ++r) {
            float *out = y + (m0 + r) * N;
            for (int64_t n = 0; n < N; ++n) out[n] = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                const float xv = x[(m0 + r) * K + k];
                const float *wr = wt + k * N;
                for (int64_t n = 0; n < N; ++n) out[n] += xv * wr[n];
            }
            if (bias)
                for (int64_t n = 0; n < N; ++n) out[n] += bias[n];
        }
    }
    free(wt);
}
