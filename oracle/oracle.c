/*
 * The oracle (oracle.h): TEST INFRASTRUCTURE, never part of the library.
 * Built with -ffp-contract=off, so that each operation rounds as written.
 */
#include "oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ scalar math */

/* sources/scalar_math.h:34-51: x clamped, n = round(x / ln 2) by the sum with
 * 1.5 * 2^23, r = x - n ln 2 in two fused steps, Cephes' expf polynomial,
 * 2^n from the exponent bits. */
float oracle_exponential(float x) {
    x = fminf(fmaxf(x, -87.3f), 88.73f);
    const float magic = 12582912.0f;
    const float z = fmaf(x, 1.44269504088896341f, magic);
    const float n = z - magic;
    float r = fmaf(n, -0.693359375f, x);
    r = fmaf(n, 2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    p = fmaf(p * r, r, r) + 1.0f;
    int32_t zi;
    memcpy(&zi, &z, 4);
    const uint32_t e = (uint32_t)(zi - 0x4b400000 + 127) << 23;
    float two;
    memcpy(&two, &e, 4);
    return p * two;
}

/* scalar_math.h:54-56 */
float oracle_silu(float x) { return x / (1.0f + oracle_exponential(-x)); }

void oracle_silu_array(float *x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = oracle_silu(x[i]);
}

/* scalar_math.h:58-63 */
float oracle_gelu(float x) {
    const float y = x * fmaf(0.044715f * x, x, 1.0f);
    return x / (1.0f + oracle_exponential(-1.5957691216057308f * y));
}

void oracle_exponential_array(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_exponential(x[i]);
}

void oracle_gelu_array(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_gelu(x[i]);
}

void oracle_gated_gelu_array(const float *x, const float *gate, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] * oracle_gelu(gate[i]);
}

/* ------------------------------------------------------------------ float64 */

void oracle_exact_mul_mat(const float *w, int64_t ldw, const float *x, int64_t ldx, int64_t M, int64_t N,
                          int64_t K, double *y, double *mag) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            double s = 0.0, a = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                const double p = (double)w[n * ldw + k] * (double)x[m * ldx + k];
                s += p;
                a += fabs(p);
            }
            y[m * N + n] = s;
            mag[m * N + n] = a;
        }
    }
}

void oracle_exact_conv2d(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w, int64_t oc,
                         int64_t kh, int64_t kw, int s0, int s1, int p0, int p1, int d0, int d1, int64_t oh,
                         int64_t ow, double *y, double *mag) {
    for (int64_t b = 0; b < n; ++b) {
        for (int64_t o = 0; o < oc; ++o) {
            for (int64_t oy = 0; oy < oh; ++oy) {
                for (int64_t ox = 0; ox < ow; ++ox) {
                    double s = 0.0, a = 0.0;
                    for (int64_t c = 0; c < ic; ++c) {
                        for (int64_t ky = 0; ky < kh; ++ky) {
                            const int64_t yy = oy * s1 + ky * d1 - p1;
                            if (yy < 0 || yy >= ih) continue;
                            for (int64_t kx = 0; kx < kw; ++kx) {
                                const int64_t xx = ox * s0 + kx * d0 - p0;
                                if (xx < 0 || xx >= iw) continue;
                                const double p = (double)w[((o * ic + c) * kh + ky) * kw + kx] *
                                                 (double)x[((b * ic + c) * ih + yy) * iw + xx];
                                s += p;
                                a += fabs(p);
                            }
                        }
                    }
                    const int64_t at = ((b * oc + o) * oh + oy) * ow + ox;
                    y[at] = s;
                    mag[at] = a;
                }
            }
        }
    }
}

void oracle_exact_conv2d_at(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w,
                            int64_t oc, int64_t kh, int64_t kw, int s0, int s1, int p0, int p1, int d0, int d1,
                            int64_t oh, int64_t ow, const int64_t *index, int64_t count, double *y, double *mag) {
    (void)n;
    for (int64_t t = 0; t < count; ++t) {
        const int64_t at = index[t];
        const int64_t ox = at % ow;
        const int64_t oy = (at / ow) % oh;
        const int64_t o = (at / (ow * oh)) % oc;
        const int64_t b = at / (ow * oh * oc);
        double s = 0.0, a = 0.0;
        for (int64_t c = 0; c < ic; ++c) {
            for (int64_t ky = 0; ky < kh; ++ky) {
                const int64_t yy = oy * s1 + ky * d1 - p1;
                if (yy < 0 || yy >= ih) continue;
                for (int64_t kx = 0; kx < kw; ++kx) {
                    const int64_t xx = ox * s0 + kx * d0 - p0;
                    if (xx < 0 || xx >= iw) continue;
                    const double p = (double)w[((o * ic + c) * kh + ky) * kw + kx] *
                                     (double)x[((b * ic + c) * ih + yy) * iw + xx];
                    s += p;
                    a += fabs(p);
                }
            }
        }
        y[t] = s;
        mag[t] = a;
    }
}

void oracle_exact_attention(const float *q, const float *k, const float *v, int64_t d, int64_t dv, int64_t lq,
                            int64_t lk, int64_t h, int64_t hk, int64_t b, float scale, double *y, double *mag) {
    double *w = (double *)malloc((size_t)lk * sizeof(double));
    const int64_t group = h / hk;
    for (int64_t bi = 0; bi < b; ++bi) {
        for (int64_t hi = 0; hi < h; ++hi) {
            const int64_t kh = hi / group;
            for (int64_t i = 0; i < lq; ++i) {
                const float *qi = q + ((bi * lq + i) * h + hi) * d;
                double max = -HUGE_VAL;
                for (int64_t j = 0; j < lk; ++j) {
                    const float *kj = k + ((bi * lk + j) * hk + kh) * d;
                    double s = 0.0;
                    for (int64_t e = 0; e < d; ++e) s += (double)qi[e] * (double)kj[e];
                    w[j] = s * (double)scale;
                    if (w[j] > max) max = w[j];
                }
                double total = 0.0;
                for (int64_t j = 0; j < lk; ++j) {
                    w[j] = exp(w[j] - max);
                    total += w[j];
                }
                for (int64_t e = 0; e < dv; ++e) {
                    double s = 0.0, a = 0.0;
                    for (int64_t j = 0; j < lk; ++j) {
                        const double p = w[j] / total * (double)v[((bi * lk + j) * hk + kh) * dv + e];
                        s += p;
                        a += fabs(p);
                    }
                    const int64_t at = ((bi * lq + i) * h + hi) * dv + e;
                    y[at] = s;
                    mag[at] = a;
                }
            }
        }
    }
    free(w);
}

void oracle_exact_attention_at(const float *q, const float *k, const float *v, int64_t d, int64_t dv, int64_t lq,
                               int64_t lk, int64_t h, int64_t hk, int64_t b, float scale, const int64_t *query,
                               int64_t count, double *y, double *mag) {
    (void)b;
    double *w = (double *)malloc((size_t)lk * sizeof(double));
    const int64_t group = h / hk;
    for (int64_t t = 0; t < count; ++t) {
        const int64_t i = query[t] % lq;
        const int64_t hi = (query[t] / lq) % h;
        const int64_t bi = query[t] / (lq * h);
        const int64_t kh = hi / group;
        const float *qi = q + ((bi * lq + i) * h + hi) * d;
        double max = -HUGE_VAL;
        for (int64_t j = 0; j < lk; ++j) {
            const float *kj = k + ((bi * lk + j) * hk + kh) * d;
            double s = 0.0;
            for (int64_t e = 0; e < d; ++e) s += (double)qi[e] * (double)kj[e];
            w[j] = s * (double)scale;
            if (w[j] > max) max = w[j];
        }
        double total = 0.0;
        for (int64_t j = 0; j < lk; ++j) {
            w[j] = exp(w[j] - max);
            total += w[j];
        }
        for (int64_t e = 0; e < dv; ++e) {
            double s = 0.0, a = 0.0;
            for (int64_t j = 0; j < lk; ++j) {
                const double p = w[j] / total * (double)v[((bi * lk + j) * hk + kh) * dv + e];
                s += p;
                a += fabs(p);
            }
            y[t * dv + e] = s;
            mag[t * dv + e] = a;
        }
    }
    free(w);
}

static double gelu64(double v) { return 0.5 * v * (1.0 + tanh(0.79788456080286535587989211986876 * (v + 0.044715 * v * v * v))); }

void oracle_exact_gated(const float *w, const float *x, const float *bias, int64_t M, int64_t half, int64_t K,
                        double *y, double *mag) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t j = 0; j < half; ++j) {
            double sum[2], a[2];
            for (int side = 0; side < 2; ++side) {
                const int64_t n = side * half + j;
                sum[side] = bias ? (double)bias[n] : 0.0;
                a[side] = fabs(sum[side]);
                for (int64_t e = 0; e < K; ++e) {
                    const double p = (double)w[n * K + e] * (double)x[m * K + e];
                    sum[side] += p;
                    a[side] += fabs(p);
                }
            }
            /* d/dv of GELU(v) lies within [-0.13, 1.13] (ops_test.cc:761-764). */
            y[m * half + j] = sum[0] * gelu64(sum[1]);
            mag[m * half + j] = a[0] * fabs(gelu64(sum[1])) + fabs(sum[0]) * 1.13 * a[1];
        }
    }
}

/* ------------------------------------------------------------------ chain */

void oracle_apply_chain(float *out, const int64_t ne[4], int count, const int *kinds, const float *const *operands,
                        const int64_t *nb) {
    for (int64_t i3 = 0; i3 < ne[3]; ++i3)
        for (int64_t i2 = 0; i2 < ne[2]; ++i2)
            for (int64_t i1 = 0; i1 < ne[1]; ++i1)
                for (int64_t i0 = 0; i0 < ne[0]; ++i0) {
                    float *o = out + ((i3 * ne[2] + i2) * ne[1] + i1) * ne[0] + i0;
                    float v = *o;
                    for (int s = 0; s < count; ++s) {
                        if (kinds[s] == 2) {
                            v = oracle_silu(v);
                            continue;
                        }
                        const int64_t *b = nb + 4 * s;
                        const float op = operands[s][i0 * b[0] + i1 * b[1] + i2 * b[2] + i3 * b[3]];
                        v = kinds[s] == 0 ? v + op : v * op;
                    }
                    *o = v;
                }
}

/* ------------------------------------------------------------------ norms */

/* The sum of a row in double, in 8 lanes (norm.cc:44-62). */
static double row_sum(const float *x, int64_t n) {
    double part[8] = {0};
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) part[l] += (double)x[i + l];
    double s = 0.0;
    for (; i < n; ++i) s += (double)x[i];
    for (int l = 0; l < 8; ++l) s += part[l];
    return s;
}

/* The squares of (x - mean) in single precision summed in double (norm.cc:64-84). */
static double row_squares(const float *x, int64_t n, float mean) {
    double part[8] = {0};
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; ++l) {
            const float v = x[i + l] - mean;
            part[l] += (double)(v * v);
        }
    double s = 0.0;
    for (; i < n; ++i) {
        const float v = x[i] - mean;
        s += (double)(v * v);
    }
    for (int l = 0; l < 8; ++l) s += part[l];
    return s;
}

void oracle_group_norm(const float *x, float *y, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, int groups,
                       float eps) {
    const int64_t per = (ne2 + groups - 1) / groups;
    const int64_t plane = ne0 * ne1;
    for (int64_t i3 = 0; i3 < ne3; ++i3) {
        for (int64_t g = 0; g < groups; ++g) {
            const int64_t c0 = g * per;
            const int64_t c1 = c0 + per < ne2 ? c0 + per : ne2;
            if (c0 >= c1) continue;
            const int64_t count = plane * (c1 - c0);
            const float *in = x + (i3 * ne2 + c0) * plane;
            float *out = y + (i3 * ne2 + c0) * plane;
            const float mean = (float)(row_sum(in, count) / (double)count);
            const float variance = (float)(row_squares(in, count, mean) / (double)count);
            const float scale = 1.0f / sqrtf(variance + eps);
            for (int64_t i = 0; i < count; ++i) out[i] = (in[i] - mean) * scale;
        }
    }
}

void oracle_norm(const float *x, float *y, int64_t ne0, int64_t rows, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *in = x + r * ne0;
        float *out = y + r * ne0;
        const float mean = (float)(row_sum(in, ne0) / (double)ne0);
        const float variance = (float)(row_squares(in, ne0, mean) / (double)ne0);
        const float scale = 1.0f / sqrtf(variance + eps);
        for (int64_t i = 0; i < ne0; ++i) out[i] = (in[i] - mean) * scale;
    }
}

/* ------------------------------------------------------------------ bits mode */

static float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* quant.cc:282-315: least and greatest with 0 between them, scale (hi - lo) /
 * levels, the inverse 0 for a scale of 0, the zero point rounded to the
 * nearest-even, each byte rint(x * inverse) + zero clamped to [0, levels];
 * the group's tail the zero point. */
void oracle_quantize_input_row(const float *x, int64_t n, int64_t group, int levels, uint8_t *dst, float *scale,
                               float *offset) {
    float least = 0.0f, greatest = 0.0f;
    for (int64_t e = 0; e < n; ++e) {
        least = fminf(least, x[e]);
        greatest = fmaxf(greatest, x[e]);
    }
    const float s = (greatest - least) / (float)levels;
    const float inverse = s > 0.0f ? 1.0f / s : 0.0f;
    const float zero = nearbyintf(-least * inverse);
    const float top = (float)levels;
    int64_t e = 0;
    for (; e < n; ++e) dst[e] = (uint8_t)clampf(nearbyintf(x[e] * inverse) + zero, 0.0f, top);
    for (; e < group; ++e) dst[e] = (uint8_t)zero;
    *scale = s;
    *offset = s * zero;
}

/* quant.cc:204-243 with quantize_weight_group (186-199): the scale of the
 * group's (or with weight_groups = 0, the whole row's) greatest magnitude over
 * weight_max; each weight rint(w * inverse) clamped to +-weight_max; the
 * offset the scale times the group's integer sum; zeros past k. */
void oracle_quantize_weights(const float *w, int64_t ld, int64_t rows, int64_t k, int64_t group, int weight_max,
                             int weight_groups, int8_t *q, float *scale, float *offset, int32_t *sums) {
    const int64_t groups = (k + group - 1) / group;
    const float max = (float)weight_max;
    for (int64_t r = 0; r < rows; ++r) {
        float row_max = 0.0f;
        if (!weight_groups) {
            for (int64_t e = 0; e < k; ++e) row_max = fmaxf(row_max, fabsf(w[r * ld + e]));
        }
        for (int64_t g = 0; g < groups; ++g) {
            const int64_t n = k - g * group < group ? k - g * group : group;
            float m = row_max;
            if (weight_groups) {
                for (int64_t e = 0; e < n; ++e) m = fmaxf(m, fabsf(w[r * ld + g * group + e]));
            }
            const float s = m / max;
            const float inverse = s > 0.0f ? 1.0f / s : 0.0f;
            int32_t sum = 0;
            int8_t *dst = q + r * groups * group + g * group;
            for (int64_t e = 0; e < group; ++e) {
                const float v = e < n ? w[r * ld + g * group + e] : 0.0f;
                const int32_t qv = (int32_t)clampf(nearbyintf(v * inverse), -max, max);
                dst[e] = (int8_t)qv;
                sum += qv;
            }
            scale[r * groups + g] = s;
            offset[r * groups + g] = s * (float)sum;
            sums[r * groups + g] = sum;
        }
    }
}

/* qgemm (quant.cc:113-164): y[m][n] = init (or 0), then per group g in order
 * t = fma(sa sb, S, t); t = fma(-oa, ob, t), S the exact integer sum of the
 * group's products; operands [rows][groups * group], scales and offsets
 * [rows][groups]. */
void oracle_qgemm(const uint8_t *xq, const float *xs, const float *xo, const int8_t *wq, const float *ws,
                  const float *wo, int64_t M, int64_t N, int64_t groups, int64_t group, const float *init, float *y) {
    const int64_t kp = groups * group;
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            float t = init ? init[m * N + n] : 0.0f;
            for (int64_t g = 0; g < groups; ++g) {
                int32_t s = 0;
                const uint8_t *a = xq + m * kp + g * group;
                const int8_t *b = wq + n * kp + g * group;
                for (int64_t e = 0; e < group; ++e) s += (int32_t)a[e] * (int32_t)b[e];
                const float ab = xs[m * groups + g] * ws[n * groups + g];
                t = fmaf(ab, (float)s, t);
                t = fmaf(-xo[m * groups + g], wo[n * groups + g], t);
            }
            y[m * N + n] = t;
        }
    }
}

void oracle_quantized_mul_mat(const float *w, const float *x, int64_t M, int64_t N, int64_t K, int64_t group,
                              int input_levels, int weight_max, int weight_groups, const float *init, float *y,
                              uint8_t *xq, float *xscale, float *xoffset, int8_t *wq, float *wscale, float *woffset,
                              int32_t *wsums) {
    const int64_t groups = (K + group - 1) / group;
    const int64_t kp = groups * group;
    uint8_t *qx = xq ? xq : (uint8_t *)malloc((size_t)(M * kp));
    float *sa = xscale ? xscale : (float *)malloc((size_t)(M * groups) * sizeof(float));
    float *oa = xoffset ? xoffset : (float *)malloc((size_t)(M * groups) * sizeof(float));
    int8_t *qw = wq ? wq : (int8_t *)malloc((size_t)(N * kp));
    float *sb = wscale ? wscale : (float *)malloc((size_t)(N * groups) * sizeof(float));
    float *ob = woffset ? woffset : (float *)malloc((size_t)(N * groups) * sizeof(float));
    int32_t *qs = wsums ? wsums : (int32_t *)malloc((size_t)(N * groups) * sizeof(int32_t));
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t g = 0; g < groups; ++g) {
            const int64_t n = K - g * group < group ? K - g * group : group;
            oracle_quantize_input_row(x + m * K + g * group, n, group, input_levels, qx + m * kp + g * group,
                                      &sa[m * groups + g], &oa[m * groups + g]);
        }
    }
    oracle_quantize_weights(w, K, N, K, group, weight_max, weight_groups, qw, sb, ob, qs);
    oracle_qgemm(qx, sa, oa, qw, sb, ob, M, N, groups, group, init, y);
    if (!xq) free(qx);
    if (!xscale) free(sa);
    if (!xoffset) free(oa);
    if (!wq) free(qw);
    if (!wscale) free(sb);
    if (!woffset) free(ob);
    if (!wsums) free(qs);
}

/* attention.cc:612-824 (compute_quantized), with the quantizers above:
 * over_dims (the keys and queries: one group of 4 ceil(d / 4) over the
 * dimensions, attention.cc:632-637) and over_keys (the values and
 * exponentials: groups of `group` keys, 639-643); key_block the stretch of
 * the exponentials, a multiple of the group (663-664). */
void oracle_quantized_attention(const float *q, const float *k, const float *v, int64_t d, int64_t dv, int64_t lq,
                                int64_t lk, int64_t h, int64_t hk, int64_t b, float scale, int64_t group,
                                int input_levels, int weight_max, int64_t key_block, float *y) {
    const int64_t gd = (d + 3) / 4 * 4;
    const int64_t groups = (lk + group - 1) / group;
    int8_t *kq = (int8_t *)malloc((size_t)(lk * gd));
    float *ks = (float *)malloc((size_t)lk * sizeof(float)), *ko = (float *)malloc((size_t)lk * sizeof(float));
    int32_t *ksum = (int32_t *)malloc((size_t)lk * sizeof(int32_t));
    float *vt = (float *)malloc((size_t)(dv * lk) * sizeof(float));
    int8_t *vq = (int8_t *)malloc((size_t)(dv * groups * group));
    float *vs = (float *)malloc((size_t)(dv * groups) * sizeof(float));
    float *vo = (float *)malloc((size_t)(dv * groups) * sizeof(float));
    int32_t *vsum = (int32_t *)malloc((size_t)(dv * groups) * sizeof(int32_t));
    float *krow = (float *)malloc((size_t)(lk * d) * sizeof(float));
    float *scores = (float *)malloc((size_t)lk * sizeof(float));
    uint8_t *qq = (uint8_t *)malloc((size_t)gd);
    uint8_t *eq = (uint8_t *)malloc((size_t)group);
    float *t = (float *)malloc((size_t)dv * sizeof(float));
    for (int64_t bi = 0; bi < b; ++bi) {
        for (int64_t kh = 0; kh < hk; ++kh) {
            /* The head's keys, rows of d, and its values by dimension. */
            for (int64_t j = 0; j < lk; ++j)
                for (int64_t e = 0; e < d; ++e) krow[j * d + e] = k[((bi * lk + j) * hk + kh) * d + e];
            for (int64_t c = 0; c < dv; ++c)
                for (int64_t j = 0; j < lk; ++j) vt[c * lk + j] = v[((bi * lk + j) * hk + kh) * dv + c];
            oracle_quantize_weights(krow, d, lk, d, gd, weight_max, 1, kq, ks, ko, ksum);
            oracle_quantize_weights(vt, lk, dv, lk, group, weight_max, 1, vq, vs, vo, vsum);
            for (int64_t hh = 0; hh < h; ++hh) {
                if (hh / (h / hk) != kh) continue;
                for (int64_t i = 0; i < lq; ++i) {
                    const float *qrow = q + ((bi * lq + i) * h + hh) * d;
                    float qs, qo;
                    oracle_quantize_input_row(qrow, d, gd, input_levels, qq, &qs, &qo);
                    qs = qs * scale; /* attention.cc:754-764 */
                    qo = qo * scale;
                    float top = -INFINITY;
                    for (int64_t j = 0; j < lk; ++j) {
                        int32_t s = 0;
                        for (int64_t e = 0; e < gd; ++e) s += (int32_t)kq[j * gd + e] * (int32_t)qq[e];
                        float x = fmaf(ks[j] * qs, (float)s, 0.0f);
                        x = fmaf(-ko[j], qo, x);
                        scores[j] = x;
                        top = fmaxf(top, x);
                    }
                    double total = 0.0;
                    for (int64_t c = 0; c < dv; ++c) t[c] = 0.0f;
                    for (int64_t j0 = 0; j0 < lk; j0 += key_block) {
                        const int64_t j1 = j0 + key_block < lk ? j0 + key_block : lk;
                        const int64_t whole = j0 + (j1 - j0) / 8 * 8;
                        for (int64_t j = j0; j < j1; ++j) {
                            const float e = j < whole ? oracle_exponential(scores[j] - top) : expf(scores[j] - top);
                            scores[j] = e;
                            total += (double)e;
                        }
                        for (int64_t g0 = j0; g0 < j1; g0 += group) {
                            const int64_t n = j1 - g0 < group ? j1 - g0 : group;
                            float es, eo;
                            oracle_quantize_input_row(scores + g0, n, group, input_levels, eq, &es, &eo);
                            const int64_t g = g0 / group;
                            for (int64_t c = 0; c < dv; ++c) {
                                int32_t s = 0;
                                const int8_t *row = vq + (c * groups + g) * group;
                                for (int64_t e = 0; e < group; ++e) s += (int32_t)row[e] * (int32_t)eq[e];
                                t[c] = fmaf(vs[c * groups + g] * es, (float)s, t[c]);
                                t[c] = fmaf(-vo[c * groups + g], eo, t[c]);
                            }
                        }
                    }
                    const float reciprocal = (float)(1.0 / total);
                    float *out = y + ((bi * lq + i) * h + hh) * dv;
                    for (int64_t c = 0; c < dv; ++c) out[c] = t[c] * reciprocal;
                }
            }
        }
    }
    free(kq); free(ks); free(ko); free(ksum); free(vt); free(vq); free(vs); free(vo); free(vsum);
    free(krow); free(scores); free(qq); free(eq); free(t);
}

/* ------------------------------------------------------------------ bits mode: convolutions */

/* The columns of a direct convolution (conv2d.cc:228-316): position p = (n,
 * oy, ox), k = ic KH KW + kh KW + kw, zeros outside the image. */
static float column_at(const float *x, int64_t ic, int64_t ih, int64_t iw, int64_t kh, int64_t kw, int s0, int s1, int p0,
                       int p1, int d0, int d1, int64_t oh, int64_t ow, int64_t p, int64_t k) {
    const int64_t n = p / (oh * ow), r = p % (oh * ow), oy = r / ow, ox = r % ow;
    const int64_t c = k / (kh * kw), t = k % (kh * kw), y = oy * s1 - p1 + (t / kw) * d1, xx = ox * s0 - p0 + (t % kw) * d0;
    return (y >= 0 && y < ih && xx >= 0 && xx < iw) ? x[((n * ic + c) * ih + y) * iw + xx] : 0.0f;
}

/* A mistake planted on purpose, for the tests that show the quantized
 * convolutions' checks can see one (0: none): 1, the direct convolution's
 * columns and kernels enumerated tap-major (k = (kh KW + kw) IC + ic) instead
 * of conv2d.cc:255-258's order -- the same sum, other groups; 2, Winograd's
 * weights quantized over every input channel at once instead of per stretch;
 * 3, per stretch of one group. */
int oracle_plant = 0;

void oracle_set_plant(int mode) { oracle_plant = mode; }

void oracle_quantized_conv2d(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w, int64_t oc,
                             int64_t kh, int64_t kw, int s0, int s1, int p0, int p1, int d0, int d1, int64_t oh,
                             int64_t ow, int64_t group, int input_levels, int weight_max, int weight_groups,
                             const float *init, float *y) {
    const int64_t K = ic * kh * kw, P = n * oh * ow, taps = kh * kw;
    float *cols = (float *)malloc((size_t)(P * K) * sizeof(float));
    float *t = (float *)malloc((size_t)(P * oc) * sizeof(float));
    float *it = init ? (float *)malloc((size_t)(P * oc) * sizeof(float)) : NULL;
    float *wk = (float *)malloc((size_t)(oc * K) * sizeof(float));
    /* Column k of the reference's order at place `at` of this one. */
    for (int64_t k = 0; k < K; ++k) {
        const int64_t at = oracle_plant == 1 ? (k % taps) * ic + k / taps : k;
        for (int64_t p = 0; p < P; ++p)
            cols[p * K + at] = column_at(x, ic, ih, iw, kh, kw, s0, s1, p0, p1, d0, d1, oh, ow, p, k);
        for (int64_t o = 0; o < oc; ++o) wk[o * K + at] = w[o * K + k];
    }
    for (int64_t p = 0; p < P; ++p) {
        const int64_t b = p / (oh * ow), r = p % (oh * ow);
        for (int64_t o = 0; o < oc; ++o) {
            if (it) it[p * oc + o] = init[(b * oc + o) * oh * ow + r];
        }
    }
    oracle_quantized_mul_mat(wk, cols, P, oc, K, group, input_levels, weight_max, weight_groups, it, t, NULL, NULL,
                             NULL, NULL, NULL, NULL, NULL);
    for (int64_t p = 0; p < P; ++p) {
        const int64_t b = p / (oh * ow), r = p % (oh * ow);
        for (int64_t o = 0; o < oc; ++o) y[(b * oc + o) * oh * ow + r] = t[p * oc + o];
    }
    free(cols);
    free(t);
    free(it);
    free(wk);
}

/* Row i of F(2x2)'s B^T of four numbers (winograd.cc:321-332). */
static float bt2(int i, float d0, float d1, float d2, float d3) {
    switch (i) {
    case 0: return d0 - d2;
    case 1: return d1 + d2;
    case 2: return d2 - d1;
    default: return d1 - d3;
    }
}

/* F(2x2, 3x3) with quantized products (winograd.cc:1826-2103): V = B^T d B
 * as transform_inputs_small computes it (each row of d by bt(s), then the
 * rows by bt(r), winograd.cc:631-672), U = G g G^T as transform_weights does
 * (G g a column at a time, then (G g) G^T a row at a time, each sum of three
 * left to right and halved after, winograd.cc:681-729); for each of the 16
 * points, the tiles' V quantized per (tile, group of input channels) and the
 * output channels' U per (channel, group), or per stretch of `stretch` input
 * channels with weight_groups = 0 (the scale of the stretch's greatest, as the
 * weights of a stretch are quantized at a time, winograd.cc:1917-1930); the
 * quantized products M per point (qgemm); then Y = A^T M A as
 * transform_outputs sums it (winograd.cc:509-623), added to y where
 * from_redirect.  x [n][ic][ih][iw], w [oc][ic][3][3]; y [n][oc][oh][ow]. */
void oracle_quantized_winograd2(const float *x, int64_t n, int64_t ic, int64_t ih, int64_t iw, const float *w,
                                int64_t oc, int p0, int p1, int64_t oh, int64_t ow, int64_t group, int input_levels,
                                int weight_max, int weight_groups, int64_t stretch, int from_redirect, float *y) {
    const int64_t tw = (ow + 1) / 2, th = (oh + 1) / 2, tiles = n * tw * th;
    const int64_t groups = (ic + group - 1) / group, kp = groups * group;
    float *v = (float *)malloc((size_t)(16 * tiles * ic) * sizeof(float));
    float *u = (float *)malloc((size_t)(16 * oc * ic) * sizeof(float));
    for (int64_t b = 0; b < n; ++b)
        for (int64_t ty = 0; ty < th; ++ty)
            for (int64_t tx = 0; tx < tw; ++tx)
                for (int64_t c = 0; c < ic; ++c) {
                    const int64_t tile = (b * th + ty) * tw + tx;
                    float d[4][4];
                    for (int i = 0; i < 4; ++i)
                        for (int j = 0; j < 4; ++j) {
                            const int64_t yy = 2 * ty - p1 + i, xx = 2 * tx - p0 + j;
                            d[i][j] = (yy >= 0 && yy < ih && xx >= 0 && xx < iw) ? x[((b * ic + c) * ih + yy) * iw + xx]
                                                                                   : 0.0f;
                        }
                    for (int s4 = 0; s4 < 4; ++s4) {
                        float row[4];
                        for (int i = 0; i < 4; ++i) row[i] = bt2(s4, d[i][0], d[i][1], d[i][2], d[i][3]);
                        for (int r = 0; r < 4; ++r)
                            v[((int64_t)(r * 4 + s4) * tiles + tile) * ic + c] = bt2(r, row[0], row[1], row[2], row[3]);
                    }
                }
    for (int64_t o = 0; o < oc; ++o)
        for (int64_t c = 0; c < ic; ++c) {
            const float *g = w + (o * ic + c) * 9;
            float t[4][3];
            for (int j = 0; j < 3; ++j) {
                const float g0 = g[0 * 3 + j], g1 = g[1 * 3 + j], g2 = g[2 * 3 + j];
                t[0][j] = g0;
                t[1][j] = 0.5f * (g0 + g1 + g2);
                t[2][j] = 0.5f * (g0 - g1 + g2);
                t[3][j] = g2;
            }
            for (int i = 0; i < 4; ++i) {
                const float a = t[i][0], bb = t[i][1], dd = t[i][2];
                u[((int64_t)(i * 4 + 0) * oc + o) * ic + c] = a;
                u[((int64_t)(i * 4 + 1) * oc + o) * ic + c] = 0.5f * (a + bb + dd);
                u[((int64_t)(i * 4 + 2) * oc + o) * ic + c] = 0.5f * (a - bb + dd);
                u[((int64_t)(i * 4 + 3) * oc + o) * ic + c] = dd;
            }
        }
    uint8_t *xq = (uint8_t *)malloc((size_t)(tiles * kp));
    float *xs = (float *)malloc((size_t)(tiles * groups) * sizeof(float));
    float *xo = (float *)malloc((size_t)(tiles * groups) * sizeof(float));
    int8_t *wq = (int8_t *)malloc((size_t)(oc * kp));
    float *ws = (float *)malloc((size_t)(oc * groups) * sizeof(float));
    float *wo = (float *)malloc((size_t)(oc * groups) * sizeof(float));
    int32_t *wsum = (int32_t *)malloc((size_t)(oc * groups) * sizeof(int32_t));
    if (oracle_plant == 2) stretch = (ic + group - 1) / group * group;
    if (oracle_plant == 3) stretch = group;
    const int64_t sg = stretch / group;  /* groups of a stretch */
    int8_t *tq = (int8_t *)malloc((size_t)(oc * sg * group));
    float *ts = (float *)malloc((size_t)(oc * sg) * sizeof(float));
    float *to = (float *)malloc((size_t)(oc * sg) * sizeof(float));
    int32_t *tsum = (int32_t *)malloc((size_t)(oc * sg) * sizeof(int32_t));
    float *m = (float *)malloc((size_t)(16 * tiles * oc) * sizeof(float));
    for (int xi = 0; xi < 16; ++xi) {
        const float *vx = v + (int64_t)xi * tiles * ic;
        const float *ux = u + (int64_t)xi * oc * ic;
        for (int64_t t = 0; t < tiles; ++t)
            for (int64_t g = 0; g < groups; ++g) {
                const int64_t cnt = ic - g * group < group ? ic - g * group : group;
                oracle_quantize_input_row(vx + t * ic + g * group, cnt, group, input_levels, xq + t * kp + g * group,
                                          &xs[t * groups + g], &xo[t * groups + g]);
            }
        if (weight_groups) {
            oracle_quantize_weights(ux, ic, oc, ic, group, weight_max, 1, wq, ws, wo, wsum);
        } else {
            for (int64_t k0 = 0; k0 < ic; k0 += stretch) {
                const int64_t kc = ic - k0 < stretch ? ic - k0 : stretch;
                const int64_t kg = (kc + group - 1) / group;
                oracle_quantize_weights(ux + k0, ic, oc, kc, group, weight_max, 0, tq, ts, to, tsum);
                for (int64_t o = 0; o < oc; ++o) {
                    memcpy(wq + o * kp + k0, tq + o * kg * group, (size_t)(kg * group));
                    for (int64_t g = 0; g < kg; ++g) {
                        ws[o * groups + k0 / group + g] = ts[o * kg + g];
                        wo[o * groups + k0 / group + g] = to[o * kg + g];
                        wsum[o * groups + k0 / group + g] = tsum[o * kg + g];
                    }
                }
            }
        }
        oracle_qgemm(xq, xs, xo, wq, ws, wo, tiles, oc, groups, group, NULL, m + (int64_t)xi * tiles * oc);
    }
    for (int64_t b = 0; b < n; ++b)
        for (int64_t o = 0; o < oc; ++o)
            for (int64_t ty = 0; ty < th; ++ty)
                for (int64_t tx = 0; tx < tw; ++tx) {
                    const int64_t tile = (b * th + ty) * tw + tx;
                    float vv[16];
                    for (int xi = 0; xi < 16; ++xi) vv[xi] = m[((int64_t)xi * tiles + tile) * oc + o];
                    float a0[4], a1[4];
                    for (int j = 0; j < 4; ++j) {
                        a0[j] = vv[0 * 4 + j] + vv[1 * 4 + j] + vv[2 * 4 + j];
                        a1[j] = vv[1 * 4 + j] - vv[2 * 4 + j] - vv[3 * 4 + j];
                    }
                    const float out[2][2] = {{a0[0] + a0[1] + a0[2], a0[1] - a0[2] - a0[3]},
                                             {a1[0] + a1[1] + a1[2], a1[1] - a1[2] - a1[3]}};
                    for (int i = 0; i < 2; ++i)
                        for (int j = 0; j < 2; ++j) {
                            const int64_t yy = 2 * ty + i, xx = 2 * tx + j;
                            if (yy >= oh || xx >= ow) continue;
                            float *p = y + ((b * oc + o) * oh + yy) * ow + xx;
                            *p = from_redirect ? *p + out[i][j] : out[i][j];
                        }
                }
    free(v); free(u); free(xq); free(xs); free(xo); free(wq); free(ws); free(wo); free(wsum);
    free(tq); free(ts); free(to); free(tsum); free(m);
}

/* Whether this host runs port.c's code, which is built for AVX-512 F, BW, DQ,
 * VL and VNNI; this file is not, so the check itself runs anywhere. */
int oracle_port_available(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512dq") && __builtin_cpu_supports("avx512vl") &&
           __builtin_cpu_supports("avx512vnni");
}
