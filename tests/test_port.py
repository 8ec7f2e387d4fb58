"""The CPU baseline (oracle/port.c) computes what it is timed as: each of its
restatements against the float64 oracle within the reference's bounds for
the operation (tests/ops_test.cc:154-211), at ragged shapes that reach every
partial tile, panel and stretch of its blocking, and on one thread and
several alike; its bits-mode product bit for bit the oracle's qgemm.  A
figure timed on a port that computed something else would be no baseline."""

import numpy as np
import pytest

import oracle_lib as orc
from helpers import rng, uniform

pytestmark = pytest.mark.skipif(not orc.port_available(), reason="the host lacks AVX-512 with VNNI")


def f16(a):
    return a.astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("four", [True, False])
@pytest.mark.parametrize("n,ic,h,w,oc", [(2, 13, 18, 22, 11), (1, 70, 9, 7, 130), (2, 520, 8, 8, 70)])
def test_winograd(four, n, ic, h, w, oc):
    r = rng(n * 1000 + ic + oc)
    x = uniform(r, (n, ic, h, w), 1.0)
    k = f16(uniform(r, (oc, ic, 3, 3), 0.25))
    b = uniform(r, (oc,), 1.0)
    res = uniform(r, (n, oc, h, w), 1.0)
    y1 = orc.port_winograd(x, k, 1, b, res, four=four, threads=1)
    y3 = orc.port_winograd(x, k, 1, b, res, four=four, threads=3)
    exact, mag = orc.exact_conv2d(x, k, 1, 1, 1, 1, 1, 1)
    add = b[None, :, None, None].astype(np.float64) + res
    # The reference's bounds: F(4x4) 5-11e-7 published, F(2x2) ~2e-7.
    assert orc.metric(y1, exact + add, mag + np.abs(add)) <= (2e-6 if four else 1e-6)
    assert np.array_equal(y1, y3)
    y0 = orc.port_winograd(x, k, 1, four=four, threads=2)
    assert orc.metric(y0, exact, mag) <= (2e-6 if four else 1e-6)


@pytest.mark.parametrize("k,stride,pad", [(1, 1, 0), (3, 1, 1), (3, 2, 1), (1, 2, 0)])
def test_conv2d(k, stride, pad):
    r = rng(31 + k + stride)
    n, ic, h, w, oc = 2, 37, 13, 19, 70
    x = uniform(r, (n, ic, h, w), 1.0)
    kern = f16(uniform(r, (oc, ic, k, k), 0.25))
    b = uniform(r, (oc,), 1.0)
    exact, mag = orc.exact_conv2d(x, kern, stride, stride, pad, pad, 1, 1)
    res = uniform(r, exact.shape, 1.0)
    y1 = orc.port_conv2d(x, kern, stride, pad, b, res, threads=1)
    y4 = orc.port_conv2d(x, kern, stride, pad, b, res, threads=4)
    add = b[None, :, None, None].astype(np.float64) + res
    assert orc.metric(y1, exact + add, mag + np.abs(add)) <= 1e-6
    assert np.array_equal(y1, y4)


def test_mul_mat():
    r = rng(21)
    N, K, M = 137, 300, 43
    w = f16(uniform(r, (N, K), 0.25))
    x = uniform(r, (M, K), 1.0)
    b = uniform(r, (N,), 1.0)
    exact, mag = orc.exact_mul_mat(w, x)
    y1 = orc.port_mul_mat(w, x, b, threads=1)
    y3 = orc.port_mul_mat(w, x, b, threads=3)
    assert orc.metric(y1, exact + b, mag + np.abs(b)) <= 1e-6
    assert np.array_equal(y1, y3)


@pytest.mark.parametrize("lq,lk,h,d,dv", [(50, 77, 2, 40, 40), (97, 300, 1, 64, 64), (20, 33, 3, 80, 80)])
def test_attention(lq, lk, h, d, dv):
    r = rng(lq + lk)
    q = uniform(r, (2, lq, h, d), 1.0)
    k = uniform(r, (2, lk, h, d), 1.0)
    v = uniform(r, (2, lk, h, dv), 1.0)
    scale = 1.0 / np.sqrt(d)
    y1 = orc.port_attention(q, k, v, scale, threads=1)
    y2 = orc.port_attention(q, k, v, scale, threads=2)
    exact, mag = orc.exact_attention(q, k, v, scale)
    assert orc.metric(y1, exact, mag) <= 1e-6  # the north star's attention bound
    assert np.array_equal(y1, y2)


@pytest.mark.parametrize("lq,lk,h,hk,d,group", [(60, 988, 2, 2, 64, 64), (33, 300, 4, 2, 40, 32), (20, 700, 1, 1, 80, 128)])
def test_quantized_attention(lq, lk, h, hk, d, group):
    """The bits-mode attention of the CPU baseline: the oracle's algorithm
    (its exponentials by the port's own polynomial, so a quantized byte may
    differ by one step), within the reference's bound for quantized forms of
    float64 and close to the oracle."""
    r = rng(lk + d)
    q, k, v = uniform(r, (2, lq, h, d), 1.0), uniform(r, (2, lk, hk, d), 1.0), uniform(r, (2, lk, hk, d), 1.0)
    scale = float(1.0 / np.sqrt(d))
    kb = max(group, 256 // group * group)
    got = orc.port_quantized_attention(q, k, v, scale, group, key_block=kb, threads=4)
    want = orc.quantized_attention(q, k, v, scale, group, key_block=kb)
    exact, mag = orc.exact_attention(q, k, v, scale)
    assert orc.metric(got, exact, mag) <= 1e-2 * (2.0 / 255 + 1.0 / 127) / (2.0 / 255 + 1.0 / 127)
    assert orc.metric(got, want, mag) <= 1e-3


@pytest.mark.parametrize("silu", [False, True])
def test_group_norm(silu):
    r = rng(5)
    x = uniform(r, (2, 64, 12, 20), 3.0)
    g = 1.0 + uniform(r, (64,), 0.1)
    b = uniform(r, (64,), 0.1)
    want = orc.group_norm(x, 32, 1e-5) * g[None, :, None, None] + b[None, :, None, None]
    if silu:
        want = want / (1.0 + np.exp(-want.astype(np.float64)))
    got = orc.port_group_norm(x, 32, 1e-5, g, b, silu, threads=3)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)


def test_norm():
    r = rng(6)
    x = uniform(r, (2, 37, 320), 3.0)
    g = 1.0 + uniform(r, (320,), 0.1)
    b = uniform(r, (320,), 0.1)
    want = orc.norm(x, 1e-5) * g + b
    assert np.allclose(orc.port_norm(x, 1e-5, g, b, threads=2), want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("weight_groups", [0, 1])
@pytest.mark.parametrize("M,N,K", [(13, 70, 150), (40, 64, 256)])
def test_quantized_linear_is_the_oracles_qgemm(weight_groups, M, N, K):
    """The bits mode's product bit for bit the oracle's (quant.cc:113-164),
    the bias added after; its gated form the GELU of the second half."""
    r = rng(M + N + K)
    w = f16(uniform(r, (N, K), 0.25))
    x = uniform(r, (M, K), 1.0)
    b = uniform(r, (N,), 1.0)
    want, *_ = orc.quantized_mul_mat(w, x, group=64, weight_groups=weight_groups)
    wq, ws, wo, _ = orc.quantize_weights(w, 64, 127, weight_groups)
    packed = orc.port_pack_qweights(wq, ws, wo, 64)
    y1 = orc.port_quantized_linear(x, packed, N, 64, 255, b, threads=1)
    y3 = orc.port_quantized_linear(x, packed, N, 64, 255, b, threads=3)
    assert np.array_equal(y1, (want + b).astype(np.float32))
    assert np.array_equal(y1, y3)
    y, out = orc.port_quantized_linear(x, packed, N, 64, 255, b, gated=True, threads=2)
    half = N // 2
    g = y[:, half:2 * half].astype(np.float64)
    gelu = g / (1.0 + np.exp(-1.5957691216057308 * g * (1.0 + 0.044715 * g * g)))
    assert np.allclose(out, y[:, :half] * gelu, rtol=1e-5, atol=1e-6)


def test_gated():
    r = rng(9)
    y = uniform(r, (37, 2 * 70), 3.0)
    g = y[:, 70:].astype(np.float64)
    want = y[:, :70] * (g / (1.0 + np.exp(-1.5957691216057308 * g * (1.0 + 0.044715 * g * g))))
    assert np.allclose(orc.port_gated(y, threads=2), want, rtol=2e-6, atol=1e-7)


def test_fma_peak():
    one = orc.port_fma_peak(1, 0.1)
    assert one > 1.0  # GFLOP/s
