"""bits=16, the products of 16 bits (tests/ops_test.cc:304-380, 837-919 with
bits = 16): MUL_MAT, its gated GELU and the direct convolutions of FP16
weights multiply them by their other operand rounded to FP16, one product
each, summed in single precision -- the reference's FP16 format
(cpu.cc:336-366, the split forms' first parts alone); Winograd, attention and
single-precision weights stay single precision, as on the reference's vector
units.  Held to the reference's kHalf = 8e-3 of the exact result, and to
single-precision sums (2e-6) of the products of the rounded operand."""

import numpy as np
import pytest
import torch

import oracle_lib as orc
import sdhip
from helpers import dev, rng, uniform, unwritten, weights_f16

K_HALF = 8e-3  # ops_test.cc:305
BOUND_SUM = 2e-6


def rounded(x):
    """x as the products of 16 bits take it: its first FP16 part (x 2^-4
    rounded to FP16, times 2^4)."""
    return ((x.astype(np.float32) * np.float32(0.0625)).astype(np.float16).astype(np.float64) * 16.0)


def run_mul_mat(gpu, K, N, M, B, tuning, seed):
    r = rng(seed)
    wh, w32 = weights_f16(r, (N, K))
    x = uniform(r, (B, M, K), 1.0)
    y = unwritten((B, M, N), gpu)
    sdhip.set_tuning(tuning)
    try:
        sdhip.mul_mat(dev(wh, gpu), dev(x, gpu), y)
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    return w32, x.reshape(B * M, K), y.cpu().numpy().reshape(B * M, N)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,M,B", [(320, 320, 512, 2), (768, 1280, 300, 1), (1280, 320, 256, 1), (300, 17, 131, 3),
                                     (768, 320, 77, 2), (5120, 1280, 64, 1)])
def test_mul_mat_half(gpu, K, N, M, B):
    w, x, y = run_mul_mat(gpu, K, N, M, B, "bits=16", K + N)
    exact, mag = orc.exact_mul_mat(w, x)
    err = orc.metric(y, exact, mag)
    ex16, mag16 = orc.exact_mul_mat(w, rounded(x))
    err16 = orc.metric(y, ex16, mag16)
    _, _, y0 = run_mul_mat(gpu, K, N, M, B, "", K + N)
    print(f"bits=16 mul_mat {K}->{N} x {M}x{B}: {err:.3g} of exact, {err16:.3g} of the rounded products")
    assert err <= K_HALF and err16 <= BOUND_SUM
    assert orc.metric(y0, exact, mag) < err / 10  # the mode takes effect: single precision is far nearer


@pytest.mark.gpu
def test_single_precision_weights_stay_single_under_half(gpu):
    """Single-precision weights have no FP16 form (mul_mat.cc:660-666): they
    stay in the split form under bits=16."""
    r = rng(4)
    w = uniform(r, (100, 77), 0.25)
    x = uniform(r, (300, 77), 1.0)
    y = unwritten((300, 100), gpu)
    sdhip.set_tuning("bits=16")
    try:
        sdhip.mul_mat(dev(w, gpu), dev(x, gpu), y)
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    exact, mag = orc.exact_mul_mat(w, x)
    assert orc.metric(y.cpu().numpy(), exact, mag) <= 2e-6


@pytest.mark.gpu
@pytest.mark.parametrize("K,half,M", [(320, 1280, 200), (96, 2000, 300), (40, 100, 300)])
def test_gated_half(gpu, K, half, M):
    r = rng(K + half + 7)
    wh, w32 = weights_f16(r, (2 * half, K))
    x = uniform(r, (M, K), 1.0)
    bias = uniform(r, (2 * half,), 1.0)
    y = unwritten((M, 2 * half), gpu)
    out = unwritten((M, half), gpu)
    sdhip.set_tuning("bits=16")
    try:
        sdhip.mul_mat_gated(dev(wh, gpu), dev(x, gpu), y, out, sdhip.epilogue([("add", dev(bias, gpu))]))
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    exact, mag = orc.exact_gated(w32, x, bias)
    err = orc.metric(out.cpu().numpy(), exact, mag)
    ex16, mag16 = orc.exact_gated(w32, rounded(x).astype(np.float32), bias)
    print(f"bits=16 gated {K}->2x{half} x {M}: {err:.3g} of exact")
    assert err <= K_HALF
    assert orc.metric(out.cpu().numpy(), ex16, mag16) <= 1e-5


def out_size(i, k, s, p, d):
    return (i + 2 * p - d * (k - 1) - 1) // s + 1


@pytest.mark.gpu
@pytest.mark.parametrize("c,winograd", [
    ((32, 32, 64, 40, 1, 1, 1, 1, 0, 0, 1, 1, 2), False),
    ((33, 33, 24, 30, 3, 3, 2, 2, 1, 1, 1, 1, 1), False),
    ((40, 9, 7, 13, 5, 3, 1, 2, 2, 0, 2, 1, 1), False),
    ((32, 32, 64, 64, 3, 3, 2, 2, 1, 1, 1, 1, 2), False),   # by columns
    ((64, 64, 64, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2), True),
    ((16, 16, 96, 64, 3, 3, 1, 1, 1, 1, 1, 1, 2), True),
], ids=lambda c: "x".join(map(str, c)) if isinstance(c, tuple) else str(c))
def test_conv2d_half(gpu, c, winograd):
    w_, h_, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n = c
    r = rng(sum(c))
    kh16, k32 = weights_f16(r, (oc, ic, kh, kw))
    x = uniform(r, (n, ic, h_, w_), 1.0)
    oh, ow = out_size(h_, kh, s1, p1, d1), out_size(w_, kw, s0, p0, d0)
    y = unwritten((n, oc, oh, ow), gpu)
    params = sdhip.conv_params(s0, s1, p0, p1, d0, d1)
    sdhip.set_tuning("bits=16")
    try:
        sdhip.conv2d(dev(kh16, gpu), dev(x, gpu), y, params)
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    got = y.cpu().numpy()
    exact, mag = orc.exact_conv2d(x, k32, s0, s1, p0, p1, d0, d1)
    err = orc.metric(got, exact, mag)
    print(f"bits=16 conv {c}: {err:.3g} of exact")
    if winograd:
        assert err <= 2e-5  # Winograd's products stay single precision
    else:
        ex16, mag16 = orc.exact_conv2d(rounded(x).astype(np.float32), k32, s0, s1, p0, p1, d0, d1)
        assert err <= K_HALF and orc.metric(got, ex16, mag16) <= BOUND_SUM
        assert err > 1e-5  # rounded to FP16, not split
