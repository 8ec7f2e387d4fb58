"""bits=16, the products of 16 bits (tests/ops_test.cc:304-380, 837-919 with
bits = 16): MUL_MAT, its gated GELU and the direct convolutions of FP16
weights multiply them by their other operand rounded to FP16, one product
each, summed in single precision -- the reference's FP16 format
(cpu.cc:336-366, the split forms' first parts alone); Winograd, attention and
single-precision weights stay single precision, as on the reference's vector
units.  Held to the reference's kHalf = 8e-3 of the exact result, and to
single-precision sums (2e-6) of the products of the rounded operand.

half_format=1, the bfloat16 form (cpu.cc:319-321, attention.cc:309-323):
both operands of those products rounded to bfloat16, and attention's products
of bfloat16 first parts, each held to kHalf of the exact result and to the
float64 products of the bfloat16 operands -- for attention, of the
reference's two-pass softmax, whose exponentials are rounded from
exp(s - max) of the whole row."""

import sys

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


def rounded_bf16(x):
    """x rounded to bfloat16, to nearest with ties to even, as
    vcvtne2ps2bf16 rounds the first parts of half_format=1 (amx.S:181, the
    FP16 weights widened first, amx.S:178)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


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
@pytest.mark.parametrize("K,N,M,B", [(320, 320, 512, 2), (768, 1280, 300, 1), (300, 17, 131, 3), (5120, 1280, 64, 1)])
def test_mul_mat_bfloat16(gpu, K, N, M, B):
    """half_format=1: both operands rounded to bfloat16 (the weights from
    FP16), their products summed in single precision: within kHalf of the
    exact result, and the single-precision sums of the bfloat16 products --
    which the FP16 form is not."""
    w, x, y = run_mul_mat(gpu, K, N, M, B, "bits=16,half_format=1", K + N + 1)
    exact, mag = orc.exact_mul_mat(w, x)
    err = orc.metric(y, exact, mag)
    wb, xb = rounded_bf16(w).astype(np.float32), rounded_bf16(x).astype(np.float32)
    exb, magb = orc.exact_mul_mat(wb, xb)
    errb = orc.metric(y, exb, magb)
    _, _, y16 = run_mul_mat(gpu, K, N, M, B, "bits=16", K + N + 1)
    print(f"bits=16 bfloat16 mul_mat {K}->{N} x {M}x{B}: {err:.3g} of exact, {errb:.3g} of the bfloat16 products")
    assert err <= K_HALF and errb <= BOUND_SUM
    assert orc.metric(y16, exb, magb) > 100 * BOUND_SUM  # the FP16 form's are other products


@pytest.mark.gpu
@pytest.mark.parametrize("K,half,M", [(320, 1280, 200), (40, 100, 300)])
def test_gated_bfloat16(gpu, K, half, M):
    r = rng(K + half + 8)
    wh, w32 = weights_f16(r, (2 * half, K))
    x = uniform(r, (M, K), 1.0)
    bias = uniform(r, (2 * half,), 1.0)
    y = unwritten((M, 2 * half), gpu)
    out = unwritten((M, half), gpu)
    sdhip.set_tuning("bits=16,half_format=1")
    try:
        sdhip.mul_mat_gated(dev(wh, gpu), dev(x, gpu), y, out, sdhip.epilogue([("add", dev(bias, gpu))]))
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    exact, mag = orc.exact_gated(w32, x, bias)
    err = orc.metric(out.cpu().numpy(), exact, mag)
    exb, magb = orc.exact_gated(rounded_bf16(w32).astype(np.float32), rounded_bf16(x).astype(np.float32), bias)
    print(f"bits=16 bfloat16 gated {K}->2x{half} x {M}: {err:.3g} of exact")
    assert err <= K_HALF
    assert orc.metric(out.cpu().numpy(), exb, magb) <= 1e-5


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


@pytest.mark.gpu
@pytest.mark.parametrize("c", [
    (32, 32, 64, 40, 1, 1, 1, 1, 0, 0, 1, 1, 2),
    (33, 33, 24, 30, 3, 3, 2, 2, 1, 1, 1, 1, 1),
    (32, 32, 64, 64, 3, 3, 2, 2, 1, 1, 1, 1, 2),   # by columns
], ids=lambda c: "x".join(map(str, c)))
def test_conv2d_bfloat16(gpu, c):
    """half_format=1 for the direct convolutions: kernels and columns rounded
    to bfloat16, single-precision sums."""
    w_, h_, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n = c
    r = rng(sum(c) + 1)
    kh16, k32 = weights_f16(r, (oc, ic, kh, kw))
    x = uniform(r, (n, ic, h_, w_), 1.0)
    oh, ow = out_size(h_, kh, s1, p1, d1), out_size(w_, kw, s0, p0, d0)
    y = unwritten((n, oc, oh, ow), gpu)
    params = sdhip.conv_params(s0, s1, p0, p1, d0, d1)
    sdhip.set_tuning("bits=16,half_format=1")
    try:
        sdhip.conv2d(dev(kh16, gpu), dev(x, gpu), y, params)
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    got = y.cpu().numpy()
    exact, mag = orc.exact_conv2d(x, k32, s0, s1, p0, p1, d0, d1)
    err = orc.metric(got, exact, mag)
    exb, magb = orc.exact_conv2d(rounded_bf16(x).astype(np.float32), rounded_bf16(k32).astype(np.float32),
                                 s0, s1, p0, p1, d0, d1)
    errb = orc.metric(got, exb, magb)
    print(f"bits=16 bfloat16 conv {c}: {err:.3g} of exact, {errb:.3g} of the bfloat16 products")
    assert err <= K_HALF and errb <= BOUND_SUM


def bf16_attention(q, k, v, scale):
    """Attention of products of bfloat16 first parts, in float64 (numpy): the
    scores of bfloat16 queries and keys, then scaled; the exponentials of the
    two-pass softmax and their sum as they are, rounded to bfloat16 for the
    product by the bfloat16 values (attention.cc:466-589)."""
    b, lq, h, d = q.shape
    _, lk, hk, dv = v.shape
    qb, kb, vb = rounded_bf16(q), rounded_bf16(k), rounded_bf16(v)
    y = np.empty((b, lq, h, dv))
    for bi in range(b):
        for hi in range(h):
            kh = hi // (h // hk)
            s = (qb[bi, :, hi, :] @ kb[bi, :, kh, :].T) * float(np.float32(scale))
            p = np.exp(s - s.max(axis=1, keepdims=True))
            pb = rounded_bf16(p.astype(np.float32))
            y[bi, :, hi, :] = (pb @ vb[bi, :, kh, :]) / p.sum(axis=1, keepdims=True)
    return y


# d, lq, lk, h, hk, b, FP16 keys and values, generic
ATTENTION_BF16 = [
    (40, 300, 1024, 2, 2, 1, False, False),   # the fast form's
    (64, 130, 77, 2, 1, 2, False, False),
    (160, 70, 300, 1, 1, 1, False, False),
    (64, 50, 100, 2, 1, 1, True, False),      # FP16 keys and values: the generic form
    (40, 100, 300, 2, 2, 1, False, True),     # the generic form on the fast form's operands
    (512, 40, 200, 1, 1, 1, False, False),    # the VAE's heads: the wide form
    (384, 65, 130, 2, 1, 2, True, False),     # wide heads sharing FP16 keys and values
    (320, 64, 1000, 1, 1, 1, False, False),   # wide heads over keys the single-precision form splits
    (13, 37, 29, 4, 2, 3, False, False),      # edges: no multiple of a tile, heads sharing keys
    (40, 1, 1, 1, 1, 1, False, False),        # one query, one key
]


@pytest.mark.gpu
@pytest.mark.parametrize("c", ATTENTION_BF16, ids=lambda c: "x".join(map(str, c)))
def test_attention_bfloat16(gpu, c):
    """bits=16 with half_format=1: attention's products of bfloat16 first
    parts, as on the reference's vector units of AVX512-BF16 -- within kHalf of
    the exact result, near the float64 attention of the bfloat16 operands,
    and (unlike the FP16 format, whose attention stays single precision) not
    single precision's."""
    d, lq, lk, h, hk, b, half, generic = c
    r = rng(d + lq + lk + 5)
    q = uniform(r, (b, lq, h, d), 1.0)
    k = uniform(r, (b, lk, hk, d), 1.0)
    v = uniform(r, (b, lk, hk, d), 1.0)
    if half:
        k, v = k.astype(np.float16), v.astype(np.float16)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))

    def run(tuning):
        y = unwritten((b, lq, h, d), gpu)
        qd, kd, vd = dev(q, gpu), dev(k, gpu), dev(v, gpu)
        sdhip.set_tuning(tuning)
        try:
            sdhip.attention(qd.permute(0, 2, 1, 3), kd.permute(0, 2, 1, 3), vd.permute(0, 2, 1, 3), y, scale)
            torch.cuda.synchronize()
        finally:
            sdhip.set_tuning("")
        return y.cpu().numpy()

    extra = ",attention_generic=1" if generic else ""
    y = run("bits=16,half_format=1" + extra)
    k32, v32 = k.astype(np.float32), v.astype(np.float32)
    exact, mag = orc.exact_attention(q, k32, v32, scale)
    err = orc.metric(y, exact, mag)
    errb = orc.metric(y, bf16_attention(q, k32, v32, scale), mag)
    err16 = orc.metric(run("bits=16" + extra), exact, mag)
    print(f"bits=16 bfloat16 attention {c}: {err:.3g} of exact, {errb:.3g} of the bfloat16 products, "
          f"FP16 format {err16:.3g}")
    assert np.isfinite(y).all()
    assert err <= K_HALF and errb <= 1e-4
    assert err16 <= 1e-6 < err / 10


def test_rounded_bf16_pinned():
    """The bfloat16 rounding the checks above take is torch's conversion
    (to nearest, ties to even): on random numbers over many binades, on exact
    ties, which go to the even neighbour, and at the largest finite floats."""
    r = np.random.default_rng(3)
    x = (r.standard_normal(200000) * np.exp2(r.integers(-60, 60, 200000))).astype(np.float32)
    ties = np.array([1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, -(1 + 2.0 ** -8), 2.0 ** -130 * (1 + 2.0 ** -8)], np.float32)
    x = np.concatenate([x, ties, np.array([3.0e38, -3.0e38, 0.0, -0.0], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy().astype(np.float64)
    assert np.array_equal(rounded_bf16(x), ref)
    assert rounded_bf16(ties)[0] == 1.0 and rounded_bf16(ties)[1] == 1 + 2.0 ** -6


def test_bf16_attention_restatement_pinned(monkeypatch):
    """The float64 restatement of attention's bfloat16 products: with its
    roundings taken out it is the exact attention of the oracle (heads
    sharing keys, ragged sizes); with them, within kHalf of it and not
    nearer than the roundings allow."""
    r = np.random.default_rng(4)
    q = r.uniform(-1, 1, (2, 19, 4, 24)).astype(np.float32)
    k = r.uniform(-1, 1, (2, 33, 2, 24)).astype(np.float32)
    v = r.uniform(-1, 1, (2, 33, 2, 24)).astype(np.float32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(24)))
    exact, mag = orc.exact_attention(q, k, v, scale)
    rounded_err = orc.metric(bf16_attention(q, k, v, scale), exact, mag)
    assert 1e-4 < rounded_err <= K_HALF
    monkeypatch.setattr(sys.modules[__name__], "rounded_bf16", lambda x: np.asarray(x, np.float64))
    assert orc.metric(bf16_attention(q, k, v, scale), exact, mag) <= 1e-7
