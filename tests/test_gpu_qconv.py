"""CONV_2D in the bits mode (quantize & 2) on the device: the direct
convolution's products quantized (conv2d.cc:338-483) and Winograd's F(2x2)
with quantized products for every convolution Winograd takes
(winograd.cc:1826-2103, 2230-2244), at the reference's quantized cases
(tests/ops_test.cc:843-853, 895-905).  Bit for bit with the oracle's
restatement -- the columns' and transformed operands' bytes, scales and
offsets, the exact integer sums, the dequantisation's fused multiply-adds in
the reference's order, the transforms' single-precision roundings -- and
within the reference's bound for quantized forms against float64."""

import numpy as np
import pytest
import torch

import oracle_lib as orc
import sdhip
from helpers import anchored, dev, rng, two_valued, uniform, unwritten, weights_f16, winograd_exact_operands
from test_gpu_quant import bound, quant_params

# w, h, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n, single-precision kernel
CASES = [
    (64, 64, 64, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2, False),
    (16, 16, 96, 64, 3, 3, 1, 1, 1, 1, 1, 1, 2, False),
    (8, 8, 96, 64, 3, 3, 1, 1, 1, 1, 1, 1, 2, False),
    (32, 32, 64, 40, 1, 1, 1, 1, 0, 0, 1, 1, 2, False),
    (33, 33, 24, 30, 3, 3, 2, 2, 1, 1, 1, 1, 1, False),
    (17, 13, 5, 7, 3, 3, 1, 1, 1, 1, 1, 1, 3, True),
    (65, 33, 24, 20, 3, 3, 1, 1, 1, 1, 1, 1, 2, False),
    (64, 20, 13, 11, 3, 3, 1, 1, 0, 0, 1, 1, 1, False),
    (96, 16, 32, 17, 3, 3, 1, 1, 1, 1, 1, 1, 1, True),
    (40, 9, 7, 13, 5, 3, 1, 2, 2, 0, 2, 1, 1, True),   # direct, 5x3, strides and dilations (ops_test.cc:810)
]


def out_size(i, k, s, p, d):
    return (i + 2 * p - d * (k - 1) - 1) // s + 1


def stretch_of(tuning, ic, n, oh, ow):
    """The stretch of input channels the reference quantizes Winograd's
    weights over at a time (winograd.cc:1859-1866, 236-266)."""
    t = dict(kv.split("=") for kv in tuning.split(",") if kv)
    group = quant_params(tuning)[0]
    small = n * ((ow + 1) // 2) * ((oh + 1) // 2) <= int(t.get("winograd_small_tiles", 256))
    want = max(8, int(t.get("winograd_small_kc", 128))) if small else int(t.get("winograd_kc", 256))
    return max(group, min(ic, want) // group * group)


def run(gpu, c, tuning, seed, residual=None, bias=True):
    w_, h_, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n, f32 = c
    r = rng(seed)
    kh16, k32 = weights_f16(r, (oc, ic, kh, kw))
    if f32:
        k32 = (k32 + uniform(r, k32.shape, 2.0 ** -14)).astype(np.float32)
    x = uniform(r, (n, ic, h_, w_), 1.0)
    b = uniform(r, (1, oc, 1, 1), 1.0)
    oh, ow = out_size(h_, kh, s1, p1, d1), out_size(w_, kw, s0, p0, d0)
    k_d = dev(k32 if f32 else kh16, gpu)
    x_d, b_d = dev(x, gpu), dev(b, gpu)
    y_d = unwritten((n, oc, oh, ow), gpu)
    steps = [("add", b_d)] if bias else []
    params = sdhip.conv_params(s0, s1, p0, p1, d0, d1)
    sdhip.set_tuning(tuning)
    try:
        path = sdhip.conv2d_path(k_d, x_d, y_d, params)
        if residual is not None:
            out = dev(residual, gpu)
            sdhip.conv2d(k_d, x_d, y_d, params, sdhip.epilogue(steps, redirect=out, from_redirect=True))
        else:
            out = y_d
            sdhip.conv2d(k_d, x_d, y_d, params, sdhip.epilogue(steps))
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    return x, k32, b, out.cpu().numpy(), path, (s0, s1, p0, p1, d0, d1), (oh, ow)


def want_of(tuning, c, x, k32, p, path, oh, ow, residual=None):
    group, levels, wmax, wg = quant_params(tuning)
    s0, s1, p0, p1, d0, d1 = p
    if path == 2:
        return orc.quantized_winograd2(x, k32, p0, p1, group, levels, wmax, wg,
                                       stretch_of(tuning, c[2], c[12], oh, ow), init=residual)
    return orc.quantized_conv2d(x, k32, s0, s1, p0, p1, d0, d1, group, levels, wmax, wg, init=residual)


@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES, ids=lambda c: "x".join(map(str, c[:13])) + ("_f32" if c[13] else ""))
@pytest.mark.parametrize("tuning", ["bits=8", "bits=8,weight_group=0", "bits=8,group=32", "bits=7",
                                    "bits=8,input_bits=7"])
def test_quantized_conv2d(gpu, c, tuning):
    x, k32, b, got, path, p, (oh, ow) = run(gpu, c, tuning, seed=sum(c[:13]) + len(tuning))
    is_winograd = c[4] == 3 and c[5] == 3 and p[:2] == (1, 1) and p[4:] == (1, 1)
    assert path == (2 if is_winograd else 0)
    want = (want_of(tuning, c, x, k32, p, path, oh, ow) + b).astype(np.float32)
    same = np.array_equal(got.view(np.uint32), want.view(np.uint32))
    exact, mag = orc.exact_conv2d(x, k32, *p)
    err = orc.metric(got, exact + b, mag + np.abs(b))
    _, levels, wmax, _ = quant_params(tuning)
    print(f"quantized conv {c} path {path} [{tuning}]: error {err:.3g}, bit-exact with the oracle: {same}")
    assert same, f"{np.sum(got != want)} of {got.size} differ"
    assert err <= bound(levels, wmax)


@pytest.mark.gpu
@pytest.mark.parametrize("c", [CASES[0], CASES[3], CASES[8]], ids=lambda c: "x".join(map(str, c[:13])))
def test_quantized_conv2d_from_redirect(gpu, c):
    """The residual already in the output's memory: the direct form begins
    its quantized sums from it (conv2d.cc:466-468), Winograd adds its
    outputs to it (winograd.cc:509-623, add)."""
    w_, h_, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n, f32 = c
    oh, ow = out_size(h_, kh, s1, p1, d1), out_size(w_, kw, s0, p0, d0)
    res = uniform(rng(99), (n, oc, oh, ow), 1.0)
    x, k32, b, got, path, p, _ = run(gpu, c, "bits=8", seed=5, residual=res)
    want = (want_of("bits=8", c, x, k32, p, path, oh, ow, residual=res) + b).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_quantized_winograd_oracle_against_float64():
    """The oracle's restatements of the bits-mode F(2x2) (winograd.cc:1826-2103)
    and direct form on ordinary operands: within the reference's bound for
    quantized forms of float64, and quantized (not single-precision-close).
    This bound does not see where the groups and stretches lie (groups of 32
    in place of 64 would pass it); test_oracle.py's exact constructions do.
    CPU only."""
    r = rng(3)
    x = uniform(r, (2, 24, 10, 12), 1.0)
    w = uniform(r, (16, 24, 3, 3), 0.25)
    exact, mag = orc.exact_conv2d(x, w, 1, 1, 1, 1, 1, 1)
    yw = orc.quantized_winograd2(x, w, 1, 1)
    yd = orc.quantized_conv2d(x, w, 1, 1, 1, 1, 1, 1)
    for y in (yw, yd):
        err = orc.metric(y, exact, mag)
        assert 1e-5 < err <= bound(255, 127), err


@pytest.mark.gpu
@pytest.mark.parametrize("tuning", ["bits=8,weight_group=0", "bits=8", "bits=8,group=32", "bits=8,group=128"])
@pytest.mark.parametrize("form", ["winograd_small", "winograd_large", "direct3", "direct1"])
def test_quantized_conv2d_exact_operands(gpu, form, tuning):
    """The device on operands that quantize exactly where the reference puts
    its groups and stretches (tests/helpers.py: anchored kernels, two-valued
    or per-group-scaled inputs): bit for bit with the oracle, and float64's
    result to single-precision rounding -- the device's groups, stretches and
    column order are the reference's, not merely the oracle's."""
    group, levels, wmax, wg = quant_params(tuning)
    r = rng(len(tuning) + len(form))
    if form.startswith("winograd"):
        n, h, w = (1, 8, 10) if form == "winograd_small" else (2, 40, 40)
        ic, oc, kk = 320, 24, 3
        stretch = stretch_of(tuning, ic, n, h, w)
        spans = ([(s, min(s + stretch, ic)) for s in range(0, ic, stretch)] if wg == 0
                 else [(g, min(g + group, ic)) for g in range(0, ic, group)])
        x, k32 = winograd_exact_operands(r, (n, ic, h, w), oc, group, spans)
    else:
        kk = 3 if form == "direct3" else 1
        n, h, w, oc = 2, 9, 11, 24
        ic = 29 if kk == 3 else 150
        K = ic * kk * kk
        spans = [(0, K)] if wg == 0 else [(g, min(g + group, K)) for g in range(0, K, group)]
        k32 = anchored(r, oc, K, spans).reshape(oc, ic, kk, kk)
        x = two_valued(r, (n, ic, h, w))
    pad = kk // 2
    st = 2 if form == "direct3" else 1  # a stride of 2: the bits mode takes every 3x3 of stride 1 by F(2x2)
    p = (st, st, pad, pad, 1, 1)
    oh, ow = out_size(h, kk, st, pad, 1), out_size(w, kk, st, pad, 1)
    k_d, x_d = dev(k32.astype(np.float16), gpu), dev(x, gpu)
    y_d = unwritten((n, oc, oh, ow), gpu)
    params = sdhip.conv_params(*p)
    sdhip.set_tuning(tuning)
    try:
        path = sdhip.conv2d_path(k_d, x_d, y_d, params)
        sdhip.conv2d(k_d, x_d, y_d, params, sdhip.epilogue([]))
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    assert path == (2 if form.startswith("winograd") else 0)
    got = y_d.cpu().numpy()
    want = (orc.quantized_winograd2(x, k32, pad, pad, group, levels, wmax, wg, stretch_of(tuning, ic, n, oh, ow))
            if path == 2 else orc.quantized_conv2d(x, k32, *p, group, levels, wmax, wg))
    exact, mag = orc.exact_conv2d(x, k32, *p)
    err = orc.metric(got, exact, mag)
    print(f"exact operands {form} [{tuning}] path {path}: error {err:.3g}")
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert err <= 1e-6
