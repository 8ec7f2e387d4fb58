"""Pins of the oracle, on the CPU.  Each restated function is checked against
something that fixes it independently: a closed form, a library routine of
the textbook case, a brute-force recomputation, or invariants a plausible
mistake (a dropped term, a wrong sign or index, a transposed operand) breaks.
The reference keeps no golden vectors for this path (its tests compare every
form with float64 recomputations, tests/ops_test.cc:154-211)."""

import math

import os

import numpy as np
import pytest
import torch

import oracle_lib as orc
from helpers import anchored, rng, two_valued, uniform, winograd_exact_operands

# ------------------------------------------------------------------ scalar math


def test_exponential_against_exp():
    """scalar_math.h:34-51 is within two units in the last place of exp over
    its range, and clamps beyond it."""
    xs = np.concatenate([np.linspace(-87.0, 88.0, 20001, dtype=np.float32),
                         np.float32([0.0, -0.0, 1e-8, -1e-8, 0.5, -0.5, 10.0, -20.0])])
    L = orc.lib()
    worst = 0.0
    for x in xs:
        got = L.oracle_exponential(float(x))
        want = math.exp(float(x))
        worst = max(worst, abs(got - want) / want)
    assert worst <= 2.5 * 2.0 ** -24
    assert L.oracle_exponential(-1000.0) == pytest.approx(math.exp(-87.3), rel=1e-6)
    assert L.oracle_exponential(0.0) == 1.0


def scalar_sweep():
    """A dense sweep of single-precision arguments: every 61st bit pattern of
    [0, 88.73] with both signs, the clamp edges and their neighbours, points
    past them, and the integers and half-integers of the range."""
    top = np.float32(88.73).view(np.uint32)
    pos = np.arange(0, int(top) + 1, 61, dtype=np.uint32).view(np.float32)
    edges = np.float32([-87.3, 88.73, -87.29999, 88.72999, -87.30001, 88.73001, -88.0, 89.0, -100.0, 100.0,
                        -1e30, 1e30, 0.0, -0.0, 1e-38, -1e-38, 1e-45, -1e-45])
    near = np.concatenate([np.nextafter(edges, np.float32(np.inf)), np.nextafter(edges, np.float32(-np.inf))])
    grid = np.arange(-180, 181, dtype=np.float32) * np.float32(0.5)
    return np.concatenate([pos, -pos, edges, near, grid]).astype(np.float32)


@pytest.mark.skipif(not os.path.exists(orc.REF_SO), reason="oracle/_ref not built: the reference checkout is absent")
@pytest.mark.parametrize("name", ["exponential", "silu", "gelu"])
def test_scalar_math_bit_identical_to_the_reference(name):
    """oracle.c's exponential, SiLU and GELU against the reference's own
    sources/scalar_math.h compiled unmodified (oracle/ref.mk): the same bits
    at every argument of a dense sweep, the clamp edges included.  A changed
    low-order digit of a Cephes coefficient, a dropped reduction step or a
    wrong clamp shows here even where it stays within an ulp of exp.  The
    sweep includes every finite FP16 number times 16, the arguments
    test_gpu_scalar_math.py adds for the device."""
    with np.errstate(invalid="ignore", over="ignore"):
        halves = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32) * 16
    xs = np.concatenate([scalar_sweep(), halves[np.isfinite(halves)]])
    if name == "silu":
        got = orc.silu(xs)
    elif name == "gelu":
        got = orc.gelu(xs)
    else:
        got = orc.exponential(xs)
    want = orc.ref_array(name, xs)
    bad = got.view(np.uint32) != want.view(np.uint32)
    assert not bad.any(), f"{bad.sum()} of {xs.size} differ, first at x = {xs[bad][:5]}"


def test_silu_and_gelu_closed_forms():
    L = orc.lib()
    for x in np.linspace(-10, 10, 401, dtype=np.float32):
        x = float(x)
        assert L.oracle_silu(x) == pytest.approx(x / (1.0 + math.exp(-x)), rel=1e-6, abs=1e-7)
        g = 0.5 * x * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))
        assert L.oracle_gelu(x) == pytest.approx(g, rel=1e-6, abs=1e-7)
    v = uniform(rng(1), (1000,), 8.0)
    assert np.allclose(orc.silu(v), v / (1 + np.exp(-v.astype(np.float64))), rtol=1e-6, atol=1e-7)
    g = uniform(rng(2), (1000,), 6.0)
    want = v * (0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g.astype(np.float64) ** 3))))
    assert np.allclose(orc.gated_gelu(v, g), want, rtol=2e-6, atol=1e-6)

# ------------------------------------------------------------------ float64 references


def test_exact_mul_mat_is_the_matrix_product():
    r = rng(3)
    w = uniform(r, (17, 33), 0.25)
    x = uniform(r, (29, 33), 1.0)
    y, mag = orc.exact_mul_mat(w, x)
    w64, x64 = w.astype(np.float64), x.astype(np.float64)
    assert np.allclose(y, x64 @ w64.T, rtol=0, atol=1e-13)
    assert np.allclose(mag, np.abs(x64) @ np.abs(w64).T, rtol=0, atol=1e-13)


@pytest.mark.parametrize("c", [
    (9, 7, 3, 4, 3, 3, 1, 1, 1, 1, 1, 1, 2),
    (11, 8, 2, 3, 5, 3, 1, 2, 2, 0, 2, 1, 1),
    (10, 10, 4, 2, 1, 1, 1, 1, 0, 0, 1, 1, 2),
    (12, 9, 3, 5, 3, 3, 2, 2, 1, 1, 1, 1, 1),
])
def test_exact_conv2d_is_torch_conv2d(c):
    """ggml's CONV_2D layouts and op_params (s0, s1, p0, p1, d0, d1) against
    torch's float64 conv2d (a cross-correlation, as ggml's is)."""
    w_, h_, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n = c
    r = rng(sum(c))
    x = uniform(r, (n, ic, h_, w_), 1.0)
    k = uniform(r, (oc, ic, kh, kw), 0.25)
    y, mag = orc.exact_conv2d(x, k, s0, s1, p0, p1, d0, d1)
    t = torch.nn.functional.conv2d(torch.from_numpy(x).double(), torch.from_numpy(k).double(), stride=(s1, s0),
                                   padding=(p1, p0), dilation=(d1, d0))
    assert y.shape == tuple(t.shape)
    assert np.allclose(y, t.numpy(), rtol=0, atol=1e-12)
    tm = torch.nn.functional.conv2d(torch.from_numpy(np.abs(x)).double(), torch.from_numpy(np.abs(k)).double(),
                                    stride=(s1, s0), padding=(p1, p0), dilation=(d1, d0))
    assert np.allclose(mag, tm.numpy(), rtol=0, atol=1e-12)
    index = np.array([0, y.size // 3, y.size - 1])
    ys, ms = orc.exact_conv2d(x, k, s0, s1, p0, p1, d0, d1, index=index)
    assert np.array_equal(ys, y.reshape(-1)[index]) and np.array_equal(ms, mag.reshape(-1)[index])


def test_exact_attention_is_softmax():
    """ggml's head layout (q [b][lq][h][d], heads sharing keys h / (h / hk))
    against a float64 softmax written with numpy."""
    r = rng(5)
    b, lq, lk, h, hk, d = 2, 5, 7, 4, 2, 3
    q, k, v = uniform(r, (b, lq, h, d), 1.0), uniform(r, (b, lk, hk, d), 1.0), uniform(r, (b, lk, hk, d), 1.0)
    scale = 0.4
    y, mag = orc.exact_attention(q, k, v, scale)
    for bi in range(b):
        for hi in range(h):
            kh = hi // (h // hk)
            s = q[bi, :, hi, :].astype(np.float64) @ k[bi, :, kh, :].astype(np.float64).T * scale
            p = np.exp(s - s.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            vv = v[bi, :, kh, :].astype(np.float64)
            assert np.allclose(y[bi, :, hi, :], p @ vv, atol=1e-14)
            assert np.allclose(mag[bi, :, hi, :], p @ np.abs(vv), atol=1e-14)
    queries = np.array([0, 7, 39])
    ys, _ = orc.exact_attention(q, k, v, scale, queries=queries)
    for t, qq in enumerate(queries):
        bi, hi, i = qq // (h * lq), (qq // lq) % h, qq % lq
        assert np.array_equal(ys[t], y[bi, i, hi])


def test_exact_gated():
    r = rng(6)
    K, half, M = 9, 4, 3
    w, x, b = uniform(r, (2 * half, K), 0.25), uniform(r, (M, K), 1.0), uniform(r, (2 * half,), 1.0)
    y, _ = orc.exact_gated(w, x, b)
    p = x.astype(np.float64) @ w.astype(np.float64).T + b
    g = p[:, half:]
    gelu = 0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)))
    assert np.allclose(y, p[:, :half] * gelu, atol=1e-13)


def test_winograd_matrices_compute_the_convolution():
    """The F(2x2,3x3) and F(4x4,3x3) matrices of winograd.cc:19-22,
    1155-1183, 1259-1264 (the ones oracle/port.c and the device use) satisfy
    A^T [(G g G^T) * (B^T d B)] A = the 3x3 cross-correlation of d and g."""
    BT4 = np.array([[1, 1.5, -2, -1.5, 1, 0], [0, -1, -2.5, -.5, 1, 0], [0, 1, .5, -2.5, 1, 0],
                    [0, -.5, -1, .5, 1, 0], [0, 2, -1, -2, 1, 0], [0, 1, 1.5, -2, -1.5, 1]])
    G4 = np.array([[1, 0, 0], [-1 / 3, -1 / 3, -1 / 3], [1 / 3, -1 / 3, 1 / 3], [1 / 15, 2 / 15, 4 / 15],
                   [-16 / 15, 8 / 15, -4 / 15], [0, 0, 1]])
    AT4 = np.array([[1, 1, 1, 1, 1, 0], [0, 1, -1, 2, -.5, 0], [0, 1, 1, 4, .25, 0], [0, 1, -1, 8, -.125, 1]])
    BT2 = np.array([[1, 0, -1, 0], [0, 1, 1, 0], [0, -1, 1, 0], [0, 1, 0, -1]])
    G2 = np.array([[1, 0, 0], [.5, .5, .5], [.5, -.5, .5], [0, 0, 1]])
    AT2 = np.array([[1, 1, 1, 0], [0, 1, -1, -1]])
    r = rng(7)
    for BT, G, AT, m in ((BT4, G4, AT4, 4), (BT2, G2, AT2, 2)):
        d = r.standard_normal((m + 2, m + 2))
        g = r.standard_normal((3, 3))
        y = AT @ ((G @ g @ G.T) * (BT @ d @ BT.T)) @ AT.T
        want = np.array([[np.sum(d[i:i + 3, j:j + 3] * g) for j in range(m)] for i in range(m)])
        assert np.allclose(y, want, atol=1e-13)


# ------------------------------------------------------------------ norms


@pytest.mark.parametrize("shape,groups", [((2, 64, 20, 36), 32), ((1, 30, 7, 13), 10), ((1, 30, 7, 13), 7)])
def test_group_norm_against_float64(shape, groups):
    """norm.cc's statistics in single precision agree with float64 group
    normalisation to single precision, groups of ceil(C / G) channels."""
    x = uniform(rng(9), shape, 3.0)
    y = orc.group_norm(x, groups, 1e-5)
    per = -(-shape[1] // groups)
    want = np.empty(shape)
    for b in range(shape[0]):
        for c0 in range(0, shape[1], per):
            blk = x[b, c0:c0 + per].astype(np.float64)
            want[b, c0:c0 + per] = (blk - blk.mean()) / np.sqrt(blk.var() + 1e-5)
    assert np.abs(y - want).max() <= 2e-6 * np.abs(want).max()


def test_norm_against_float64():
    x = uniform(rng(10), (3, 7, 130), 3.0)
    y = orc.norm(x, 1e-5)
    x64 = x.astype(np.float64)
    want = (x64 - x64.mean(-1, keepdims=True)) / np.sqrt(x64.var(-1, keepdims=True) + 1e-5)
    assert np.abs(y - want).max() <= 2e-6 * np.abs(want).max()


def test_apply_chain_broadcasts_as_numpy():
    import ctypes

    L = orc.lib()
    r = rng(11)
    out = uniform(r, (2, 3, 4, 5), 1.0)
    bias = uniform(r, (1, 3, 1, 1), 1.0)
    res = uniform(r, (2, 3, 4, 5), 1.0)
    ne = (ctypes.c_int64 * 4)(5, 4, 3, 2)
    kinds = (ctypes.c_int * 3)(1, 0, 2)
    ops = (ctypes.c_void_p * 3)(bias.ctypes.data, res.ctypes.data, None)
    nb = (ctypes.c_int64 * 12)(0, 0, 1, 0, 1, 5, 20, 60, 0, 0, 0, 0)
    L.oracle_apply_chain.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p]
    got = out.copy()
    L.oracle_apply_chain(got.ctypes.data, ne, 3, kinds, ops, nb)
    want = orc.silu((out * bias + res).astype(np.float32))
    assert np.allclose(got, want, rtol=1e-6, atol=1e-7)

# ------------------------------------------------------------------ bits mode


@pytest.mark.parametrize("levels", [255, 127])
def test_input_quantization_invariants(levels):
    """quant.cc:282-315: bytes in [0, levels]; 0 maps to the zero point
    exactly; the scale is (hi - lo) / levels of the group's range with 0; each
    number is reconstructed within half a step; the tail is the zero point."""
    r = rng(12)
    for trial in range(50):
        n = int(r.integers(1, 64))
        x = uniform(r, (n,), float(r.uniform(0.1, 5.0)))
        if trial % 5 == 0:
            x = np.abs(x)  # all of one sign: the range still holds 0
        x[0] = 0.0
        q, s, o = orc.quantize_input_row(x, 64, levels)
        lo, hi = min(0.0, x.min()), max(0.0, x.max())
        assert s == np.float32(np.float32(hi - lo) / np.float32(levels))
        z = int(q[0])
        assert o == np.float32(s * np.float32(z))
        assert np.all(q[n:] == z)
        assert q.max() <= levels
        recon = s * (q[:n].astype(np.float64) - z)
        assert np.all(np.abs(recon - x) <= 0.5 * s * (1 + 1e-5) + 1e-7)


@pytest.mark.parametrize("levels", [255, 127])
def test_input_quantization_rounds_ties_to_even(levels):
    """quant.cc:282-315 rounds x / s with rint, to the nearest and ties to
    even.  Inputs from 0 up to levels / 128 give the scale 1/128 exactly (a
    power of two) and the zero point 0, so that x = (k + 1/2) / 128 makes
    x inv = k + 1/2 exactly: each such input must land on the even one of k
    and k + 1 -- rounding half away from zero (roundf) lands on k + 1 half of
    the time, truncation on k."""
    step = np.float32(1.0 / 128)
    k = np.arange(0, 62, dtype=np.float32)
    x = np.concatenate([np.float32([0.0, levels / 128.0]), (k + np.float32(0.5)) * step]).astype(np.float32)
    q, s, o = orc.quantize_input_row(x, 64, levels)
    assert s == step and o == 0.0 and q[0] == 0 and q[1] == levels
    want = 2 * np.floor((k + 0.5) / 2 + 0.25).astype(np.int64)  # the even neighbour of k + 1/2
    assert np.array_equal(q[2:2 + k.size].astype(np.int64), want)
    # With a zero point: the range [-z/128, (levels - z)/128] puts z at
    # rint(z) = z, and the ties stay ties after adding it.
    z = 37
    xz = np.concatenate([np.float32([-z / 128.0, (levels - z) / 128.0]),
                         (np.arange(-30, 30, dtype=np.float32) + np.float32(0.5)) * step]).astype(np.float32)
    qz, sz, oz = orc.quantize_input_row(xz, 64, levels)
    assert sz == step and qz[0] == 0 and qz[1] == levels
    t = np.arange(-30, 30) + 0.5
    assert np.array_equal(qz[2:62].astype(np.int64) - z, 2 * np.floor(t / 2 + 0.25).astype(np.int64))


def test_weight_quantization_rounds_ties_to_even():
    """quant.cc:186-243 rounds w / s with rint.  A group whose greatest
    magnitude is 127/64 has the scale 1/64 exactly, so that w = (k + 1/2) / 64
    makes w inv = k + 1/2: ties to even, both signs."""
    k = np.arange(-60, 60, dtype=np.float32)
    w = np.zeros((1, 128), np.float32)
    w[0, 0] = 127.0 / 64
    w[0, 1:1 + 60] = (k[:60] + np.float32(0.5)) / 64
    w[0, 64] = -127.0 / 64
    w[0, 65:125] = (k[60:] + np.float32(0.5)) / 64
    q, sc, of, su = orc.quantize_weights(w, 64, 127, 1)
    assert sc[0, 0] == np.float32(1.0 / 64) and sc[0, 1] == np.float32(1.0 / 64)
    t = k + 0.5
    want = 2 * np.floor(t / 2 + 0.25).astype(np.int64)
    got = np.concatenate([q[0, 1:61], q[0, 65:125]]).astype(np.int64)
    assert np.array_equal(got, want)
    assert q[0, 0] == 127 and q[0, 64] == -127


@pytest.mark.parametrize("weight_groups", [1, 0])
def test_weight_quantization_invariants(weight_groups):
    """quant.cc:186-243: |q| <= wmax, the greatest magnitude of the group (or
    the row) reaching wmax, each weight within half a step, the offset the
    scale times the integer sum."""
    r = rng(13)
    w = uniform(r, (6, 150), 0.25)
    q, s, o, su = orc.quantize_weights(w, 64, 127, weight_groups)
    groups = 3
    assert np.abs(q).max() <= 127
    for row in range(6):
        if not weight_groups:
            assert np.all(s[row] == s[row, 0])
            assert s[row, 0] == np.float32(np.abs(w[row]).max() / np.float32(127))
        for g in range(groups):
            seg = w[row, 64 * g:64 * (g + 1)]
            qs = q[row, 64 * g:64 * g + seg.size].astype(np.int64)
            assert np.all(q[row, 64 * g + seg.size:64 * (g + 1)] == 0)
            assert su[row, g] == qs.sum()
            assert o[row, g] == np.float32(s[row, g] * np.float32(qs.sum()))
            assert np.all(np.abs(s[row, g] * qs - seg) <= 0.5 * s[row, g] * (1 + 1e-5))
            if weight_groups:
                assert np.abs(qs).max() == 127


def test_quantized_product_against_its_own_integers_and_float64():
    """The quantized MUL_MAT: the output agrees with a float64 recomputation
    from the oracle's own bytes, scales and offsets (pins the integer sums,
    their indexing and the dequantisation's signs), and with the exact product
    within the reference's bound kQuantized = 1e-2 (ops_test.cc:213-223)."""
    r = rng(14)
    N, K, M = 9, 150, 7
    w = uniform(r, (N, K), 0.25).astype(np.float16).astype(np.float32)
    x = uniform(r, (M, K), 1.0)
    y, xq, xs, xo, wq, ws, wo, wsum = orc.quantized_mul_mat(w, x)
    groups = 3
    S = np.einsum("mgk,ngk->mng", xq.reshape(M, groups, 64).astype(np.int64),
                  wq.reshape(N, groups, 64).astype(np.int64))
    recon = (xs[:, None, :] * ws[None, :, :] * S - xo[:, None, :] * wo[None, :, :]).sum(-1)
    assert np.allclose(y, recon, rtol=1e-5, atol=1e-5)
    exact, mag = orc.exact_mul_mat(w, x)
    assert orc.metric(y, exact, mag) <= 1e-2
    init = uniform(r, (M, N), 1.0)
    y2 = orc.quantized_mul_mat(w, x, init=init)[0]
    assert np.allclose(y2, y + init, atol=1e-5)


# ------------------------------------------------------------------ quantized attention

K_QUANTIZED = 1e-2  # tests/ops_test.cc:221


def quantized_bound(levels, wmax):
    """The reference's bound for a quantized form against float64
    (ops_test.cc:213-240): kQuantized scaled by (2/L + 1/W)."""
    return K_QUANTIZED * (2.0 / levels + 1.0 / wmax) / (2.0 / 255 + 1.0 / 127)


@pytest.mark.parametrize("c,levels,wmax", [
    ((40, 120, 700, 2, 2, 1), 255, 127),
    ((13, 37, 290, 4, 2, 3), 255, 127),    # the reference's edge case (ops_test.cc:920)
    ((80, 60, 1024, 2, 1, 1), 255, 127),
    ((40, 50, 500, 2, 2, 1), 255, 63),     # weights of 7 bits
    ((40, 50, 500, 2, 2, 1), 127, 127),    # inputs of 7 bits
])
def test_quantized_attention_within_the_reference_bound(c, levels, wmax):
    """The bits-mode self-attention against the float64 softmax, by the
    reference's metric and its own bound for quantized forms."""
    d, lq, lk, h, hk, b = c
    r = rng(d + lk)
    q, k, v = (uniform(r, (b, n, hh, d), 1.0) for n, hh in ((lq, h), (lk, hk), (lk, hk)))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    y = orc.quantized_attention(q, k, v, scale, input_levels=levels, weight_max=wmax)
    exact, mag = orc.exact_attention(q, k, v, scale)
    err = orc.metric(y, exact, mag)
    assert err <= quantized_bound(levels, wmax), err
    assert err > 1e-5  # quantized, not single precision


def test_quantized_attention_groups_exactly():
    """Keys of zeros make every score 0 and every exponential 1, so each
    output is the mean of the dequantized values; values that are integers
    times a power of two per (dimension, group of 64 keys), with +-127 of them
    in each group, dequantize exactly.  The output is then the plain mean to
    single-precision rounding: a group misplaced against the stretches or the
    keys, a wrong scale or offset, or a dropped term would be off by a step
    of a byte."""
    b, lq, h, d, lk = 1, 5, 2, 16, 300
    r = rng(11)
    q = uniform(r, (b, lq, h, d), 1.0)
    k = np.zeros((b, lk, h, d), np.float32)
    ints = r.integers(-127, 128, size=(b, lk, h, d)).astype(np.float32)
    ints[:, ::64] = 127.0  # each group's greatest
    powers = np.float32(2.0) ** -r.integers(0, 12, size=((lk + 63) // 64, h, d)).astype(np.float32)
    v = ints * np.repeat(powers, 64, axis=0)[None, :lk]
    y = orc.quantized_attention(q, k, v.astype(np.float32), 0.25)
    mean = v.astype(np.float64).mean(axis=1)  # [b, h, d]
    want = np.broadcast_to(mean[:, None], y.shape)
    assert np.max(np.abs(y - want) / np.abs(v).max()) < 1e-6


# ------------------------------------------------------------------ quantized convolutions, exactly


EXACT_BAR = 1e-6   # single-precision roundings of the dequantised sums only
OFF_BAR = 1e-4     # a grouping mistake misquantizes a fraction of the weights by up to half a step


@pytest.mark.parametrize("kernel", [3, 1])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("weight_groups", [1, 0])
def test_quantized_conv2d_groups_exactly(kernel, group, weight_groups):
    """The bits-mode direct convolution (conv2d.cc:338-483) on operands that
    quantize exactly where the reference puts its groups: the kernels'
    groups of `group` consecutive k = ic KH KW + kh KW + kw (conv2d.cc:255-258)
    of an output channel, or its whole row with weight_group=0 (quant.cc:
    186-243), each an integer multiple of its own power of two with one +-127
    of it.  The result is then float64's to single-precision rounding; the
    same operands under the columns in another order (planted: tap-major), or
    under groups of half or twice the length, are off by a step of a byte."""
    r = rng(1000 * kernel + group + weight_groups)
    n, ic, h, w, oc = 2, 29 if kernel == 3 else 150, 9, 11, 6
    K = ic * kernel * kernel
    spans = [(0, K)] if weight_groups == 0 else [(g, min(g + group, K)) for g in range(0, K, group)]
    wts = anchored(r, oc, K, spans).reshape(oc, ic, kernel, kernel)
    assert np.array_equal(wts.astype(np.float16).astype(np.float32), wts)
    x = two_valued(r, (n, ic, h, w))
    pad = kernel // 2
    p = (1, 1, pad, pad, 1, 1)
    exact, mag = orc.exact_conv2d(x, wts, *p)

    def err(**kw):
        return orc.metric(orc.quantized_conv2d(x, wts, *p, group=kw.pop("g", group), weight_groups=kw.pop(
            "wg", weight_groups)), exact, mag)

    assert err() <= EXACT_BAR
    if kernel == 3 and weight_groups == 1:
        # With one scale per whole row the order of k is not observable.
        with orc.planted(1):
            assert err() > OFF_BAR
    if weight_groups == 1:
        assert err(g=group // 2) > OFF_BAR
        assert err(g=group * 2) > OFF_BAR
    else:
        assert err(wg=1) > OFF_BAR   # per group where the reference takes the whole row


def stretch_for(group, ic, small):
    """The stretch of input channels over which the bits mode quantizes
    Winograd's weights at a time: max(group, kc rounded down to the group),
    kc = min(ic, max(8, winograd_small_kc = 128)) for small images and
    min(ic, winograd_kc = 256) for large (winograd.cc:238-255, 1859-1866)."""
    kc = min(ic, 128) if small else min(ic, 256)
    return max(group, kc // group * group)


@pytest.mark.parametrize("size", ["small", "large"])
@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("weight_groups", [0, 1])
def test_quantized_winograd2_groups_exactly(size, group, weight_groups):
    """The bits-mode F(2x2) (winograd.cc:1826-2103) on operands whose
    transforms quantize exactly where the reference puts its scales:
    * inputs d_c = k_c 2^(b_g) D, D one small-integer image for every
      channel, k_c in [0, 255] with one 255 in each group g of input
      channels, b_g the group's: each (tile, group, point) of V = B^T d B is
      k_c 2^(b_g) times one integer, exact at the group's scale and zero point;
    * kernels, per output channel and stretch of input channels
      (weight_group=0) or group (1), 4 k 2^e with |k| <= 14 except one anchor
      channel of +-127 2^e at the four corners, whose G g G^T is +-127 2^e at
      all sixteen points (G (1, 0, 1)^T = (1, 1, 1, 1)^T): every point's
      greatest |U| is 127 2^e, the others multiples of 2^e below it.
    IC = 320 is above the stretch, so that the weights' scale changes between
    stretches.  The result is float64's to single-precision rounding; the
    weights over every input channel at once, or over stretches of one group
    (both planted), or groups of another length, are off by a step."""
    r = rng(7 * group + weight_groups + (0 if size == "small" else 1))
    n, h, w = (1, 8, 10) if size == "small" else (2, 40, 40)  # 1600 positions an image: Winograd, not small
    ic, oc = 320, 5
    tiles = n * ((h + 1) // 2) * ((w + 1) // 2)
    assert (tiles <= 256) == (size == "small")  # winograd_small_tiles (winograd.cc:194-196)
    stretch = stretch_for(group, ic, size == "small")
    assert stretch < ic
    spans = ([(s, min(s + stretch, ic)) for s in range(0, ic, stretch)] if weight_groups == 0
             else [(g, min(g + group, ic)) for g in range(0, ic, group)])
    x, wts = winograd_exact_operands(r, (n, ic, h, w), oc, group, spans)
    exact, mag = orc.exact_conv2d(x, wts, 1, 1, 1, 1, 1, 1)

    def err(g=group, wg=weight_groups, st=stretch):
        return orc.metric(orc.quantized_winograd2(x, wts, 1, 1, g, weight_groups=wg, stretch=st), exact, mag)

    assert err() <= EXACT_BAR
    if weight_groups == 0:
        with orc.planted(2):
            assert err() > OFF_BAR
        if stretch > group:
            with orc.planted(3):
                assert err() > OFF_BAR
    else:
        assert err(g=group // 2, st=stretch_for(group // 2, ic, size == "small")) > OFF_BAR
        if group * 2 <= 128:
            assert err(g=group * 2, st=stretch_for(group * 2, ic, size == "small")) > OFF_BAR
