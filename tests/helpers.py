"""Inputs as the reference's tests make them (tests/ops_test.cc:61-78):
uniform in [-0.25, 0.25] for weights (rounded to FP16) and [-1, 1] for the
rest -- from numpy's generator with a seed per case, not mt19937."""

import numpy as np
import torch

KUNWRITTEN = float("nan")


def rng(seed):
    return np.random.default_rng(seed)


def uniform(r, shape, scale):
    return r.uniform(-scale, scale, size=shape).astype(np.float32)


def weights_f16(r, shape, scale=0.25):
    """FP16 weights and their exact widening to float32."""
    h = uniform(r, shape, scale).astype(np.float16)
    return h, h.astype(np.float32)


def normal(r, shape, mean=0.0, std=1.0):
    return (mean + std * r.standard_normal(size=shape)).astype(np.float32)


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def unwritten(shape, device):
    return torch.full(shape, KUNWRITTEN, dtype=torch.float32, device=device)


# ------------------------------------------------------------------ exactly quantizable operands


def two_valued(r, shape, z0=100, b=-6):
    """Inputs of two values, -z0 2^b and (255 - z0) 2^b.  A group of columns
    holding both quantizes with scale 2^b and zero point z0 exactly; one
    holding either alone (or with the padding's zeros) to within a rounding of
    its scale: whatever the grouping, the inputs are exact, so that the
    weights' grouping alone decides the error."""
    lo, hi = -z0 * 2.0 ** b, (255 - z0) * 2.0 ** b
    return np.where(r.random(shape) < 0.5, lo, hi).astype(np.float32)


def anchored(r, rows, k, spans):
    """Weights [rows][k], FP16-exact, that quantize exactly at the given spans
    of k (each a (begin, end) the reference gives one scale): each (row,
    span) integers in [-126, 126] times its own power of two 2^e, one of them
    +-127 2^e at a random place, e differing between neighbouring spans."""
    w = np.empty((rows, k), np.float32)
    for o in range(rows):
        for i, (a, b) in enumerate(spans):
            e = -5 - (o + i) % 4
            ints = r.integers(-126, 127, size=b - a).astype(np.float32)
            ints[r.integers(0, b - a)] = 127.0 * r.choice([-1.0, 1.0])
            w[o, a:b] = ints * np.float32(2.0 ** e)
    return w


def winograd_exact_operands(r, shape, oc, group, spans):
    """Inputs [n, ic, h, w] and FP16-exact 3x3 kernels [oc, ic, 3, 3] whose
    F(2x2) transforms quantize exactly where the reference puts its scales:
    * d_c = k_c 2^(b_g) D, D one small-integer image for every channel, k_c
      in [0, 255] with one 255 in each group g of `group` input channels, b_g
      the group's: each (tile, group, point) of V = B^T d B is k_c 2^(b_g)
      times one integer, exact at the group's scale and zero point;
    * per output channel and span of input channels (the stretch or group
      that gets one scale), kernels 4 k 2^e with |k| <= 14 except one anchor
      channel of +-127 2^e at the four corners, whose G g G^T is +-127 2^e at
      all sixteen points (G (1, 0, 1)^T = (1, 1, 1, 1)^T): every point's
      greatest |U| is 127 2^e, the others multiples of 2^e below it."""
    n, ic, h, w = shape
    base = r.integers(-4, 5, size=(n, 1, h, w)).astype(np.float32)
    k = r.integers(0, 255, size=ic).astype(np.float32)
    powers = np.empty(ic, np.float32)
    for g0 in range(0, ic, group):
        k[g0 + r.integers(0, min(group, ic - g0))] = 255.0
        powers[g0:g0 + group] = 2.0 ** ((g0 // group) % 3 - 1)
    x = (base * (k * powers)[None, :, None, None]).astype(np.float32)
    wts = np.empty((oc, ic, 3, 3), np.float32)
    for o in range(oc):
        for i, (a, b) in enumerate(spans):
            e = np.float32(2.0 ** (-5 - (o + i) % 4))
            wts[o, a:b] = 4.0 * r.integers(-14, 15, size=(b - a, 3, 3)) * e
            anchor = a + r.integers(0, b - a)
            wts[o, anchor] = 0.0
            wts[o, anchor, ::2, ::2] = 127.0 * e * r.choice([-1.0, 1.0])
    assert np.array_equal(wts.astype(np.float16).astype(np.float32), wts)
    return x, wts
