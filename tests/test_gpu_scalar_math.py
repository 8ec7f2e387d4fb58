"""The device's exponential, SiLU and GELU (csrc/device.h) against the
oracle's oracle_silu / oracle_gelu, bit for bit over a dense sweep of
arguments, the clamp edges included.  The oracle's functions are themselves
held bit-identical, over the same sweep, to the reference's own
sources/scalar_math.h compiled unmodified into oracle/_ref (test_oracle.py,
in the build container): the device meets the reference's bits without
anything built from the reference being loaded on the GPU box.

The device functions are reached through the C ABI: a MUL_MAT by the identity
returns its input exactly where the input's split into two FP16 parts is exact
(csrc/device.h, split2: x 2^-4 = hi + lo with both parts normal), so that
the chain's SILU step sees x itself, and the gated GELU of a product by two
identities gives x GELU(x).  The sweep keeps the arguments whose split is
exact, checked here on the host."""

import numpy as np
import pytest
import torch

import oracle_lib as orc
import sdhip
from helpers import dev, unwritten
from test_oracle import scalar_sweep

K = 16


def exact_split(x):
    """The arguments x whose x 2^-4 is exactly hi + lo, both FP16 parts normal
    or zero, and within FP16's range."""
    x = x[np.isfinite(x) & (np.abs(x) < 65504.0 * 16)]
    s = x * np.float32(0.0625)
    hi = s.astype(np.float16).astype(np.float32)
    lo = (s - hi).astype(np.float16).astype(np.float32)
    # The parts give back x itself (not a flushed x 2^-4), and x is no -0:
    # the product's sum of +0 and -0 terms is +0 whatever x's sign.
    ok = (hi.astype(np.float64) + lo.astype(np.float64)) * 16.0 == x.astype(np.float64)
    ok &= ~((x == 0) & np.signbit(x))
    ok &= (lo == 0) | (np.abs(lo) >= 2.0 ** -14)
    ok &= (hi == 0) | (np.abs(hi) >= 2.0 ** -14)
    return x[ok]


def arguments():
    # And every FP16 number times 16 (its split is itself and 0): the small
    # arguments, down to 2^-10, densely.
    with np.errstate(invalid="ignore", over="ignore"):
        halves = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32) * 16
    xs = exact_split(np.concatenate([scalar_sweep(), halves]))
    # Arguments of SiLU and GELU of a few hundred units in magnitude, then
    # rows of K.
    xs = xs[np.abs(xs) <= 200.0]
    n = xs.size // K * K
    return xs[:n].reshape(-1, K)


@pytest.mark.gpu
def test_device_silu_bit_identical_to_the_reference(gpu):
    x = arguments()
    eye = np.eye(K, dtype=np.float16)
    y = unwritten(x.shape, gpu)
    sdhip.mul_mat(dev(eye, gpu), dev(x, gpu), y, sdhip.epilogue([("silu", None)]))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = orc.silu(x)
    bad = got.view(np.uint32) != want.view(np.uint32)
    print(f"SiLU of {x.size} arguments, {bad.sum()} differ")
    assert not bad.any(), f"first at x = {x[bad][:5]}: {got[bad][:5]} against {want[bad][:5]}"


@pytest.mark.gpu
def test_device_gelu_bit_identical_to_the_reference(gpu):
    x = arguments()
    eye2 = np.concatenate([np.eye(K, dtype=np.float16)] * 2)
    y = unwritten((x.shape[0], 2 * K), gpu)
    out = unwritten(x.shape, gpu)
    sdhip.mul_mat_gated(dev(eye2, gpu), dev(x, gpu), y, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = (x * orc.gelu(x)).astype(np.float32)  # out = x GELU(gate), one rounding
    bad = got.view(np.uint32) != want.view(np.uint32)
    print(f"x GELU(x) of {x.size} arguments, {bad.sum()} differ")
    assert not bad.any(), f"first at x = {x[bad][:5]}: {got[bad][:5]} against {want[bad][:5]}"
