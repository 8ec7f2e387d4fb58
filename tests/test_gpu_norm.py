"""GROUP_NORM and NORM with their chains on the device against the oracle's
restatement of norm.cc (the same statistics in the same precisions), and
against float64 for the normalisation itself."""

import numpy as np
import pytest
import torch

import oracle_lib as orc
import sdhip
from helpers import dev, normal, rng, uniform, unwritten

# Fused and apart within 1e-6 of the largest output, as the reference's
# fusion tests hold them (ops_test.cc:567-637); the statistics here are the
# reference's own, so the outputs agree to a few units in the last place.
CLOSE = 1e-6


def chain_ref(y, gamma, beta, silu):
    out = y * gamma
    out = out + beta
    if silu:
        out = orc.silu(out)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("shape,groups,eps,silu", [
    ((2, 64, 20, 36), 32, 1e-6, True),     # ops_test.cc:1062-1075
    ((1, 30, 7, 13), 10, 1e-5, True),      # rows of no multiple of eight
    ((2, 1280, 8, 8), 32, 1e-5, True),     # cfg3a's GroupNorm + SiLU
    ((2, 1280, 32, 32), 32, 1e-5, True),   # cfg3b's
    ((1, 30, 7, 13), 7, 1e-5, False),      # groups of ceil(30/7) = 5 channels, the last of none
    ((1, 128, 128, 128), 32, 1e-6, True),  # groups of many slices
])
def test_group_norm(gpu, shape, groups, eps, silu):
    r = rng(sum(shape) + groups)
    x = uniform(r, shape, 3.0)
    c = shape[1]
    gamma = normal(r, (1, c, 1, 1), 1.0, 0.1)
    beta = normal(r, (1, c, 1, 1), 0.0, 0.1)
    x_d, g_d, b_d = dev(x, gpu), dev(gamma, gpu), dev(beta, gpu)
    y = unwritten(shape, gpu)
    steps = [("mul", g_d), ("add", b_d)] + ([("silu", None)] if silu else [])
    sdhip.group_norm(x_d, y, groups, eps, sdhip.epilogue(steps))
    torch.cuda.synchronize()
    want = chain_ref(orc.group_norm(x, groups, eps), gamma, beta, silu)
    got = y.cpu().numpy()
    assert np.isfinite(got).all()
    diff = np.abs(got - want).max() / np.abs(want).max()
    print(f"group_norm {shape}/{groups}: {diff:.3g} of the largest")
    assert diff <= CLOSE


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(2, 64, 32, 32), (1, 30, 7, 13)])
def test_group_norm_operand_per_position(gpu, shape):
    """A chain operand that varies along the rows (a residual of the output's
    shape, and one broadcast over channels): the per-element path."""
    r = rng(7 + sum(shape))
    x = uniform(r, shape, 2.0)
    res = uniform(r, shape, 1.0)
    rows = uniform(r, (1, 1, shape[2], shape[3]), 1.0)
    x_d, res_d, rows_d = dev(x, gpu), dev(res, gpu), dev(rows, gpu)
    y = unwritten(shape, gpu)
    sdhip.group_norm(x_d, y, 16 if shape[1] % 16 == 0 else 10, 1e-5,
                     sdhip.epilogue([("add", res_d), ("mul", rows_d)]))
    torch.cuda.synchronize()
    want = (orc.group_norm(x, 16 if shape[1] % 16 == 0 else 10, 1e-5) + res) * rows
    got = y.cpu().numpy()
    diff = np.abs(got - want).max() / np.abs(want).max()
    print(f"group_norm per position {shape}: {diff:.3g}")
    assert diff <= CLOSE


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(2, 77, 320), (2, 988, 1280), (3, 5, 33)])
def test_norm(gpu, shape):
    r = rng(sum(shape))
    x = uniform(r, shape, 3.0)
    n = shape[-1]
    gamma = normal(r, (n,), 1.0, 0.1)
    beta = normal(r, (n,), 0.0, 0.1)
    x_d, g_d, b_d = dev(x, gpu), dev(gamma, gpu), dev(beta, gpu)
    y = unwritten(shape, gpu)
    sdhip.norm(x_d, y, 1e-5, sdhip.epilogue([("mul", g_d), ("add", b_d)]))
    torch.cuda.synchronize()
    want = chain_ref(orc.norm(x, 1e-5), gamma, beta, False)
    got = y.cpu().numpy()
    diff = np.abs(got - want).max() / np.abs(want).max()
    print(f"norm {shape}: {diff:.3g} of the largest")
    assert diff <= CLOSE


@pytest.mark.gpu
@pytest.mark.parametrize("shape,view", [((2, 50, 4), False), ((1, 7, 2048), False), ((1, 9, 2052), False),
                                        ((2, 300, 640), True), ((3, 33, 1280), True), ((2, 64, 320), False),
                                        ((1, 7, 128), False), ((2, 33, 200), True), ((2, 65, 320), True),
                                        ((1, 5, 324), True), ((2, 33, 600), False)],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_norm_rows_and_operands(gpu, shape, view):
    """NORM over rows of 4 .. 2048 numbers a float4 at a time (up to 320:
    four rows a wave, 16 lanes each, row counts no multiple of four among
    them; 2052: the general form), the input a view whose rows lie further apart where
    `view`; the chain a per-column scale, a residual of the output's shape
    starting one number past a 16-byte boundary (read a number at a time), a
    per-row scale (broadcast along the row) and the SiLU."""
    r = rng(sum(shape) + view)
    n = shape[-1]
    full = uniform(r, shape[:-1] + (n + 8,), 3.0)
    x = np.ascontiguousarray(full[..., :n])
    gamma = normal(r, (n,), 1.0, 0.1)
    res_full = uniform(r, shape[:-1] + (n + 4,), 1.0)
    res = np.ascontiguousarray(res_full[..., 1:n + 1])
    per_row = normal(r, shape[:-1] + (1,), 1.0, 0.5)
    x_d = dev(full, gpu)[..., :n] if view else dev(x, gpu)
    g_d, pr_d = dev(gamma, gpu), dev(per_row, gpu)
    r_d = dev(res_full, gpu)[..., 1:n + 1]
    y = unwritten(shape, gpu)
    sdhip.norm(x_d, y, 1e-5, sdhip.epilogue([("mul", g_d), ("add", r_d), ("mul", pr_d), ("silu", None)]))
    torch.cuda.synchronize()
    want = orc.silu((orc.norm(x, 1e-5) * gamma + res) * per_row)
    got = y.cpu().numpy()
    diff = np.abs(got - want).max() / np.abs(want).max()
    print(f"norm {shape} view={view}: {diff:.3g} of the largest")
    assert diff <= CLOSE
