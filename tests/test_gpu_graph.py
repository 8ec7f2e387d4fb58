"""Graphs computed through sdhip_compute_nodes on the device, fused and apart
(tests/ops_test.cc:596-637): each of the reference's fusion cases
(ops_test.cc:952-1117) computed with fuse=1 -- the chain, residual redirect
and gated GELU inside the library's kernels -- and with fuse=0 -- the library
computing the operation alone and the chain's nodes computed as ggml would,
node by node -- must agree within the reference's 1e-6 of the largest output.
And the entry points' own apart form (a chain handed to an entry point under
fuse=0 or fuse_residual=0, computed in a pass after the operation) against the
fused form."""

import numpy as np
import pytest
import torch

import graph_lib as gl
import oracle_lib as orc
import sdhip
from helpers import dev, rng, uniform, weights_f16


def leaf_f16(g, r, shape):
    return g.leaf(torch.from_numpy(weights_f16(r, shape)[0]))


def leaf_f32(g, r, shape, scale=1.0):
    return g.leaf(torch.from_numpy(uniform(r, shape, scale)))


def conv_case(g, r, ic, oc, w_, h_, n, k, pad, bias=True):
    wt = leaf_f16(g, r, (oc, ic, k, k))
    x = leaf_f32(g, r, (n, ic, h_, w_))
    y = g.conv2d(wt, x, 1, 1, pad, pad, 1, 1)
    if not bias:
        return y
    b = leaf_f32(g, r, (oc,))
    return g.add_inplace(y, g.reshape(b, (1, oc, 1, 1)))


def case(name, g, r):
    if name == "conv2d, bias":
        return conv_case(g, r, 24, 40, 40, 36, 2, 3, 1)
    if name == "conv2d 1x1, bias, scale per image":
        return g.mul_inplace(conv_case(g, r, 16, 20, 17, 9, 2, 1, 0), leaf_f32(g, r, (2, 20, 1, 1)))
    if name == "conv2d by Winograd, bias, residual":
        return g.add_inplace(conv_case(g, r, 16, 24, 66, 40, 1, 3, 1), leaf_f32(g, r, (1, 24, 40, 66)))
    if name == "conv2d, bias, residual not in place":
        return g.add(conv_case(g, r, 24, 40, 40, 36, 2, 3, 1), leaf_f32(g, r, (2, 40, 36, 40)))
    if name == "conv2d of small images by Winograd, residual on the left":
        res = leaf_f32(g, r, (2, 48, 16, 16))
        return g.add(res, conv_case(g, r, 64, 48, 16, 16, 2, 3, 1, bias=False))
    if name == "linear, bias, residual not in place":
        w, x, b = leaf_f16(g, r, (70, 96)), leaf_f32(g, r, (2, 50, 96)), leaf_f32(g, r, (70,))
        return g.add(g.add_inplace(g.mul_mat(w, x), b), leaf_f32(g, r, (2, 50, 70)))
    if name == "conv2d, bias, residual in its own memory":
        res = g.dup(leaf_f32(g, r, (2, 40, 36, 40)))
        return g.add_inplace(res, conv_case(g, r, 96, 40, 40, 36, 2, 1, 0))
    if name == "conv2d by Winograd, residual in its own memory":
        res = g.dup(leaf_f32(g, r, (1, 24, 40, 66)))
        return g.add_inplace(res, conv_case(g, r, 16, 24, 66, 40, 1, 3, 1))
    if name == "conv2d of small images by Winograd, residual in its own memory":
        res = g.dup(leaf_f32(g, r, (2, 48, 9, 15)))
        return g.add_inplace(res, conv_case(g, r, 64, 48, 15, 9, 2, 3, 1, bias=False))
    if name == "linear, bias, residual in its own memory":
        w, x, b = leaf_f16(g, r, (70, 300)), leaf_f32(g, r, (2, 1100, 300)), leaf_f32(g, r, (70,))
        res = g.dup(leaf_f32(g, r, (2, 1100, 70)))
        return g.add_inplace(res, g.add_inplace(g.mul_mat(w, x), b))
    if name == "linear, bias":
        w, x, b = leaf_f16(g, r, (70, 96)), leaf_f32(g, r, (2, 50, 96)), leaf_f32(g, r, (70,))
        return g.add_inplace(g.mul_mat(w, x), b)
    if name == "group norm, scale, shift, SiLU":
        x = leaf_f32(g, r, (2, 64, 20, 36), 3.0)
        y = g.group_norm(x, 32, 1e-6)
        y = g.mul_inplace(y, leaf_f32(g, r, (1, 64, 1, 1)))
        return g.silu_inplace(g.add_inplace(y, leaf_f32(g, r, (1, 64, 1, 1))))
    if name == "group norm of rows of no multiple of eight, scale, shift":
        x = leaf_f32(g, r, (1, 30, 7, 13), 3.0)
        y = g.group_norm(x, 10, 1e-5)
        y = g.mul_inplace(y, leaf_f32(g, r, (1, 30, 1, 1)))
        return g.silu_inplace(g.add_inplace(y, leaf_f32(g, r, (1, 30, 1, 1))))
    if name == "layer norm, scale, shift":
        x = leaf_f32(g, r, (2, 77, 320), 3.0)
        y = g.mul_inplace(g.norm(x, 1e-5), leaf_f32(g, r, (320,)))
        return g.add_inplace(y, leaf_f32(g, r, (320,)))
    if name == "gated GELU":
        w, x, b = leaf_f16(g, r, (2 * 640, 320)), leaf_f32(g, r, (2, 200, 320)), leaf_f32(g, r, (2 * 640,))
        p = g.add_inplace(g.mul_mat(w, x), b)
        gate = g.gelu_inplace(g.cont(g.view_columns(p, 640, 640)))
        return g.mul(g.view_columns(p, 0, 640), gate)
    raise KeyError(name)


CASES = [
    "conv2d, bias", "conv2d 1x1, bias, scale per image", "conv2d by Winograd, bias, residual",
    "conv2d, bias, residual not in place", "conv2d of small images by Winograd, residual on the left",
    "linear, bias, residual not in place", "conv2d, bias, residual in its own memory",
    "conv2d by Winograd, residual in its own memory",
    "conv2d of small images by Winograd, residual in its own memory", "linear, bias, residual in its own memory",
    "linear, bias", "group norm, scale, shift, SiLU", "group norm of rows of no multiple of eight, scale, shift",
    "layer norm, scale, shift", "gated GELU",
]


def compute(gpu, name, tuning):
    g = gl.Graph(gpu)
    out = case(name, g, rng(sum(map(ord, name))))
    order, arr = g.build(out)
    sdhip.set_tuning(tuning)
    try:
        by_library = gl.run(sdhip.load(), order, arr)
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    return out.data.cpu().numpy().copy(), by_library, len(order)


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_fused_and_apart(gpu, name):
    fused, n_fused, n = compute(gpu, name, "")
    apart, n_apart, _ = compute(gpu, name, "fuse=0")
    largest = np.abs(apart.astype(np.float64)).max()
    rel = np.abs(fused.astype(np.float64) - apart).max() / largest
    print(f"{name}: {n_fused} of {n} nodes by the library fused, {n_apart} apart; {rel:.3g}")
    assert np.isfinite(fused).all() and np.isfinite(apart).all()
    assert rel <= 1e-6
    assert n_fused > n_apart


@pytest.mark.gpu
@pytest.mark.parametrize("tuning", ["fuse=0", "fuse_residual=0"])
@pytest.mark.parametrize("from_redirect", [False, True])
def test_entry_point_apart(gpu, tuning, from_redirect):
    """A chain ending in a residual connection handed to sdhip_mul_mat and
    sdhip_conv2d under fuse=0 or fuse_residual=0: computed after the operation
    in a pass of its own, into the redirect, bit for bit what the fused form
    writes (the same single-precision steps in the same order), and the
    operation's own tensor holding its output, as ggml's nodes leave it."""
    r = rng(77)
    wh, w32 = weights_f16(r, (70, 300))
    x = uniform(r, (2, 1100, 300), 1.0)
    b = uniform(r, (70,), 1.0)
    res = uniform(r, (2, 1100, 70), 1.0)
    w_d, x_d, b_d, res_d = dev(wh, gpu), dev(x, gpu), dev(b, gpu), dev(res, gpu)

    def go(t):
        y = torch.full((2, 1100, 70), float("nan"), device=gpu)
        if from_redirect:
            out = res_d.clone()
            chain = sdhip.epilogue([("add", b_d)], redirect=out, from_redirect=True)
        else:
            out = torch.full_like(y, float("nan"))
            chain = sdhip.epilogue([("add", b_d), ("add", res_d)], redirect=out)
        sdhip.set_tuning(t)
        try:
            sdhip.mul_mat(w_d, x_d, y, chain)
            torch.cuda.synchronize()
        finally:
            sdhip.set_tuning("")
        return y.cpu().numpy(), out.cpu().numpy()

    y_fused, out_fused = go("")
    y_apart, out_apart = go(tuning)
    assert np.isnan(y_fused).all()
    assert not np.isnan(y_apart).any()
    if from_redirect:
        # Begun from the residual (fused) or the residual added last (apart):
        # the same additions in another order.
        rel = np.abs(out_fused.astype(np.float64) - out_apart).max() / np.abs(out_apart).max()
        assert rel <= 1e-6
    else:
        assert np.array_equal(out_fused.view(np.uint32), out_apart.view(np.uint32))
    exact, mag = orc.exact_mul_mat(w32, x.reshape(-1, 300))
    add = b.astype(np.float64) + res.reshape(-1, 70)
    assert orc.metric(out_apart.reshape(-1, 70), exact + add, mag + np.abs(add)) <= 2e-5
