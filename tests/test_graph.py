"""The planner (sdhip_plan_nodes) on the CPU: which node of a graph is taken,
and which nodes after it are fused into it, over graphs built as ggml builds
them.  The cases are the reference's fusion cases (tests/ops_test.cc:952-1117)
with the plan match_chain, redirect_apart and match_gated_gelu make of each
(fusion.cc:136-394, hooks.cc:100-147), and the cases where they must not fuse:
a tensor read after the chain, a graph output, a redirect whose memory is an
operand's, a broadcast the positions of an image cannot take, fuse=0 and
fuse_residual=0.  The predicates read descriptors only, so the tensors here
are host memory."""

import ctypes

import numpy as np
import pytest
import torch

import graph_lib as gl
import sdhip

STEP = {0: "add", 1: "mul", 2: "silu"}


@pytest.fixture(scope="module")
def lib():
    return gl.bind(sdhip.load())


@pytest.fixture(autouse=True)
def default_tuning():
    sdhip.set_tuning("")
    yield
    sdhip.set_tuning("")


def f16(shape):
    return torch.zeros(shape, dtype=torch.float16)


def f32(shape):
    return torch.zeros(shape, dtype=torch.float32)


def planned(lib, out, index_of, outputs=()):
    order, arr = out[0].build(out[1], outputs)
    index = order.index(index_of)
    status, p = gl.plan(lib, arr, len(order), index)
    steps = [STEP[p.chain.steps[i].kind] for i in range(p.chain.count)]
    return order, status, p, steps


def conv_bias(g, ic=24, oc=40, w=40, h=36, n=2, k=3, pad=1):
    wt = g.leaf(f16((oc, ic, k, k)))
    x = g.leaf(f32((n, ic, h, w)))
    b = g.leaf(f32((oc,)))
    y = g.conv2d(wt, x, 1, 1, pad, pad, 1, 1)
    return y, g.add_inplace(y, g.reshape(b, (1, oc, 1, 1)))


def test_conv_bias(lib):
    g = gl.Graph("cpu")
    y, out = conv_bias(g)
    order, status, p, steps = planned(lib, (g, out), y)
    assert status == sdhip.OK and p.taken == gl.OP["CONV_2D"]
    assert [t.op for t in order] == ["CONV_2D", "RESHAPE", "ADD"]
    assert p.count == 3 and steps == ["add"] and not p.chain.redirect


def test_conv_1x1_bias_scale_per_image(lib):
    g = gl.Graph("cpu")
    y, yb = conv_bias(g, ic=16, oc=20, w=17, h=9, n=2, k=1, pad=0)
    e = g.leaf(f32((2, 20, 1, 1)))
    out = g.mul_inplace(yb, e)
    order, status, p, steps = planned(lib, (g, out), y)
    assert p.count == 4 and steps == ["add", "mul"]


def test_winograd_bias_residual_in_place(lib):
    g = gl.Graph("cpu")
    y, yb = conv_bias(g, ic=16, oc=24, w=66, h=40, n=1)
    r = g.leaf(f32((1, 24, 40, 66)))
    out = g.add_inplace(yb, r)
    order, status, p, steps = planned(lib, (g, out), y)
    assert p.count == 4 and steps == ["add", "add"] and not p.chain.redirect


def test_residual_not_in_place_is_a_redirect(lib):
    g = gl.Graph("cpu")
    y, yb = conv_bias(g)
    r = g.leaf(f32((2, 40, 36, 40)))
    out = g.add(yb, r)
    order, status, p, steps = planned(lib, (g, out), y)
    assert p.count == 4 and steps == ["add", "add"]
    assert p.chain.redirect and p.chain.redirect.contents.data == out.data.data_ptr()
    assert p.chain.from_redirect == 0
    assert p.chain.steps[1].operand.data == r.data.data_ptr()


def test_residual_on_the_left(lib):
    g = gl.Graph("cpu")
    wt = g.leaf(f16((48, 64, 3, 3)))
    x = g.leaf(f32((2, 64, 16, 16)))
    r = g.leaf(f32((2, 48, 16, 16)))
    y = g.conv2d(wt, x, 1, 1, 1, 1, 1, 1)
    out = g.add(r, y)
    order, status, p, steps = planned(lib, (g, out), y)
    assert p.count == 2 and steps == ["add"] and p.chain.redirect
    assert p.chain.steps[0].operand.data == r.data.data_ptr()


def test_linear_bias_residual_not_in_place(lib):
    g = gl.Graph("cpu")
    w = g.leaf(f16((70, 96)))
    x = g.leaf(f32((2, 50, 96)))
    b = g.leaf(f32((70,)))
    r = g.leaf(f32((2, 50, 70)))
    y = g.mul_mat(w, x)
    out = g.add(g.add_inplace(y, b), r)
    order, status, p, steps = planned(lib, (g, out), y)
    assert p.taken == gl.OP["MUL_MAT"] and p.count == 3 and steps == ["add", "add"] and p.chain.redirect


@pytest.mark.parametrize("kind", ["conv1x1", "winograd", "small", "linear"])
def test_residual_in_its_own_memory_begins_the_sum(lib, kind):
    """ggml_add_inplace(ggml_dup(r), y): the sum in the copy's memory, begun
    from it (from_redirect); the addition is no step."""
    g = gl.Graph("cpu")
    if kind == "linear":
        w = g.leaf(f16((70, 300)))
        x = g.leaf(f32((2, 1100, 300)))
        b = g.leaf(f32((70,)))
        r = g.leaf(f32((2, 1100, 70)))
        y = g.mul_mat(w, x)
        yb = g.add_inplace(y, b)
    elif kind == "small":
        wt = g.leaf(f16((48, 64, 3, 3)))
        x = g.leaf(f32((2, 64, 9, 15)))
        r = g.leaf(f32((2, 48, 9, 15)))
        y = yb = g.conv2d(wt, x, 1, 1, 1, 1, 1, 1)
    else:
        ic, oc, w_, h_, n, k, pad = (96, 40, 40, 36, 2, 1, 0) if kind == "conv1x1" else (16, 24, 66, 40, 1, 3, 1)
        y, yb = conv_bias(g, ic=ic, oc=oc, w=w_, h=h_, n=n, k=k, pad=pad)
        r = g.leaf(f32(tuple(y.data.shape)))
    d = g.dup(r)
    out = g.add_inplace(d, yb)
    order, status, p, steps = planned(lib, (g, out), y)
    assert order[0] is d  # the copy comes first, as ggml orders it
    assert p.chain.from_redirect == 1 and p.chain.redirect
    assert p.chain.redirect.contents.data == d.data.data_ptr()
    assert all(s == "add" for s in steps) and len(steps) == (0 if kind == "small" else 1)
    assert p.count == order.index(out) - order.index(y) + 1


def test_group_norm_scale_shift_silu(lib):
    g = gl.Graph("cpu")
    x = g.leaf(f32((2, 64, 20, 36)))
    gam = g.leaf(f32((1, 64, 1, 1)))
    bet = g.leaf(f32((1, 64, 1, 1)))
    y = g.group_norm(x, 32, 1e-6)
    out = g.silu_inplace(g.add_inplace(g.mul_inplace(y, gam), bet))
    order, status, p, steps = planned(lib, (g, out), y)
    assert p.taken == gl.OP["GROUP_NORM"] and p.count == 4 and steps == ["mul", "add", "silu"]


def test_layer_norm_scale_shift(lib):
    g = gl.Graph("cpu")
    x = g.leaf(f32((2, 77, 320)))
    gam = g.leaf(f32((320,)))
    bet = g.leaf(f32((320,)))
    y = g.norm(x, 1e-5)
    out = g.add_inplace(g.mul_inplace(y, gam), bet)
    order, status, p, steps = planned(lib, (g, out), y)
    assert p.taken == gl.OP["NORM"] and p.count == 3 and steps == ["mul", "add"]


def test_silu_not_fused_after_a_product(lib):
    """SiLU joins chains after normalisations only (hooks.cc:144-146)."""
    g = gl.Graph("cpu")
    w = g.leaf(f16((70, 96)))
    x = g.leaf(f32((50, 96)))
    b = g.leaf(f32((70,)))
    y = g.mul_mat(w, x)
    out = g.silu_inplace(g.add_inplace(y, b))
    order, status, p, steps = planned(lib, (g, out), y)
    assert p.count == 2 and steps == ["add"]


def test_gated_gelu(lib):
    """SD.cpp's GEGLU: the product and its bias, the halves viewed, the gate
    made contiguous and its GELU taken in place, x times it into a tensor of
    its own -- fused whole into the product (fusion.cc:347-394)."""
    g = gl.Graph("cpu")
    w = g.leaf(f16((2 * 640, 320)))
    x = g.leaf(f32((2, 200, 320)))
    b = g.leaf(f32((2 * 640,)))
    y = g.mul_mat(w, x)
    p_ = g.add_inplace(y, b)
    xv = g.view_columns(p_, 0, 640)
    gate = g.gelu_inplace(g.cont(g.view_columns(p_, 640, 640)))
    out = g.mul(xv, gate)
    order, status, p, steps = planned(lib, (g, out), y)
    assert [t.op for t in order] == ["MUL_MAT", "ADD", "VIEW", "VIEW", "CONT", "UNARY", "MUL"]
    assert steps == ["add"] and p.count == 7
    assert p.gated_out and p.gated_out.contents.tensor.data == out.data.data_ptr()
    # With the gate read by a later node, the halves must be written: no fusion.
    extra = g.add(gate, gate)
    order, status, p, steps = planned(lib, (g, extra), y)
    assert not p.gated_out and p.count == 2


@pytest.mark.parametrize("views", [1, 3])
def test_gated_gelu_with_views_in_the_chain(lib, views):
    """The GEGLU pattern after a chain whose steps are separated by views
    (RESHAPE nodes of the same memory): with one view a step the product,
    its 6 steps and their views are 13 nodes and the pattern is fused; with
    three a step they are 25, more than the planner tracks as never written,
    and it declines the gated form rather than check only some of them (the
    chain itself is still fused)."""
    g = gl.Graph("cpu")
    w = g.leaf(f16((2 * 64, 32)))
    x = g.leaf(f32((2, 20, 32)))
    y = g.mul_mat(w, x)
    p_ = y
    for i in range(6):
        for _ in range(views):
            p_ = g.reshape(p_, (2, 20, 2 * 64))
        p_ = g.add_inplace(p_, g.leaf(f32((2 * 64,))))
    xv = g.view_columns(p_, 0, 64)
    gate = g.gelu_inplace(g.cont(g.view_columns(p_, 64, 64)))
    out = g.mul(xv, gate)
    order, status, p, steps = planned(lib, (g, out), y)
    assert steps == ["add"] * 6
    chain_nodes = 1 + 6 * (views + 1)
    if views == 1:
        assert p.gated_out and p.count == chain_nodes + 5
    else:
        assert not p.gated_out and p.count == chain_nodes


def test_redirect_refused_when_the_head_is_read_after(lib):
    g = gl.Graph("cpu")
    y, yb = conv_bias(g)
    r = g.leaf(f32((2, 40, 36, 40)))
    s = g.add(yb, r)
    out = g.mul(s, g.reshape(yb, tuple(yb.data.shape)))  # y's memory read after the sum
    order, status, p, steps = planned(lib, (g, out), y)
    assert not p.chain.redirect and p.count == 3 and steps == ["add"]


def test_redirect_refused_for_a_graph_output(lib):
    g = gl.Graph("cpu")
    y, yb = conv_bias(g)
    r = g.leaf(f32((2, 40, 36, 40)))
    out = g.add(yb, r)
    order, status, p, steps = planned(lib, (g, out), y, outputs=[y])
    assert not p.chain.redirect and p.count == 3


def test_redirect_apart_falls_back(lib):
    """A redirect whose memory is the operation's input (the allocator's reuse)
    is not taken: the chain without it is (hooks.cc:114-118)."""
    g = gl.Graph("cpu")
    w = g.leaf(f16((70, 70)))
    xt = torch.zeros((2, 50, 70), dtype=torch.float32)
    x = g.leaf(xt)
    b = g.leaf(f32((70,)))
    r = g.leaf(f32((2, 50, 70)))
    y = g.mul_mat(w, x)
    s = gl.T(x.data, "ADD", [g.add_inplace(y, b), r])  # the sum written over x
    order, status, p, steps = planned(lib, (g, s), y)
    assert not p.chain.redirect and p.count == 2 and steps == ["add"]


def test_positions_take_broadcast_or_rows_only(lib):
    """After a convolution, an operand broadcast over the rows but not the
    columns of an image is no step (fusion.cc:189-196)."""
    g = gl.Graph("cpu")
    y, yb = conv_bias(g)
    col = g.leaf(f32((1, 1, 1, 40)))  # one number per column x
    out = g.add_inplace(yb, col)
    order, status, p, steps = planned(lib, (g, out), y)
    assert p.count == 3 and steps == ["add"]


def test_fuse_zero_and_fuse_residual_zero(lib):
    g = gl.Graph("cpu")
    y, yb = conv_bias(g)
    r = g.leaf(f32((2, 40, 36, 40)))
    out = g.add(yb, r)
    sdhip.set_tuning("fuse_residual=0")
    order, status, p, steps = planned(lib, (g, out), y)
    assert p.count == 3 and steps == ["add"] and not p.chain.redirect
    sdhip.set_tuning("fuse=0")
    order, status, p, steps = planned(lib, (g, out), y)
    assert p.count == 1 and steps == [] and p.taken == gl.OP["CONV_2D"]


def test_not_taken_nodes(lib):
    g = gl.Graph("cpu")
    w = g.leaf(f32((70, 96)))  # single-precision weights: not taken (yet)
    x = g.leaf(f32((50, 96)))
    y = g.mul_mat(w, x)
    order, status, p, steps = planned(lib, (g, y), y)
    assert status in (sdhip.OK, sdhip.UNSUPPORTED)
    b = g.leaf(f32((50, 70)))
    s = g.add(y, b)
    order, status, p, steps = planned(lib, (g, s), s)
    assert status == sdhip.UNSUPPORTED and p.taken == 0 and p.count == 0


def test_token_downsampling():
    lib = sdhip.load()
    assert lib.sdhip_token_downsampling(64, 64) == 1
    sdhip.set_tuning("todo=2")
    assert lib.sdhip_token_downsampling(64, 64) == 2  # 4096 tokens >= 2048
    assert lib.sdhip_token_downsampling(32, 32) == 1  # 1024 < 2048
    assert lib.sdhip_token_downsampling(0, 64) == 1
    sdhip.set_tuning("todo=3,todo_tokens=1024")
    assert lib.sdhip_token_downsampling(32, 32) == 3
    sdhip.set_tuning("todo=1")
    assert lib.sdhip_token_downsampling(64, 64) == 1
