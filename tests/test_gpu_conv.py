"""CONV_2D on the device -- direct, Winograd F(2x2, 3x3) and F(4x4, 3x3) --
against the float64 oracle by the reference's metric, at the reference's
test shapes (ops_test.cc:801-819, FP16 kernels) and the SD1.5 configurations
of the bench (at full size the oracle checks a sample of the outputs)."""

import numpy as np
import pytest
import torch

import oracle_lib as orc
import sdhip
from helpers import dev, normal, rng, uniform, unwritten, weights_f16

BOUND = 2e-5

# w, h, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n  (ops_test.cc:801-819, FP16 ones)
CASES = [
    (64, 64, 64, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2),
    (16, 16, 96, 64, 3, 3, 1, 1, 1, 1, 1, 1, 2),
    (8, 8, 96, 64, 3, 3, 1, 1, 1, 1, 1, 1, 2),
    (32, 32, 64, 40, 1, 1, 1, 1, 0, 0, 1, 1, 2),
    (33, 33, 24, 30, 3, 3, 2, 2, 1, 1, 1, 1, 1),
    (100, 3, 20, 25, 3, 3, 1, 1, 0, 1, 1, 1, 1),
    (512, 4, 16, 3, 3, 3, 1, 1, 1, 1, 1, 1, 1),
    (65, 33, 24, 20, 3, 3, 1, 1, 1, 1, 1, 1, 2),
    (64, 20, 13, 11, 3, 3, 1, 1, 0, 0, 1, 1, 1),
    (128, 128, 8, 8, 3, 3, 1, 1, 1, 1, 1, 1, 1),
    (40, 9, 7, 13, 5, 3, 1, 2, 2, 0, 2, 1, 1),
    (17, 13, 5, 7, 3, 3, 1, 1, 1, 1, 1, 1, 3),
    (32, 32, 64, 64, 3, 3, 2, 2, 1, 1, 1, 1, 2),   # the UNet's downsampling, fewer channels
    (20, 20, 16, 8, 3, 3, 1, 1, 2, 2, 2, 2, 1),    # 3x3 dilated: direct
    (16, 16, 1280, 640, 1, 1, 1, 1, 0, 0, 1, 1, 2),  # 1x1 of few blocks and long K: split along K by columns
    (8, 8, 2560, 1280, 1, 1, 1, 1, 0, 0, 1, 1, 1),   # the same at the UNet's 8 x 8, one image
]


def out_size(i, k, s, p, d):
    return (i + 2 * p - d * (k - 1) - 1) // s + 1


def conv_case(gpu, c, seed, chain_steps=(), redirect=None, from_redirect=False, tuning="", f32=False):
    w_, h_, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n = c
    r = rng(seed)
    kh16, k32 = weights_f16(r, (oc, ic, kh, kw))
    if f32:
        # Single-precision kernels, not FP16 numbers (the reference's
        # GGML_TYPE_F32 cases): FP16 ones plus a part below FP16's step.
        k32 = (k32 + uniform(r, k32.shape, 2.0 ** -14)).astype(np.float32)
        kh16 = k32
    x = uniform(r, (n, ic, h_, w_), 1.0)
    oh, ow = out_size(h_, kh, s1, p1, d1), out_size(w_, kw, s0, p0, d0)
    k_d, x_d = dev(kh16, gpu), dev(x, gpu)
    y_d = unwritten((n, oc, oh, ow), gpu)
    params = sdhip.conv_params(s0, s1, p0, p1, d0, d1)
    sdhip.set_tuning(tuning)
    try:
        path = sdhip.conv2d_path(k_d, x_d, y_d, params)
        sdhip.conv2d(k_d, x_d, y_d, params, sdhip.epilogue(chain_steps, redirect, from_redirect))
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    return x, k32, y_d, path, (s0, s1, p0, p1, d0, d1)


@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("tuning", ["", "winograd=1", "winograd=0", "winograd_fp32=1"])
def test_conv2d(gpu, c, tuning):
    x, k32, y, path, p = conv_case(gpu, c, seed=sum(c), tuning=tuning)
    exact, mag = orc.exact_conv2d(x, k32, *p)
    err = orc.metric(y.cpu().numpy(), exact, mag)
    print(f"conv {c} path {path} [{tuning}]: {err:.3g}")
    assert err <= BOUND


# The reference's single-precision kernels (ops_test.cc:809-810, 817) and a
# large 3x3 one: F(2x2) where FP16 kernels would take F(4x4)
# (winograd.cc:1204-1206), directly where not Winograd.
F32_CASES = [
    ((17, 13, 5, 7, 3, 3, 1, 1, 1, 1, 1, 1, 3), 2),
    ((40, 9, 7, 13, 5, 3, 1, 2, 2, 0, 2, 1, 1), 0),
    ((96, 16, 32, 17, 3, 3, 1, 1, 1, 1, 1, 1, 1), 2),
    ((64, 64, 64, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2), 2),
    ((32, 32, 64, 40, 1, 1, 1, 1, 0, 0, 1, 1, 2), 0),
    ((33, 33, 24, 30, 3, 3, 2, 2, 1, 1, 1, 1, 1), 0),
]


@pytest.mark.gpu
@pytest.mark.parametrize("c,want_path", F32_CASES, ids=lambda c: "x".join(map(str, c)) if isinstance(c, tuple) else str(c))
@pytest.mark.parametrize("tuning", ["", "winograd=0", "winograd_fp32=1"])
def test_conv2d_single_precision_kernels(gpu, c, want_path, tuning):
    r = rng(sum(c) + 3)
    b = uniform(r, (1, c[3], 1, 1), 1.0)
    b_d = dev(b, gpu)
    x, k32, y, path, p = conv_case(gpu, c, seed=sum(c) + 1, chain_steps=[("add", b_d)], tuning=tuning, f32=True)
    if tuning == "":
        assert path == want_path
    exact, mag = orc.exact_conv2d(x, k32, *p)
    exact = exact + b.astype(np.float64)
    err = orc.metric(y.cpu().numpy(), exact, mag + np.abs(b))
    print(f"conv single-precision kernels {c} path {path} [{tuning}]: {err:.3g}")
    assert err <= BOUND


@pytest.mark.gpu
@pytest.mark.parametrize("c,tuning", [
    ((8, 8, 24, 40, 3, 3, 1, 1, 1, 1, 1, 1, 2), ""),                  # F(2x2), IC % 16 = 8, OC % 16 = 8
    ((6, 6, 40, 20, 3, 3, 1, 1, 1, 1, 1, 1, 1), ""),                  # F(2x2), 9 tiles: one tile group
    ((16, 16, 72, 24, 3, 3, 1, 1, 1, 1, 1, 1, 1), ""),                # F(4x4), 16 tiles
    ((17, 18, 56, 36, 3, 3, 1, 1, 1, 1, 1, 1, 1), ""),                # F(4x4), 25 tiles, ragged edges
    ((8, 8, 200, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2), "winograd_splits=3"),  # splits of 96, 96 and 8 channels
    ((16, 16, 264, 40, 3, 3, 1, 1, 1, 1, 1, 1, 2), "winograd_splits=5"),  # three of 96, the last past IC
    ((16, 16, 64, 32, 3, 3, 1, 1, 1, 1, 1, 1, 2), "winograd_splits=1"),
])
def test_winograd_small_images(gpu, c, tuning):
    """The small images' path (every tile of all images in one group, the
    transformed weights made in registers): channel counts that end partway
    through a step of 32 or a group of 16 output channels, one group of 16
    tiles, and splits of the input channels of unequal lengths."""
    x, k32, y, path, p = conv_case(gpu, c, seed=sum(c) + 5, tuning=tuning)
    exact, mag = orc.exact_conv2d(x, k32, *p)
    err = orc.metric(y.cpu().numpy(), exact, mag)
    print(f"small images {c} path {path} [{tuning}]: {err:.3g}")
    assert path == (4 if c[0] * c[1] >= 256 else 2)
    assert err <= BOUND


@pytest.mark.gpu
def test_path_selection(gpu):
    """The paths the reference's predicates choose (winograd.cc:194-196,
    1204-1206, 2107-2123; hooks.cc:36-41)."""
    def path(w_, h_, ic, oc, kk, s, p, n, tuning=""):
        k = torch.zeros((oc, ic, kk, kk), dtype=torch.float16, device=gpu)
        x = torch.zeros((n, ic, h_, w_), dtype=torch.float32, device=gpu)
        oh, ow = out_size(h_, kk, s, p, 1), out_size(w_, kk, s, p, 1)
        y = torch.zeros((n, oc, oh, ow), dtype=torch.float32, device=gpu)
        sdhip.set_tuning(tuning)
        try:
            return sdhip.conv2d_path(k, x, y, sdhip.conv_params(s, s, p, p, 1, 1))
        finally:
            sdhip.set_tuning("")
    assert path(64, 64, 320, 320, 3, 1, 1, 2) == 4      # F(4x4): >= 1024 outputs
    assert path(8, 8, 1280, 1280, 3, 1, 1, 2) == 2      # F(2x2): small, 32 tiles
    assert path(16, 16, 1280, 1280, 3, 1, 1, 2) == 4    # small (128 tiles) and 256 outputs: F(4x4)
    assert path(32, 32, 640, 1280, 1, 1, 0, 2) == 0     # 1x1: direct
    assert path(33, 33, 24, 30, 3, 2, 1, 1) == 0        # stride 2: direct
    assert path(64, 64, 320, 320, 3, 1, 1, 2, "winograd=1") == 2
    assert path(64, 64, 320, 320, 3, 1, 1, 2, "winograd=0") == 0


@pytest.mark.gpu
@pytest.mark.parametrize("c", [
    (40, 36, 24, 40, 3, 3, 1, 1, 1, 1, 1, 1, 2),   # Winograd F(4x4), 1440 outputs
    (66, 40, 16, 24, 3, 3, 1, 1, 1, 1, 1, 1, 1),   # Winograd F(4x4), odd tiles
    (15, 9, 64, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2),    # small images, F(2x2)
    (40, 36, 96, 40, 1, 1, 1, 1, 0, 0, 1, 1, 2),   # 1x1
])
@pytest.mark.parametrize("mode", ["bias", "residual", "from_redirect"])
def test_conv2d_chain(gpu, c, mode):
    """conv + bias, + residual not in place, or begun from the residual in its
    own memory (ops_test.cc:952-1061)."""
    w_, h_, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n = c
    oh, ow = out_size(h_, kh, s1, p1, d1), out_size(w_, kw, s0, p0, d0)
    r = rng(99)
    bias = uniform(r, (1, oc, 1, 1), 1.0)
    res = uniform(r, (n, oc, oh, ow), 1.0)
    b_d, res_d = dev(bias, gpu), dev(res, gpu)
    if mode == "bias":
        x, k32, y, path, p = conv_case(gpu, c, 7, [("add", b_d)])
        out = y
        add = np.broadcast_to(bias, res.shape).astype(np.float64)
    elif mode == "residual":
        out = unwritten(res.shape, gpu)
        x, k32, y, path, p = conv_case(gpu, c, 7, [("add", b_d), ("add", res_d)], redirect=out)
        add = bias.astype(np.float64) + res
    else:
        out = res_d.clone()
        x, k32, y, path, p = conv_case(gpu, c, 7, [("add", b_d)], redirect=out, from_redirect=True)
        add = bias.astype(np.float64) + res
    exact, mag = orc.exact_conv2d(x, k32, *p)
    err = orc.metric(out.cpu().numpy(), exact + add, mag + np.abs(add))
    print(f"conv chain {mode} {c} path {path}: {err:.3g}")
    assert err <= BOUND


@pytest.mark.gpu
@pytest.mark.parametrize("c", [
    (40, 36, 24, 40, 3, 3, 1, 1, 1, 1, 1, 1, 2),   # F(4x4)
    (15, 9, 64, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2),    # F(2x2)
])
def test_winograd_wide_range(gpu, c):
    """Input channels 2^-30 .. 2^30 apart and output channels' weights 2^-12 ..
    2^4: the split products scale each channel into FP16's range by powers of
    two, so the bound holds at any scale an FP32 input takes."""
    w_, h_, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n = c
    r = rng(5)
    x = uniform(r, (n, ic, h_, w_), 1.0) * np.exp2(r.integers(-30, 31, size=(1, ic, 1, 1))).astype(np.float32)
    k = (r.uniform(-1, 1, size=(oc, ic, kh, kw)) * np.exp2(r.integers(-12, 5, size=(oc, 1, 1, 1))))
    k16 = k.astype(np.float16)
    k_d, x_d = dev(k16, gpu), dev(x.astype(np.float32), gpu)
    oh, ow = out_size(h_, kh, s1, p1, d1), out_size(w_, kw, s0, p0, d0)
    y = unwritten((n, oc, oh, ow), gpu)
    params = sdhip.conv_params(s0, s1, p0, p1, d0, d1)
    path = sdhip.conv2d_path(k_d, x_d, y, params)
    sdhip.conv2d(k_d, x_d, y, params)
    torch.cuda.synchronize()
    exact, mag = orc.exact_conv2d(x.astype(np.float32), k16.astype(np.float32), s0, s1, p0, p1, d0, d1)
    err = orc.metric(y.cpu().numpy(), exact, mag)
    print(f"wide range {c} path {path}: {err:.3g}")
    assert path in (2, 4)
    assert err <= BOUND


def sampled(gpu, shape, k, s, p, seed, count=3000, chain=None):
    n, ic, h_, w_ = shape
    oc = k[0]
    r = rng(seed)
    kh16 = (0.02 * r.standard_normal(size=k)).astype(np.float16)
    x = normal(r, shape)
    k_d, x_d = dev(kh16, gpu), dev(x, gpu)
    kk = k[2]
    oh, ow = out_size(h_, kk, s, p, 1), out_size(w_, kk, s, p, 1)
    y = unwritten((n, oc, oh, ow), gpu)
    params = sdhip.conv_params(s, s, p, p, 1, 1)
    path = sdhip.conv2d_path(k_d, x_d, y, params)
    sdhip.conv2d(k_d, x_d, y, params)
    torch.cuda.synchronize()
    yy = y.cpu().numpy().reshape(-1)
    assert np.isfinite(yy).all(), "every output written"
    index = r.choice(yy.size, size=count, replace=False)
    exact, mag = orc.exact_conv2d(x, kh16.astype(np.float32), s, s, p, p, 1, 1, index=index)
    return orc.metric(yy[index], exact, mag), path


@pytest.mark.gpu
@pytest.mark.parametrize("name,shape,k,s,p,want", [
    ("cfg2 F(4x4) 64x64x320", (2, 320, 64, 64), (320, 320, 3, 3), 1, 1, 4),
    ("cfg3a F(2x2) 8x8x1280", (2, 1280, 8, 8), (1280, 1280, 3, 3), 1, 1, 2),
    ("cfg3b 1x1 32x32 640->1280", (2, 640, 32, 32), (1280, 640, 1, 1), 1, 0, 0),
    ("VAE decoder 128x128 512->512", (1, 512, 128, 128), (512, 512, 3, 3), 1, 1, 4),
])
def test_conv2d_bench_shapes(gpu, name, shape, k, s, p, want):
    err, path = sampled(gpu, shape, k, s, p, seed=len(name))
    print(f"{name}: path {path}, sampled error {err:.3g}")
    assert path == want
    assert err <= BOUND


@pytest.mark.gpu
@pytest.mark.parametrize("c", [
    (64, 64, 64, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2),   # F(4x4)
    (8, 8, 96, 64, 3, 3, 1, 1, 1, 1, 1, 1, 2),     # F(2x2)
])
def test_winograd_graph_replays(gpu, c):
    """The Winograd path captured into a HIP graph and replayed with eager
    convolutions between the replays: every replay equals the eager result
    bit for bit."""
    w_, h_, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n = c
    r = rng(21)
    kh16, _ = weights_f16(r, (oc, ic, kh, kw))
    x = uniform(r, (n, ic, h_, w_), 1.0)
    k_d, x_d = dev(kh16, gpu), dev(x, gpu)
    oh, ow = out_size(h_, kh, s1, p1, d1), out_size(w_, kw, s0, p0, d0)
    params = sdhip.conv_params(s0, s1, p0, p1, d0, d1)
    eager = torch.empty((n, oc, oh, ow), device=gpu)
    sdhip.conv2d(k_d, x_d, eager, params)
    torch.cuda.synchronize()
    want = eager.cpu().numpy()
    y = torch.zeros((n, oc, oh, ow), device=gpu)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            sdhip.conv2d(k_d, x_d, y, params)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
        other = torch.empty_like(eager)
        sdhip.conv2d(k_d, x_d, other, params)
        torch.cuda.synchronize()
        assert np.array_equal(other.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("c,want_path,small_path", [
    ((40, 36, 24, 40, 3, 3, 1, 1, 1, 1, 1, 1, 2), 4, False),  # Winograd F(4x4), transforms of the large path
    ((15, 9, 64, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2), 2, False),   # F(2x2), 80 tiles: the large path
    ((8, 8, 64, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2), 2, True),     # small images, F(2x2): 32 tiles
    ((16, 16, 72, 24, 3, 3, 1, 1, 1, 1, 1, 1, 1), 4, True),   # small images, F(4x4)
    ((33, 33, 24, 30, 3, 3, 2, 2, 1, 1, 1, 1, 1), 0, False),  # direct by columns
    ((32, 32, 64, 40, 1, 1, 1, 1, 0, 0, 1, 1, 2), 0, False),  # 1x1
], ids=lambda c: "x".join(map(str, c)) if isinstance(c, tuple) else str(c))
def test_conv2d_strided_input(gpu, c, want_path, small_path):
    """The input as a view into a larger tensor: rows, planes and images
    further apart than their extents, and a start that is no multiple of 16
    bytes -- ggml's nb[1..3] of a view (the predicate takes any multiple of 4
    bytes, conv2d.cc:320-331).  The path and, for Winograd, whether the small
    images' kernels ran (no transforms launch) are checked from the profile."""
    w_, h_, ic, oc, kw, kh, s0, s1, p0, p1, d0, d1, n = c
    r = rng(sum(c) + 11)
    kh16, k32 = weights_f16(r, (oc, ic, kh, kw))
    big = uniform(r, (n, ic + 3, h_ + 2, w_ + 5), 1.0)
    x = np.ascontiguousarray(big[:, 1:ic + 1, 1:h_ + 1, 2:w_ + 2])
    big_d = dev(big, gpu)
    x_d = big_d[:, 1:ic + 1, 1:h_ + 1, 2:w_ + 2]
    assert not x_d.is_contiguous()
    oh, ow = out_size(h_, kh, s1, p1, d1), out_size(w_, kw, s0, p0, d0)
    k_d = dev(kh16, gpu)
    y_d = unwritten((n, oc, oh, ow), gpu)
    params = sdhip.conv_params(s0, s1, p0, p1, d0, d1)
    path = sdhip.conv2d_path(k_d, x_d, y_d, params)
    assert path == want_path
    sdhip.profile_reset()
    sdhip.profile_enable(True)
    try:
        sdhip.conv2d(k_d, x_d, y_d, params)
        torch.cuda.synchronize()
        ran = sdhip.profile_collect()
    finally:
        sdhip.profile_enable(False)
        sdhip.profile_reset()
    if path in (2, 4):
        tag = f"winograd{path}"
        assert f"{tag}.products" in ran
        large = f"{tag}.transforms" in ran or f"{tag}.weights" in ran
        assert large != small_path, sorted(ran)
    exact, mag = orc.exact_conv2d(x, k32, s0, s1, p0, p1, d0, d1)
    err = orc.metric(y_d.cpu().numpy(), exact, mag)
    print(f"strided input {c} path {path}: {err:.3g}")
    assert err <= BOUND


@pytest.mark.gpu
@pytest.mark.parametrize("c", [(64, 64, 64, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2), (65, 33, 24, 20, 3, 3, 1, 1, 1, 1, 1, 1, 2),
                               (96, 16, 32, 17, 3, 3, 1, 1, 1, 1, 1, 1, 1)], ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("core,tiles", [(3, 0), (3, 22), (3, 41), (3, 12), (0, 0)])
def test_winograd_products_cores_agree(gpu, c, core, tiles):
    """Winograd's products by the core whose waves load their own
    transformed inputs (gemm_core=3, V in runs of 8 channels) and by the
    default choice (0) give the bits of the register-staged core (1, V in
    runs of 32), at every block shape: the same MFMAs in the same order of k."""
    _, _, y1, path, _ = conv_case(gpu, c, seed=sum(c), tuning="gemm_core=1")
    _, _, y2, _, _ = conv_case(gpu, c, seed=sum(c), tuning=f"gemm_core={core},gemm_tiles={tiles}")
    assert path in (2, 4)
    assert np.array_equal(y1.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("c", [(64, 64, 64, 48, 3, 3, 1, 1, 1, 1, 1, 1, 2), (65, 33, 24, 20, 3, 3, 1, 1, 1, 1, 1, 1, 2),
                               (96, 16, 32, 17, 3, 3, 1, 1, 1, 1, 1, 1, 1), (40, 40, 96, 160, 3, 3, 1, 1, 1, 1, 1, 1, 2)],
                         ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("tuning", ["gemm_core=3", "gemm_core=3,gemm_tiles=22", "gemm_core=3,gemm_tiles=41",
                                    "gemm_core=3,gemm_tiles=12", "gemm_core=3,gemm_stages=4",
                                    "gemm_core=3,gemm_tiles=22,gemm_stages=4"])
def test_winograd_products_without_lds(gpu, c, tuning):
    """Winograd's products with the transformed weights shared through LDS
    and each wave's transformed inputs loaded straight into its registers
    (gemm_core=3): held to the bound against float64, with ragged rows (OC,
    tiles) at every block shape and both prefetch depths."""
    x, k32, y, path, p = conv_case(gpu, c, seed=sum(c), tuning=tuning)
    assert path in (2, 4)
    exact, mag = orc.exact_conv2d(x, k32, *p)
    err = orc.metric(y.cpu().numpy(), exact, mag)
    print(f"conv {c} path {path} [{tuning}]: {err:.3g}")
    assert err <= BOUND


CONV_PANEL_CASES = [  # w, h, ic, oc, n: 1x1 outputs of 256 panels of 64 positions by 160 channels and more
    (32, 32, 640, 1280, 2),   # cfg3b's
    (64, 64, 320, 200, 2),    # ragged OC: channels past OC read the last
    (64, 64, 384, 320, 2),
]


@pytest.mark.gpu
@pytest.mark.parametrize("c", CONV_PANEL_CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("form", ["bias_scale_residual", "from_redirect_silu", "strided_residual"])
def test_conv_panels(gpu, c, form):
    """The 1x1 convolution by panels (conv_panels) through each form of its
    chain: a bias (one number a channel), a scale per position and a residual
    (rows of positions, a float4 at a time); the sum begun from the residual
    in the output's memory, then SiLU; a residual whose rows are one float
    longer than the image's (positions strided: element by element).  Against
    float64, and within the same bound of the 64 x 64 core (conv_panels=0)."""
    w_, h_, ic, oc, n = c
    case = (w_, h_, ic, oc, 1, 1, 1, 1, 0, 0, 1, 1, n)
    r = rng(ic + oc)
    bias = uniform(r, (1, oc, 1, 1), 1.0)
    scale = uniform(r, (1, 1, h_, w_), 1.0)
    res = uniform(r, (n, oc, h_, w_), 1.0)
    b_d, s_d, res_d = dev(bias, gpu), dev(scale, gpu), dev(res, gpu)
    outs = []
    for tuning in ("", "conv_panels=0"):
        if form == "bias_scale_residual":
            x, k32, y, path, p = conv_case(gpu, case, 11, [("add", b_d), ("mul", s_d), ("add", res_d)], tuning=tuning)
            exact, mag = orc.exact_conv2d(x, k32, *p)
            b, s = bias.astype(np.float64), scale.astype(np.float64)
            want, m2 = (exact + b) * s + res, (mag + np.abs(b)) * np.abs(s) + np.abs(res)
            got = y.cpu().numpy()
        elif form == "from_redirect_silu":
            out = res_d.clone()
            x, k32, y, path, p = conv_case(gpu, case, 11, [("add", b_d), ("silu", None)], redirect=out,
                                           from_redirect=True, tuning=tuning)
            exact, mag = orc.exact_conv2d(x, k32, *p)
            t = res + exact + bias.astype(np.float64)
            want, m2 = t / (1.0 + np.exp(-t)), np.abs(res) + mag + np.abs(bias)
            got = out.cpu().numpy()
        else:
            wide = np.zeros((n, oc, h_, w_ + 1), np.float32)
            wide[..., :w_] = res
            rv = dev(wide, gpu)[..., :w_]
            x, k32, y, path, p = conv_case(gpu, case, 11, [("add", rv)], tuning=tuning)
            exact, mag = orc.exact_conv2d(x, k32, *p)
            want, m2 = exact + res, mag + np.abs(res)
            got = y.cpu().numpy()
        err = orc.metric(got, want, m2)
        print(f"conv panels {c} [{form}] {tuning or 'panels'} path {path}: {err:.3g}")
        assert err <= BOUND
        outs.append(got)
    assert orc.metric(outs[0], outs[1], m2) <= BOUND
