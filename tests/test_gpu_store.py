"""The device store (sdhip_store_arena): the bits mode's quantized weights
kept from one call to the next, as the reference keeps its quantized layouts
(store.h, store.cc:64-99), and forgotten by sdhip_forget as sdasm_forget
forgets them (store.cc:241-266)."""

import numpy as np
import pytest
import torch

import oracle_lib as orc
import sdhip
from helpers import dev, rng, uniform, unwritten, weights_f16


def product(gpu, w_d, x_d, tuning="bits=8"):
    y = unwritten((x_d.shape[0], w_d.shape[0]), gpu)
    sdhip.set_tuning(tuning)
    try:
        sdhip.mul_mat(w_d, x_d, y)
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    return y.cpu().numpy()


@pytest.fixture
def arena(gpu):
    buf = torch.empty(64 << 20, dtype=torch.uint8, device=gpu)
    sdhip.store_arena(buf)
    yield buf
    sdhip.store_arena(None)


def kernels_of(fn):
    sdhip.profile_reset()
    sdhip.profile_enable(True)
    fn()
    torch.cuda.synchronize()
    sdhip.profile_enable(False)
    return sdhip.profile_collect()


@pytest.mark.gpu
def test_kept_weights_give_the_same_products(gpu, arena):
    K, N, M = 640, 384, 300
    r = rng(1)
    wh, w32 = weights_f16(r, (N, K))
    x = uniform(r, (M, K), 1.0)
    w_d, x_d = dev(wh, gpu), dev(x, gpu)
    want = orc.quantized_mul_mat(w32, x)[0]
    first = product(gpu, w_d, x_d)
    used, entries = sdhip.store_used()
    assert entries == 1 and used > 0
    second = kernels_of(lambda: product(gpu, w_d, x_d))
    assert "quantize_weights" not in second and "quantize_inputs" in second
    again = product(gpu, w_d, x_d)
    assert np.array_equal(first.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(again.view(np.uint32), want.view(np.uint32))
    # Another variant of the same weights (per-row scales) is another entry.
    rows = product(gpu, w_d, x_d, "bits=8,weight_group=0")
    assert sdhip.store_used()[1] == 2
    assert np.array_equal(rows.view(np.uint32), orc.quantized_mul_mat(w32, x, weight_groups=0)[0].view(np.uint32))


@pytest.mark.gpu
def test_gated_product_shares_the_entry(gpu, arena):
    K, half, M = 256, 640, 300
    r = rng(2)
    wh, w32 = weights_f16(r, (2 * half, K))
    x = uniform(r, (M, K), 1.0)
    w_d, x_d = dev(wh, gpu), dev(x, gpu)
    product(gpu, w_d, x_d)
    out = unwritten((M, half), gpu)
    y = unwritten((M, 2 * half), gpu)
    sdhip.set_tuning("bits=8")
    try:
        k = kernels_of(lambda: sdhip.mul_mat_gated(w_d, x_d, y, out))
    finally:
        sdhip.set_tuning("")
    assert "quantize_weights" not in k
    p = orc.quantized_mul_mat(w32, x)[0]
    want = orc.gated_gelu(p[:, :half], p[:, half:])
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
def test_forget_drops_the_entry(gpu, arena):
    K, N, M = 320, 320, 256
    r = rng(3)
    wh, w32 = weights_f16(r, (N, K))
    x = uniform(r, (M, K), 1.0)
    w_d, x_d = dev(wh, gpu), dev(x, gpu)
    product(gpu, w_d, x_d)
    # New weights written into the same memory: kept until forgotten.
    wh2, w322 = weights_f16(rng(4), (N, K))
    w_d.copy_(torch.from_numpy(wh2).to(gpu))
    stale = product(gpu, w_d, x_d)
    assert np.array_equal(stale.view(np.uint32), orc.quantized_mul_mat(w32, x)[0].view(np.uint32))
    sdhip.forget(w_d[1:2])  # any byte of the weights
    assert sdhip.store_used()[1] == 0
    fresh = product(gpu, w_d, x_d)
    assert np.array_equal(fresh.view(np.uint32), orc.quantized_mul_mat(w322, x)[0].view(np.uint32))


@pytest.mark.gpu
def test_small_arena_keeps_nothing(gpu):
    buf = torch.empty(4096, dtype=torch.uint8, device=gpu)
    sdhip.store_arena(buf)
    try:
        K, N, M = 640, 384, 300
        r = rng(5)
        wh, w32 = weights_f16(r, (N, K))
        x = uniform(r, (M, K), 1.0)
        y = product(gpu, dev(wh, gpu), dev(x, gpu))
        assert sdhip.store_used() == (0, 0)
        assert np.array_equal(y.view(np.uint32), orc.quantized_mul_mat(w32, x)[0].view(np.uint32))
    finally:
        sdhip.store_arena(None)


@pytest.mark.gpu
def test_no_entry_made_under_capture(gpu, arena):
    """A product captured into a graph before its weights are kept derives
    them in its work buffer; replays after the weights are kept by an eager
    call stay right, and every replay equals the eager result."""
    K, N, M = 320, 256, 300
    r = rng(6)
    wh, w32 = weights_f16(r, (N, K))
    x = uniform(r, (M, K), 1.0)
    w_d, x_d = dev(wh, gpu), dev(x, gpu)
    y = torch.empty((M, N), device=gpu)
    work = torch.empty(1 << 22, dtype=torch.uint8, device=gpu)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    sdhip.set_tuning("bits=8")
    try:
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                sdhip.mul_mat(w_d, x_d, y, work=work)
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        assert sdhip.store_used()[1] == 0
        want = orc.quantized_mul_mat(w32, x)[0]
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
            eager = product(gpu, w_d, x_d)  # makes the entry, then reads it
            assert np.array_equal(eager.view(np.uint32), want.view(np.uint32))
        assert sdhip.store_used()[1] == 1
    finally:
        sdhip.set_tuning("")


def convolve(gpu, k_d, x_d, oh, ow):
    y = unwritten((x_d.shape[0], k_d.shape[0], oh, ow), gpu)
    sdhip.conv2d(k_d, x_d, y, sdhip.conv_params(1, 1, 1, 1, 1, 1))
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("shape,path", [((2, 64, 40, 36), 4), ((4, 96, 8, 8), 2)])
def test_kept_winograd_weights(gpu, arena, shape, path):
    """Winograd's transformed weights (times 2^a_o) kept, as the reference
    keeps its transformed weights (winograd.cc:2147-2149): the first call
    fills the entry, later calls skip the weights' transform and give the
    same outputs bit for bit as a call without a store; new inputs of other
    magnitudes, same weights, agree with the oracle; sdhip_forget drops it."""
    n, ic, h_, w_ = shape
    oc = 48
    r = rng(8)
    kh16, k32 = weights_f16(r, (oc, ic, 3, 3))
    x = uniform(r, shape, 1.0)
    k_d, x_d = dev(kh16, gpu), dev(x, gpu)
    assert sdhip.conv2d_path(k_d, x_d, unwritten((n, oc, h_, w_), gpu), sdhip.conv_params(1, 1, 1, 1, 1, 1)) == path
    sdhip.store_arena(None)
    plain = convolve(gpu, k_d, x_d, h_, w_)
    sdhip.store_arena(arena)
    first = convolve(gpu, k_d, x_d, h_, w_)
    assert sdhip.store_used()[1] == 1
    tag = "winograd4" if path == 4 else "winograd2"
    second = kernels_of(lambda: convolve(gpu, k_d, x_d, h_, w_))
    assert f"{tag}.weights" not in second and f"{tag}.products" in second
    again = convolve(gpu, k_d, x_d, h_, w_)
    assert np.array_equal(first.view(np.uint32), plain.view(np.uint32))
    assert np.array_equal(again.view(np.uint32), plain.view(np.uint32))
    # Inputs 2^10 larger in half the channels: the kept weights serve them.
    x2 = (x * np.where(np.arange(ic) % 2 == 0, 1024.0, 1.0).reshape(1, ic, 1, 1)).astype(np.float32)
    y2 = convolve(gpu, k_d, dev(x2, gpu), h_, w_)
    exact, mag = orc.exact_conv2d(x2, k32, 1, 1, 1, 1, 1, 1)
    assert orc.metric(y2, exact, mag) <= 2e-5
    sdhip.forget(k_d)
    assert sdhip.store_used() == (0, 0)


@pytest.mark.gpu
@pytest.mark.parametrize("ic,oc", [(64, 48), (1280, 1280)])
def test_kept_small_images_weight_exponents(gpu, arena, ic, oc):
    """The small images' path (8 x 8 maps, two images: 32 tiles) keeps each
    split's exponents of the weights, which depend on the weights alone: the
    first call fills the entry, later calls skip the weights' pass and give
    the same outputs bit for bit as a call without a store; new inputs agree
    with the oracle; sdhip_forget drops the entry."""
    r = rng(ic + oc)
    kh16, k32 = weights_f16(r, (oc, ic, 3, 3))
    x = uniform(r, (2, ic, 8, 8), 1.0)
    k_d, x_d = dev(kh16, gpu), dev(x, gpu)
    assert sdhip.conv2d_path(k_d, x_d, unwritten((2, oc, 8, 8), gpu), sdhip.conv_params(1, 1, 1, 1, 1, 1)) == 2
    sdhip.store_arena(None)
    plain = convolve(gpu, k_d, x_d, 8, 8)
    sdhip.store_arena(arena)
    first = convolve(gpu, k_d, x_d, 8, 8)
    assert sdhip.store_used()[1] == 1
    again = convolve(gpu, k_d, x_d, 8, 8)
    assert np.array_equal(first.view(np.uint32), plain.view(np.uint32))
    assert np.array_equal(again.view(np.uint32), plain.view(np.uint32))
    x2 = uniform(r, (2, ic, 8, 8), 4.0)
    y2 = convolve(gpu, k_d, dev(x2, gpu), 8, 8)
    exact, mag = orc.exact_conv2d(x2, k32, 1, 1, 1, 1, 1, 1)
    assert orc.metric(y2, exact, mag) <= 2e-5
    sdhip.forget(k_d)
    assert sdhip.store_used() == (0, 0)
