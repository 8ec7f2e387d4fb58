"""The bits mode (quant.h) of the linear layers on the device.

The integer stage -- each input's byte, scale and zero point per (row, group
of k), each weight's byte, scale and sum per (column, group) or per column,
the exact integer sums -- and the dequantisation t = fma(sa sb, S, t);
t = fma(-oa, ob, t) in the reference's order (quant.cc:113-164) make the
device's output the reference's C++ output bit for bit; the oracle restates
quant.cc, and these tests hold the device to it exactly.  They also hold it
to the reference's own bound against float64 (ops_test.cc:213-296):
kQuantized = 1e-2 scaled by (2/L + 1/W) / (2/255 + 1/127)."""

import numpy as np
import pytest
import torch

import oracle_lib as orc
import sdhip
from helpers import dev, rng, uniform, unwritten, weights_f16

K_QUANTIZED = 1e-2


def bound(levels, wmax):
    return K_QUANTIZED * (2.0 / levels + 1.0 / wmax) / (2.0 / 255 + 1.0 / 127)


def quant_params(tuning):
    t = dict(kv.split("=") for kv in tuning.split(",") if kv)
    bits = int(t.get("bits", 0))
    ib = int(t.get("input_bits", 8))
    group = max(1, min(256, int(t.get("group", 64)) // 4)) * 4
    return group, (1 << ib) - 1, (1 << (bits - 1)) - 1, int(t.get("weight_group", 1))


def run_quantized(gpu, K, N, M, B, tuning, seed, bias=True):
    r = rng(seed)
    wh, w32 = weights_f16(r, (N, K))
    x = uniform(r, (B, M, K), 1.0)
    b = uniform(r, (N,), 1.0)
    w_d, x_d, b_d = dev(wh, gpu), dev(x, gpu), dev(b, gpu)
    y = unwritten((B, M, N), gpu)
    sdhip.set_tuning(tuning)
    try:
        sdhip.mul_mat(w_d, x_d, y, sdhip.epilogue([("add", b_d)] if bias else []))
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    return w32, x.reshape(B * M, K), b, y.cpu().numpy().reshape(B * M, N)


CASES = [  # K, N, M, batch (ops_test.cc:875-883, of 256 rows and more)
    (320, 320, 512, 2),
    (768, 1280, 300, 1),
    (1280, 320, 256, 1),
    (77, 100, 300, 1),
    (300, 17, 131, 3),
    (40, 2560, 296, 1),
    (1280, 1280, 988, 2),  # the SDXL block's projections
]


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,M,B", CASES)
@pytest.mark.parametrize("tuning", ["bits=8", "bits=8,weight_group=0", "bits=8,group=128", "bits=8,group=32",
                                    "bits=7", "bits=8,input_bits=7"])
def test_quantized_mul_mat(gpu, K, N, M, B, tuning):
    group, levels, wmax, wg = quant_params(tuning)
    w32, x, b, y = run_quantized(gpu, K, N, M, B, tuning, seed=K + N + M)
    want = orc.quantized_mul_mat(w32, x, group, levels, wmax, wg)[0]
    want = (want + b).astype(np.float32)  # the bias, a chain step in single precision
    exact, mag = orc.exact_mul_mat(w32, x)
    err = orc.metric(y, exact + b, mag + np.abs(b))
    same = np.array_equal(y.view(np.uint32), want.view(np.uint32))
    print(f"quantized {K}->{N} x {M}x{B} [{tuning}]: error {err:.3g}, bit-exact with the oracle: {same}")
    assert same, f"differs from the reference's quantized product in {np.sum(y != want)} of {y.size}"
    assert err <= bound(levels, wmax)


@pytest.mark.gpu
def test_quantized_from_redirect(gpu):
    """The sum begun from the residual in the output's memory, as the
    quantized product's tiles accumulate into it (mul_mat.cc:551-558)."""
    K, N, M = 300, 70, 1100
    r = rng(3)
    wh, w32 = weights_f16(r, (N, K))
    x = uniform(r, (M, K), 1.0)
    res = uniform(r, (M, N), 1.0)
    w_d, x_d = dev(wh, gpu), dev(x, gpu)
    out = dev(res, gpu)
    y = unwritten((M, N), gpu)
    sdhip.set_tuning("bits=8")
    try:
        sdhip.mul_mat(w_d, x_d, y, sdhip.epilogue([], redirect=out, from_redirect=True))
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    want = orc.quantized_mul_mat(w32, x, init=res)[0]
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.gpu
def test_not_quantized_under_256_rows(gpu):
    """Products of fewer than 256 rows stay in single precision
    (mul_mat.cc:95-105): then the split-FP16 path's 1e-7 class holds."""
    w32, x, b, y = run_quantized(gpu, 768, 320, 77, 2, "bits=8", seed=1)
    exact, mag = orc.exact_mul_mat(w32, x)
    assert orc.metric(y, exact + b, mag + np.abs(b)) <= 2e-6


@pytest.mark.gpu
@pytest.mark.parametrize("K,half,M,tuning", [(320, 1280, 400, "bits=8"), (96, 2000, 300, "bits=8"),
                                             (256, 640, 300, "bits=8,group=128"),
                                             (1280, 5120, 988, "bits=8,weight_group=0")])
def test_quantized_gated(gpu, K, half, M, tuning):
    group, levels, wmax, wg = quant_params(tuning)
    r = rng(K + half)
    wh, w32 = weights_f16(r, (2 * half, K))
    x = uniform(r, (M, K), 1.0)
    bias = uniform(r, (2 * half,), 1.0)
    w_d, x_d, b_d = dev(wh, gpu), dev(x, gpu), dev(bias, gpu)
    y = unwritten((M, 2 * half), gpu)
    out = unwritten((M, half), gpu)
    sdhip.set_tuning(tuning)
    try:
        sdhip.mul_mat_gated(w_d, x_d, y, out, sdhip.epilogue([("add", b_d)]))
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    p = orc.quantized_mul_mat(w32, x, group, levels, wmax, wg)[0]
    p = (p + bias).astype(np.float32)
    want = orc.gated_gelu(p[:, :half], p[:, half:])
    got = out.cpu().numpy()
    exact, mag = orc.exact_gated(w32, x, bias)
    err = orc.metric(got, exact, mag)
    same = np.array_equal(got.view(np.uint32), want.view(np.uint32))
    print(f"quantized gated {K}->2x{half} x {M} [{tuning}]: error {err:.3g}, bit-exact: {same}")
    assert same
    assert err <= bound(levels, wmax)


@pytest.mark.gpu
@pytest.mark.parametrize("from_redirect", [False, True])
def test_sdxl_ff_out_with_residual(gpu, from_redirect):
    """configs[4]'s FF-out product at full size: 5120 -> 1280 over 988 x 2
    tokens, bits=8 with a scale per whole row of weights (weight_group=0),
    its bias, and the block's residual connection ending the chain -- as a
    redirect with the residual's addition as its last step, or begun from the
    residual already in the output's memory (fusion.h:64-80).  Bit for bit
    with the oracle at a sample of rows (each row's quantization and sums
    depend on that row alone), and every row within the reference's bound."""
    K, N, M, B = 5120, 1280, 988, 2
    r = rng(5120)
    wh, w32 = weights_f16(r, (N, K), 0.02 * 1.7)
    x = uniform(r, (B, M, K), 1.0)
    b = uniform(r, (N,), 0.01)
    res = uniform(r, (B, M, N), 1.0)
    w_d, x_d, b_d, res_d = dev(wh, gpu), dev(x, gpu), dev(b, gpu), dev(res, gpu)
    y = unwritten((B, M, N), gpu)
    if from_redirect:
        out = res_d.clone()
        chain = sdhip.epilogue([("add", b_d)], redirect=out, from_redirect=True)
    else:
        out = unwritten((B, M, N), gpu)
        chain = sdhip.epilogue([("add", b_d), ("add", res_d)], redirect=out)
    sdhip.set_tuning("bits=8,weight_group=0")
    try:
        sdhip.mul_mat(w_d, x_d, y, chain)
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    got = out.cpu().numpy().reshape(B * M, N)
    assert torch.isnan(y).all(), "the product's own tensor is not written under a redirect"
    xs = x.reshape(B * M, K)
    rows = np.unique(np.concatenate([np.arange(0, 8), rng(7).integers(0, B * M, 56), [B * M - 1]]))
    rs = res.reshape(B * M, N)[rows]
    if from_redirect:
        want = orc.quantized_mul_mat(w32, xs[rows], 64, 255, 127, 0, init=rs)[0]
        want = (want + b).astype(np.float32)
    else:
        want = orc.quantized_mul_mat(w32, xs[rows], 64, 255, 127, 0)[0]
        want = ((want + b).astype(np.float32) + rs).astype(np.float32)
    same = np.array_equal(got[rows].view(np.uint32), want.view(np.uint32))
    print(f"FF-out 5120->1280 x {B * M} (from_redirect={from_redirect}): {rows.size} rows bit-exact: {same}")
    assert same, f"{np.sum(got[rows] != want)} of {want.size} differ"
    exact, mag = orc.exact_mul_mat(w32, xs[rows])
    add = b.astype(np.float64) + rs
    assert orc.metric(got[rows], exact + add, mag + np.abs(add)) <= bound(255, 127)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,M", [(77, 100, 300), (40, 2560, 296)])  # ops_test.cc:878, 880
@pytest.mark.parametrize("tuning", ["bits=8", "bits=8,weight_group=0", "bits=7"])
def test_quantized_single_precision_weights(gpu, K, N, M, tuning):
    """The bits mode with single-precision weights: quantize_weights_f32
    (quant.cc:373-380), the same quantizer of the weights as they are; bit
    for bit with the oracle's restatement."""
    group, levels, wmax, wg = quant_params(tuning)
    r = rng(K + N + M + 5)
    w = uniform(r, (N, K), 0.25)
    x = uniform(r, (M, K), 1.0)
    b = uniform(r, (N,), 1.0)
    w_d, x_d, b_d = dev(w, gpu), dev(x, gpu), dev(b, gpu)
    y = unwritten((M, N), gpu)
    sdhip.set_tuning(tuning)
    try:
        sdhip.mul_mat(w_d, x_d, y, sdhip.epilogue([("add", b_d)]))
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    got = y.cpu().numpy()
    want = (orc.quantized_mul_mat(w, x, group, levels, wmax, wg)[0] + b).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    exact, mag = orc.exact_mul_mat(w, x)
    assert orc.metric(got, exact + b, mag + np.abs(b)) <= bound(levels, wmax)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,M,B", [(320, 320, 512, 2), (77, 100, 300, 1), (300, 17, 131, 3), (1280, 1280, 988, 2),
                                     (5120, 1280, 300, 1)])
@pytest.mark.parametrize("tuning", ["bits=8", "bits=8,weight_group=0", "bits=8,group=128", "bits=8,group=32",
                                    "bits=7,input_bits=7"])
def test_quantized_cores_agree(gpu, K, N, M, B, tuning):
    """The products through a ring of LDS stages (qgemm_core=2, the default)
    give the bits of the 64 x 64 kernel (qgemm_core=1): the integer sums are
    exact whatever the order of k, and the dequantisation is the same
    sequence of operations."""
    w32, x, b, y1 = run_quantized(gpu, K, N, M, B, tuning + ",qgemm_core=1", seed=K + N)
    _, _, _, y2 = run_quantized(gpu, K, N, M, B, tuning + ",qgemm_core=2", seed=K + N)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("K,half,M", [(320, 1280, 400), (96, 2000, 300), (1280, 5120, 300)])
def test_quantized_gated_cores_agree(gpu, K, half, M):
    """The gated GELU after the quantized products, both kernels, bit for bit."""
    r = rng(K + half)
    wh, _ = weights_f16(r, (2 * half, K))
    x = uniform(r, (M, K), 1.0)
    b = uniform(r, (2 * half,), 1.0)
    w_d, x_d, b_d = dev(wh, gpu), dev(x, gpu), dev(b, gpu)
    outs = []
    for core in (1, 2):
        y = unwritten((M, 2 * half), gpu)
        out = unwritten((M, half), gpu)
        sdhip.set_tuning(f"bits=8,qgemm_core={core}")
        try:
            sdhip.mul_mat_gated(w_d, x_d, y, out, sdhip.epilogue([("add", b_d)]))
            torch.cuda.synchronize()
        finally:
            sdhip.set_tuning("")
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
