"""MUL_MAT and its gated GELU on the device against the float64 oracle, by the
reference's metric (|y - exact| / sum of |products|, ops_test.cc:154-211),
at the reference's own test shapes (ops_test.cc:825-832, 900-903) and the
SD1.5 linear layer of the bench configuration."""

import numpy as np
import pytest
import torch

import oracle_lib as orc
import sdhip
from helpers import dev, rng, uniform, unwritten, weights_f16

# The bound the library is held to: 2e-5 of the magnitudes for GEMM and
# convolution.  The split-FP16 products reach a few 1e-7; BOUND_SPLIT holds
# them to that, so that a loss of the low part shows.
BOUND = 2e-5
BOUND_SPLIT = 2e-6

CASES = [  # K, N, M, batch
    (320, 320, 512, 2),
    (768, 1280, 77, 2),
    (1280, 320, 64, 1),
    (300, 17, 31, 3),
    (320, 320, 4096, 2),  # SD1.5 linear 320 -> 320, the bench's MUL_MAT
    (77, 100, 23, 1),     # K of no multiple of 8
]


def run_mul_mat(gpu, K, N, M, B, seed, chain_steps=(), redirect=None, from_redirect=False):
    r = rng(seed)
    wh, w32 = weights_f16(r, (N, K))
    x = uniform(r, (B, M, K), 1.0)
    w_d = dev(wh, gpu)
    x_d = dev(x, gpu)
    y_d = unwritten((B, M, N), gpu)
    chain = sdhip.epilogue(chain_steps, redirect=redirect, from_redirect=from_redirect)
    sdhip.mul_mat(w_d, x_d, y_d, chain)
    torch.cuda.synchronize()
    exact, mag = orc.exact_mul_mat(w32, x.reshape(B * M, K))
    return y_d, exact.reshape(B, M, N), mag.reshape(B, M, N)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,M,B", CASES)
def test_mul_mat(gpu, K, N, M, B):
    y, exact, mag = run_mul_mat(gpu, K, N, M, B, seed=K * 7 + N)
    err = orc.metric(y.cpu().numpy(), exact, mag)
    print(f"mul_mat {K}->{N} x {M}x{B}: {err:.3g}")
    assert err <= BOUND_SPLIT <= BOUND


@pytest.mark.gpu
def test_mul_mat_bias_chain(gpu):
    """linear + bias (+ a per-token scale), fused (fusion.cc:136-199)."""
    K, N, M, B = 96, 70, 50, 2
    r = rng(11)
    bias = dev(uniform(r, (N,), 1.0), gpu)
    scale = dev(uniform(r, (B, M, 1), 1.0), gpu)
    y, exact, mag = run_mul_mat(gpu, K, N, M, B, 5, [("add", bias), ("mul", scale)])
    b = bias.cpu().numpy().astype(np.float64)
    s = scale.cpu().numpy().astype(np.float64)
    want = (exact + b) * s
    m2 = (mag + np.abs(b)) * np.abs(s)
    assert orc.metric(y.cpu().numpy(), want, m2) <= BOUND_SPLIT


@pytest.mark.gpu
@pytest.mark.parametrize("from_redirect", [False, True])
def test_mul_mat_residual(gpu, from_redirect):
    """linear + bias + residual into a tensor of its own; or begun from the
    residual already in that tensor (Epilogue::redirect / from_redirect)."""
    K, N, M, B = 300, 70, 1100, 2
    r = rng(12)
    bias = dev(uniform(r, (N,), 1.0), gpu)
    res = uniform(r, (B, M, N), 1.0)
    res_d = dev(res, gpu)
    if from_redirect:
        out = res_d.clone()
        y, exact, mag = run_mul_mat(gpu, K, N, M, B, 6, [("add", bias)], redirect=out, from_redirect=True)
    else:
        out = unwritten((B, M, N), gpu)
        y, exact, mag = run_mul_mat(gpu, K, N, M, B, 6, [("add", bias), ("add", res_d)], redirect=out)
    b = bias.cpu().numpy().astype(np.float64)
    want = exact + b + res
    m2 = mag + np.abs(b) + np.abs(res)
    assert torch.isnan(y).all(), "the product's own tensor is not written under a redirect"
    assert orc.metric(out.cpu().numpy(), want, m2) <= BOUND_SPLIT


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,M,B", [
    (4096, 200, 150, 2),   # 20 blocks of 64 x 64: 16 splits of 8 K-steps (256), all alike
    (2336, 200, 150, 1),   # 12 blocks, 73 K-steps: 8 splits of 9 steps and a last one of a single step
    (1280, 1280, 256, 2),  # panels of 64 x 160 split along K: 64 panels, 4 splits of 5 chunks of 64
    (2560, 320, 77, 2),    # 6 panels, splits of chunks, rows past M in the last panel
    (2240, 640, 100, 1),   # 35 chunks: splits of 5, the panels' last ragged in M
])
@pytest.mark.parametrize("from_redirect", [False, True])
def test_mul_mat_split_chain(gpu, from_redirect, K, N, M, B):
    """A product of few output blocks and long K, split along K (about 512
    blocks, each split 8 K-steps of 32 or more, the last one what is left;
    where K and N take them, panels of 64 x 160 split along K into as many):
    the splits' sums added with bias, a per-token scale and a residual (or
    begun from the residual), the epilogue of the single pass."""
    r = rng(13 + K)
    bias = dev(uniform(r, (N,), 1.0), gpu)
    scale = dev(uniform(r, (B, M, 1), 1.0), gpu)
    res = uniform(r, (B, M, N), 1.0)
    res_d = dev(res, gpu)
    b = bias.cpu().numpy().astype(np.float64)
    s = scale.cpu().numpy().astype(np.float64)
    if from_redirect:
        out = res_d.clone()
        y, exact, mag = run_mul_mat(gpu, K, N, M, B, 7, [("add", bias), ("mul", scale)], redirect=out,
                                    from_redirect=True)
        want = (res + exact + b) * s
        m2 = (np.abs(res) + mag + np.abs(b)) * np.abs(s)
    else:
        out = unwritten((B, M, N), gpu)
        y, exact, mag = run_mul_mat(gpu, K, N, M, B, 7, [("add", bias), ("mul", scale), ("add", res_d)],
                                    redirect=out)
        want = (exact + b) * s + res
        m2 = (mag + np.abs(b)) * np.abs(s) + np.abs(res)
    assert torch.isnan(y).all(), "the product's own tensor is not written under a redirect"
    assert orc.metric(out.cpu().numpy(), want, m2) <= BOUND_SPLIT


@pytest.mark.gpu
@pytest.mark.parametrize("K,half,M,B", [(320, 1280, 200, 2), (40, 100, 37, 1), (96, 2000, 300, 1),
                                        (1280, 5120, 64, 2)])
def test_gated(gpu, K, half, M, B):
    """GEGLU after a linear layer with bias (ops_test.cc:731-779)."""
    r = rng(K + half)
    wh, w32 = weights_f16(r, (2 * half, K))
    x = uniform(r, (B, M, K), 1.0)
    bias = uniform(r, (2 * half,), 1.0)
    w_d, x_d, b_d = dev(wh, gpu), dev(x, gpu), dev(bias, gpu)
    y_d = unwritten((B, M, 2 * half), gpu)
    out = unwritten((B, M, half), gpu)
    sdhip.mul_mat_gated(w_d, x_d, y_d, out, sdhip.epilogue([("add", b_d)]))
    torch.cuda.synchronize()
    exact, mag = orc.exact_gated(w32, x.reshape(B * M, K), bias)
    err = orc.metric(out.cpu().numpy(), exact, mag)
    print(f"gated {K}->2x{half} x {M}x{B}: {err:.3g}")
    assert err <= BOUND_SPLIT
    assert torch.isnan(y_d).all(), "the product itself is never written"


F32_CASES = [  # K, N, M, batch: the reference's single-precision cases (ops_test.cc:829, 831) and SD1.5's
    (77, 100, 23, 1),
    (40, 2560, 96, 1),
    (320, 320, 512, 2),
    (1280, 320, 300, 1),
]


def weights_f32(r, shape, scale=0.25):
    """Single-precision weights: no FP16 rounding (the reference's
    GGML_TYPE_F32 weights, mul_mat.cc:190)."""
    return uniform(r, shape, scale)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,M,B", F32_CASES)
def test_mul_mat_single_precision_weights(gpu, K, N, M, B):
    """Single-precision weights, taken as the reference takes them
    (mul_mat.cc:181-194): split into two FP16 planes with a power-of-two
    scale per row, three MFMAs a product; the bias fused.  Rows of very
    different magnitudes (2^-20 .. 2^12) check the per-row scale."""
    r = rng(K + 3 * N)
    w = weights_f32(r, (N, K))
    w *= (2.0 ** r.integers(-20, 13, size=(N, 1))).astype(np.float32)
    x = uniform(r, (B, M, K), 1.0)
    b = uniform(r, (N,), 1.0)
    w_d, x_d, b_d = dev(w, gpu), dev(x, gpu), dev(b, gpu)
    assert sdhip.load().sdhip_mul_mat_supported(sdhip.desc(w_d), sdhip.desc(x_d), sdhip.desc(unwritten((B, M, N), gpu)))
    y = unwritten((B, M, N), gpu)
    sdhip.mul_mat(w_d, x_d, y, sdhip.epilogue([("add", b_d)]))
    torch.cuda.synchronize()
    exact, mag = orc.exact_mul_mat(w, x.reshape(B * M, K))
    err = orc.metric(y.cpu().numpy().reshape(B * M, N), exact + b, mag + np.abs(b))
    print(f"mul_mat single-precision weights {K}->{N} x {M}x{B}: {err:.3g}")
    assert err <= BOUND_SPLIT


@pytest.mark.gpu
@pytest.mark.parametrize("K,half,M", [(320, 1280, 200), (40, 100, 37)])
def test_gated_single_precision_weights(gpu, K, half, M):
    r = rng(K + half + 1)
    w = weights_f32(r, (2 * half, K))
    x = uniform(r, (M, K), 1.0)
    bias = uniform(r, (2 * half,), 1.0)
    w_d, x_d, b_d = dev(w, gpu), dev(x, gpu), dev(bias, gpu)
    y_d = unwritten((M, 2 * half), gpu)
    out = unwritten((M, half), gpu)
    sdhip.mul_mat_gated(w_d, x_d, y_d, out, sdhip.epilogue([("add", b_d)]))
    torch.cuda.synchronize()
    exact, mag = orc.exact_gated(w, x, bias)
    err = orc.metric(out.cpu().numpy(), exact, mag)
    print(f"gated single-precision weights {K}->2x{half} x {M}: {err:.3g}")
    assert err <= BOUND_SPLIT


PANEL_CASES = [  # K, N, M, B: outputs of 256 panels and more, of 64 x 160 or 64 x 64
    (320, 320, 4096, 2),   # 64 x 160, whole panels: the fast epilogue
    (640, 480, 4050, 2),   # 64 x 160, ragged M (8100 tokens): rows past M read the last one
    (384, 400, 8192, 1),   # 64 x 160, ragged N: features past N, the general epilogue
    (640, 640, 1024, 2),   # 64 x 64 (the UNet's 32 x 32 level)
    (2560, 600, 1000, 2),  # 64 x 64, long K, ragged M and N
]


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,M,B", PANEL_CASES)
@pytest.mark.parametrize("form", ["bias_scale_residual", "from_redirect", "misaligned"])
def test_mul_mat_panels(gpu, K, N, M, B, form):
    """The panel core (mul_mat_panels, outputs of many panels) through both of
    its epilogues: a bias, a per-token scale and a residual (contiguous, or
    one number a token: the fast epilogue where N is whole panels); the sum
    begun from the residual in the output's memory; an operand whose rows are
    not 16-byte aligned (the general epilogue).  Against float64,
    and within the same bound of the 64 x 64 core (mul_mat_panels=0)."""
    r = rng(K + N + M)
    bias = uniform(r, (N,), 1.0)
    scale = uniform(r, (B, M, 1), 1.0)
    res = uniform(r, (B, M, N), 1.0)
    bias_d, scale_d, res_d = dev(bias, gpu), dev(scale, gpu), dev(res, gpu)
    outs = []
    for tuning in ("", "mul_mat_panels=0"):
        sdhip.set_tuning(tuning)
        try:
            if form == "bias_scale_residual":
                y, exact, mag = run_mul_mat(gpu, K, N, M, B, 3, [("add", bias_d), ("mul", scale_d), ("add", res_d)])
                b, s = bias.astype(np.float64), scale.astype(np.float64)
                want, m2 = (exact + b) * s + res, (mag + np.abs(b)) * np.abs(s) + np.abs(res)
                got = y.cpu().numpy()
            elif form == "from_redirect":
                out = res_d.clone()
                y, exact, mag = run_mul_mat(gpu, K, N, M, B, 3, [("add", bias_d)], redirect=out, from_redirect=True)
                b = bias.astype(np.float64)
                want, m2 = res + exact + b, np.abs(res) + mag + np.abs(b)
                got = out.cpu().numpy()
            else:
                # The residual as a view one float into rows of N + 1: rows
                # not 16-byte aligned, the general epilogue.
                wide = np.zeros((B, M, N + 1), np.float32)
                wide[..., 1:] = res
                rv = dev(wide, gpu)[..., 1:]
                y, exact, mag = run_mul_mat(gpu, K, N, M, B, 3, [("add", rv)])
                want, m2 = exact + res, mag + np.abs(res)
                got = y.cpu().numpy()
        finally:
            sdhip.set_tuning("")
        err = orc.metric(got, want, m2)
        print(f"panels {K}->{N} x {M}x{B} [{form}] {tuning or 'panels'}: {err:.3g}")
        assert err <= BOUND_SPLIT
        outs.append(got)
    assert orc.metric(outs[0], outs[1], m2) <= BOUND_SPLIT
