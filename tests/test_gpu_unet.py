"""A whole UNet step through the library (unet_step.py) on the GPU, at a
reduced size, against the same step in float64 torch on the CPU; and the
HIP-graph replay of the step against its eager run, replay after replay."""

import numpy as np
import pytest
import torch

import oracle_lib as orc
import unet_step as u
from test_gpu_quant import quant_params
from test_unet import small_config


@pytest.mark.gpu
def test_unet_step_matches_float64(gpu):
    m = u.Model(small_config(), gpu, seed=3)
    x, t, c = m.inputs(seed=4)
    ops = u.HipOps(gpu)
    y = m.forward(ops, x, t, c)
    torch.cuda.synchronize()
    assert ops.nodes["conv3x3"] > 0 and ops.nodes["attention"] > 0
    ref = m.to_reference("cpu")
    y64 = ref.forward(u.TorchOps(torch.float64), x.cpu().double(), t.cpu(), c.cpu().double())
    err = ((y.cpu().double() - y64).norm() / y64.norm()).item()
    worst = ((y.cpu().double() - y64).abs().max() / y64.abs().max()).item()
    print(f"unet step (small): relative L2 error {err:.3g}, max {worst:.3g}")
    assert err < 2e-5 and worst < 1e-4


@pytest.mark.gpu
def test_unet_graph_replays_equal_eager(gpu):
    m = u.Model(small_config(), gpu, seed=5)
    ops = u.HipOps(gpu)
    step = u.Step(m, ops, m.inputs(seed=6))
    eager = step.eager().clone()
    for i in range(3):
        out = step.run().clone()
        torch.cuda.synchronize()
        other = step.eager()  # the program's own eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from the eager step"
        assert torch.equal(other, eager)


@pytest.mark.gpu
@pytest.mark.parametrize("tuning,low,high", [("", 0.0, 1e-5), ("bits=8,weight_group=0", 1e-5, 1e-2),
                                             ("bits=8", 1e-5, 1e-2), ("bits=16", 2e-6, 1e-4),
                                             ("bits=16,half_format=1", 5e-5, 1e-3)])
def test_sdxl_block(gpu, tuning, low, high):
    """The SDXL transformer block at a reduced size -- 300
    tokens, so that its self-attention is quantized too -- against float64
    torch: in single precision within 1e-5 of the output's norm, in the bits
    mode within the quantization's error (and measurably quantized); with
    products of 16 bits, the FP16 form (x rounded to FP16, attention single
    precision) and the bfloat16 form (both operands and attention's rounded to
    bfloat16), each measurably rounded and the bfloat16 one the coarser."""
    import sdhip

    block = u.SdxlBlock(gpu, channels=256, heads=4, seed=2)
    x = torch.randn((1, 300, 256), generator=torch.Generator(device=gpu).manual_seed(3), device=gpu)
    ops = u.HipOps(gpu)
    sdhip.set_tuning(tuning)
    try:
        y = block.forward(ops, x)
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    ref = u.SdxlBlock("cpu", channels=256, heads=4, seed=2)
    for name in ("ln1", "ln2", "wq", "wk", "wv", "wo", "ff1", "ff2"):
        setattr(ref, name, tuple(t.cpu() for t in getattr(block, name)) if isinstance(getattr(block, name), tuple)
                else getattr(block, name).cpu())
    y64 = ref.forward(u.TorchOps(torch.float64), x.cpu().double())
    err = ((y.cpu().double() - y64).norm() / y64.norm()).item()
    print(f"sdxl block [{tuning or 'single precision'}]: relative L2 error {err:.3g}")
    assert low <= err <= high


class OracleOps:
    """The SDXL block's nodes in the bits mode, each by the oracle's
    restatement of the reference's own (norm.cc:92-175, quant.cc:113-164 with
    mul_mat.cc:498-646, attention.cc:612-824, fusion.cc:290-310), in single
    precision on the CPU: the chains' additions and products in float32 in
    the order the library's chains take them."""

    def __init__(self, tuning):
        self.group, self.levels, self.wmax, self.wg = quant_params(tuning)

    @staticmethod
    def _f32(t):
        return t.detach().cpu().float().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, np.float32)

    def layer_norm(self, x, eps, gamma, beta):
        n = orc.norm(x, eps)
        return (n * self._f32(gamma)).astype(np.float32) + self._f32(beta)

    def _product(self, x, w, bias):
        k = w.shape[1]
        rows = x.reshape(-1, k)
        assert rows.shape[0] >= 256, "the bits mode quantizes products of 256 rows and more"
        y = orc.quantized_mul_mat(self._f32(w), rows, self.group, self.levels, self.wmax, self.wg)[0]
        if bias is not None:
            y = (y + self._f32(bias)).astype(np.float32)
        return y.reshape(*x.shape[:-1], w.shape[0])

    def linear(self, x, w, bias=None, add=()):
        y = self._product(x, w, bias)
        for a in add:
            y = (y + a).astype(np.float32)
        return y

    def geglu(self, x, w, bias):
        p = self._product(x, w, bias)
        half = p.shape[-1] // 2
        return orc.gated_gelu(np.ascontiguousarray(p[..., :half]), np.ascontiguousarray(p[..., half:]))

    def attention(self, q, k, v, heads):
        b, lq, c = q.shape
        d = c // heads
        scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
        views = [t.reshape(b, t.shape[1], heads, d) for t in (q, k, v)]
        y = orc.quantized_attention(*views, scale, self.group, self.levels, self.wmax, key_block=256)
        return y.reshape(b, lq, c)


@pytest.mark.gpu
@pytest.mark.parametrize("tuning", ["bits=8,weight_group=0", "bits=8"])
def test_sdxl_block_against_the_oracle(gpu, tuning):
    """The SDXL block in the bits mode (configs[4]'s, at 300 tokens by 256
    channels) against the same block composed of the oracle's nodes: every
    product quantized as the reference quantizes it, the self-attention's
    included.  The nodes agree bit for bit or within 1e-5 one by one (the
    attention's double sums aside); composed, a number that lands on a
    quantization step's edge may round the other way, so the block is held
    to 1e-5 of its norm (measured: 7e-7 and 2e-8, 94 .. 96% of the outputs
    bit-identical) -- where float64 is 6e-4 away."""
    import sdhip

    block = u.SdxlBlock(gpu, channels=256, heads=4, seed=2)
    x = torch.randn((1, 300, 256), generator=torch.Generator(device=gpu).manual_seed(3), device=gpu)
    ops = u.HipOps(gpu)
    sdhip.set_tuning(tuning)
    try:
        y = block.forward(ops, x)
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    want = block.forward(OracleOps(tuning), x.cpu().numpy())
    got = y.cpu().numpy()
    err = float(np.linalg.norm((got - want).astype(np.float64)) / np.linalg.norm(want.astype(np.float64)))
    same = float(np.mean(got.view(np.uint32) == want.view(np.uint32)))
    print(f"sdxl block [{tuning}] against the oracle: relative L2 {err:.3g}, {same:.2%} bit-identical")
    assert np.isfinite(got).all()
    assert err <= 1e-5
