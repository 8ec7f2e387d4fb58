"""A whole UNet step through the library (unet_step.py) on the GPU, at a
reduced size, against the same step in float64 torch on the CPU; and the
HIP-graph replay of the step against its eager run, replay after replay."""

import pytest
import torch

import unet_step as u
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
                                             ("bits=8", 1e-5, 1e-2)])
def test_sdxl_block(gpu, tuning, low, high):
    """The SDXL transformer block at a reduced size -- 300
    tokens, so that its self-attention is quantized too -- against float64
    torch: in single precision within 1e-5 of the output's norm, in the bits
    mode within the quantization's error (and measurably quantized)."""
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
