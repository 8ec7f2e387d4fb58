"""The synthetic SD1.5 UNet step (unet_step.py) on the CPU: its node and FLOP
inventory at 512x512 against the SD1.5 UNet's (the standard architecture:
52 3x3 and 46 1x1 convolutions, 32 attentions, 1606.5 GFLOP at batch 2),
counted on shapes alone; and the float64 checker against itself in float32
at a reduced size."""

import pytest
import torch

import unet_step as u


def test_sd15_inventory():
    m = u.Model(u.Config(), "meta")
    ops = u.TorchOps(torch.float32)
    x = torch.empty((2, 4, 64, 64), device="meta")
    t = torch.empty((2,), device="meta")
    c = torch.empty((2, 77, 768), device="meta")
    y = m.forward(ops, x, t, c)
    assert tuple(y.shape) == (2, 4, 64, 64)
    # 160 linear layers of the transformers, 2 of the time embedding and the
    # 22 ResBlocks' projections of it taken as one product: 163.
    assert ops.nodes == {"conv3x3": 52, "conv1x1": 46, "attention": 32, "linear": 163}
    g = {k: v / 1e9 for k, v in ops.by_class.items()}
    assert g["conv3x3"] == pytest.approx(800.65, abs=0.01)
    assert g["conv1x1"] == pytest.approx(87.24, abs=0.01)
    assert g["attention"] == pytest.approx(252.10, abs=0.01)
    assert g["linear"] == pytest.approx(466.55, abs=0.01)
    assert ops.flops / 1e9 == pytest.approx(1606.55, abs=0.01)


def small_config():
    # Every path of the library at a size the float64 checker runs in seconds:
    # 32x32 (F(4x4)), 16x16 (F(4x4), small), 8x8 (F(2x2)), strided and 1x1
    # direct convolutions, heads of 16 and 32 dimensions.
    return u.Config(channels=32, mult=(1, 2, 2), res_blocks=1, heads=2, attn_levels=(0, 1), context_dim=48,
                    context_len=8, latent=32, batch=2, groups=8)


def test_checker_float32_agrees_with_float64():
    m = u.Model(small_config(), "cpu", seed=3)
    x, t, c = m.inputs(seed=4, dtype=torch.float64)
    y64 = m.forward(u.TorchOps(torch.float64), x, t, c)
    y32 = m.forward(u.TorchOps(torch.float32), x.float(), t, c.float())
    err = ((y32.double() - y64).norm() / y64.norm()).item()
    assert err < 1e-5, err
    assert torch.isfinite(y64).all()
