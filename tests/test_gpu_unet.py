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
