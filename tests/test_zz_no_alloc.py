"""sdhip_group_norm_static, the entry point that allocates nothing: its
partial sums in the library's static scratch instead of a caller's work
buffer.  Against sdhip_group_norm (the same kernels with a work buffer), bit
for bit, on two calls in a row, the second of a smaller input -- the scratch
keeps the first call's sums, which the second must not read -- each with the
reference's chain after a group norm (scale, shift, SiLU), and both of shapes
whose groups take the partial sums (not the one-launch path of small groups).
A shape whose sums need more than the scratch holds is refused."""

import numpy as np
import pytest
import torch

import sdhip
from helpers import dev, normal, rng, unwritten


def run_both(gpu, shape, groups, seed):
    r = rng(seed)
    x = normal(r, shape)
    n, c = shape[0], shape[1]
    gam = normal(r, (1, c, 1, 1), 1.0, 0.1)
    bet = normal(r, (1, c, 1, 1), 0.0, 0.1)
    x_d, g_d, b_d = dev(x, gpu), dev(gam, gpu), dev(bet, gpu)
    chain = sdhip.epilogue([("mul", g_d), ("add", b_d), ("silu", None)])
    lib = sdhip.load()
    assert lib.sdhip_group_norm_work_size(sdhip.desc(x_d), sdhip.desc(x_d), groups) > 0
    want = unwritten(shape, gpu)
    sdhip.group_norm(x_d, want, groups, 1e-5, chain)
    got = unwritten(shape, gpu)
    sdhip.group_norm_static(x_d, got, groups, 1e-5, chain)
    torch.cuda.synchronize()
    return got.cpu().numpy(), want.cpu().numpy()


@pytest.mark.gpu
def test_static_group_norm_matches_the_work_buffer_form(gpu):
    for shape, groups, seed in (((2, 320, 64, 64), 32, 1), ((1, 640, 32, 32), 32, 2)):
        got, want = run_both(gpu, shape, groups, seed)
        same = np.array_equal(got.view(np.uint32), want.view(np.uint32))
        print(f"group_norm_static {shape} groups {groups}: bit-identical {same}")
        assert np.isfinite(got).all()
        assert same


@pytest.mark.gpu
def test_static_group_norm_refuses_more_than_its_scratch(gpu):
    x = torch.zeros((1, 70000, 1, 4), device=gpu)
    y = torch.zeros_like(x)
    need = sdhip.load().sdhip_group_norm_work_size(sdhip.desc(x), sdhip.desc(y), 70000)
    assert need > (1 << 20)
    with pytest.raises(sdhip.SdhipError) as e:
        sdhip.group_norm_static(x, y, 70000, 1e-5)
    assert e.value.status == sdhip.ERROR
    assert "static scratch" in str(e.value)
