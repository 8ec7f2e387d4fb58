"""The bits mode of self-attention (attention.cc:597-824) on the device,
against the oracle's restatement of it and against float64.

The device quantizes the keys, queries, values and exponentials bit for bit as
the reference's C++ form does, and sums the same integers in the same group
order, so its outputs are the oracle's but for the double-precision sum of the
exponentials (summed in another order: a rounding of float(1 / sum) at most)
and the few keys past the last multiple of 8 of the last stretch, whose
exponential is std::exp's -- glibc's expf on the CPU, the correctly rounded
value on the device, which differ in rare last bits.  The tests hold the
device within 1e-5 of the oracle (the north star's bound against the
reference's cxx output), report how many outputs are bit-identical, and hold
it to the reference's own bound against float64 (ops_test.cc:213-240)."""

import numpy as np
import pytest
import torch

import oracle_lib as orc
import sdhip
from helpers import dev, rng, uniform, unwritten
from test_gpu_quant import bound, quant_params

APART = 1e-5

CASES = [  # d, lq, lk, h, hk, b, FP16 keys and values (ops_test.cc:912-918, the SDXL block's)
    (40, 300, 4096, 2, 2, 2, False),
    (80, 100, 1024, 2, 2, 1, True),
    (160, 64, 256, 2, 2, 2, False),
    (13, 37, 290, 4, 2, 3, False),
    (64, 988, 988, 4, 4, 1, False),
]


def run(gpu, c, tuning, seed):
    d, lq, lk, h, hk, b, half = c
    r = rng(seed)
    q = uniform(r, (b, lq, h, d), 1.0)
    k = uniform(r, (b, lk, hk, d), 1.0)
    v = uniform(r, (b, lk, hk, d), 1.0)
    if half:
        k, v = k.astype(np.float16), v.astype(np.float16)
    q_d, k_d, v_d = dev(q, gpu), dev(k, gpu), dev(v, gpu)
    y = unwritten((b, lq, h, d), gpu)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    sdhip.set_tuning(tuning)
    try:
        sdhip.attention(q_d.permute(0, 2, 1, 3), k_d.permute(0, 2, 1, 3), v_d.permute(0, 2, 1, 3), y, scale)
        torch.cuda.synchronize()
    finally:
        sdhip.set_tuning("")
    return q, k.astype(np.float32), v.astype(np.float32), y.cpu().numpy(), scale


def key_block(tuning, group):
    t = dict(kv.split("=") for kv in tuning.split(",") if kv)
    keys = max(8, int(t.get("attention_keys", 256)) // 8 * 8)
    return max(group, keys // group * group)


@pytest.mark.gpu
@pytest.mark.parametrize("c", CASES, ids=lambda c: "x".join(map(str, c)))
@pytest.mark.parametrize("tuning", ["bits=8", "bits=7", "bits=8,input_bits=7", "bits=8,group=128",
                                    "bits=8,group=32", "bits=8,attention_keys=200"])
def test_quantized_attention(gpu, c, tuning):
    group, levels, wmax, _ = quant_params(tuning)
    q, k, v, y, scale = run(gpu, c, tuning, seed=sum(c[:3]))
    want = orc.quantized_attention(q, k, v, scale, group, levels, wmax, key_block(tuning, group))
    exact, mag = orc.exact_attention(q, k, v, scale)
    apart = orc.metric(y, want, mag)
    err = orc.metric(y, exact, mag)
    same = np.mean(y.view(np.uint32) == want.view(np.uint32))
    print(f"quantized attention {c} [{tuning}]: {apart:.3g} from the oracle ({same:.4%} bit-identical), "
          f"error {err:.3g} (bound {bound(levels, wmax):.3g})")
    assert np.isfinite(y).all()
    assert apart <= APART
    assert err <= bound(levels, wmax)


@pytest.mark.gpu
def test_cross_attention_stays_single_precision(gpu):
    """Fewer than 256 keys: not quantized (attention.cc:622-624)."""
    c = (40, 200, 77, 2, 2, 2, False)
    q, k, v, y, scale = run(gpu, c, "bits=8", seed=5)
    exact, mag = orc.exact_attention(q, k, v, scale)
    assert orc.metric(y, exact, mag) <= 1e-6


WIDE_AND_GROUPS = [  # case, tuning: heads to 512 dimensions and any group of keys quant() gives
    ((512, 64, 4096, 1, 1, 1, False), "bits=8"),              # the VAE's mid-block head (64 of its 4096 queries)
    ((512, 40, 1000, 1, 1, 1, False), "bits=8,group=20"),
    ((320, 50, 600, 2, 1, 1, True), "bits=8,group=300"),     # a group longer than 256 keys, FP16, GQA
    ((100, 70, 2100, 2, 2, 1, False), "bits=8,group=1024"),  # the longest group, 2100 keys in 3 groups
    ((100, 70, 700, 2, 2, 1, False), "bits=8,group=200"),
    ((40, 300, 4096, 2, 2, 2, False), "bits=8,group=20"),
    ((40, 100, 1000, 2, 2, 1, False), "bits=8,group=4"),
    ((13, 37, 290, 4, 2, 3, False), "bits=8,group=36"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("c,tuning", WIDE_AND_GROUPS, ids=lambda x: "x".join(map(str, x)) if isinstance(x, tuple)
                         else x)
def test_quantized_attention_wide_heads_and_any_group(gpu, c, tuning):
    """Heads of up to 512 dimensions (the keys' and queries' slots of up to 8
    steps of 64 bytes, the values' dimensions in chunks of 256 a workgroup)
    and groups of keys that are any multiple of 4 up to 1024 (quant.cc:59-67;
    attention.cc:612-664): tiles of 16 keys beginning at any multiple of 4,
    groups past 256 keys in parts.  Within 1e-5 of the oracle and the
    reference's bound of float64, as the other cases."""
    group, levels, wmax, _ = quant_params(tuning)
    q, k, v, y, scale = run(gpu, c, tuning, seed=sum(c[:3]) + group)
    want = orc.quantized_attention(q, k, v, scale, group, levels, wmax, key_block(tuning, group))
    exact, mag = orc.exact_attention(q, k, v, scale)
    apart = orc.metric(y, want, mag)
    err = orc.metric(y, exact, mag)
    same = np.mean(y.view(np.uint32) == want.view(np.uint32))
    print(f"quantized attention {c} [{tuning}]: {apart:.3g} from the oracle ({same:.4%} bit-identical), "
          f"error {err:.3g} (bound {bound(levels, wmax):.3g})")
    assert np.isfinite(y).all()
    assert apart <= APART
    assert err <= bound(levels, wmax)
