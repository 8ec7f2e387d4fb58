"""Inputs as the reference's tests make them (tests/ops_test.cc:61-78):
uniform in [-0.25, 0.25] for weights (rounded to FP16) and [-1, 1] for the
rest -- from numpy's generator with a seed per case, not mt19937."""

import numpy as np
import torch

KUNWRITTEN = float("nan")


def rng(seed):
    return np.random.default_rng(seed)


def uniform(r, shape, scale):
    return r.uniform(-scale, scale, size=shape).astype(np.float32)


def weights_f16(r, shape, scale=0.25):
    """FP16 weights and their exact widening to float32."""
    h = uniform(r, shape, scale).astype(np.float16)
    return h, h.astype(np.float32)


def normal(r, shape, mean=0.0, std=1.0):
    return (mean + std * r.standard_normal(size=shape)).astype(np.float32)


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def unwritten(shape, device):
    return torch.full(shape, KUNWRITTEN, dtype=torch.float32, device=device)
