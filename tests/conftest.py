import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "stable-diffusion.assembly_amd")
for p in (PKG, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950); runs the HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The device, with the library loaded and initialised on it.  No
    fallback: a missing library or device fails the test."""
    import torch

    import sdhip

    assert torch.cuda.is_available(), "no GPU: the gpu tests need an MI355X"
    lib = sdhip.load()
    sdhip.check(lib.sdhip_init(0), "init")
    sdhip.set_tuning("")
    return torch.device("cuda", 0)
