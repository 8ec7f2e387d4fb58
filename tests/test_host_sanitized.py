"""The library's host code -- predicates, work sizes, path choice, the graph
planner, the tuning's parser -- under AddressSanitizer and
UndefinedBehaviorSanitizer, driven by tests/host_check.cpp with randomized
descriptors, graphs and tuning strings (built by `make host_check`, which
__graft_entry__.build() runs).  No GPU is touched."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "stable-diffusion.assembly_amd", "_build", "host_check")


@pytest.mark.skipif(not os.path.exists(BINARY), reason="make -C stable-diffusion.assembly_amd host_check first")
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_host_code_sanitized(seed):
    run = subprocess.run([BINARY, "30000", str(seed)], capture_output=True, text=True, timeout=300)
    report = (run.stdout + run.stderr)[-4000:]
    assert run.returncode == 0, report
    assert "no error" in run.stdout, report
