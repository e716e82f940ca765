"""pytest configuration: the `gpu` marker and import paths.

GPU tests call the HIP library through its C ABI on a real MI355X and compare
with the CPU oracle; CPU tests cover the oracle, the ABI contract and the host
logic.  Run `python -m pytest tests -m "not gpu"` without a GPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("flash-attention3_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
