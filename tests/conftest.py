"""Shared test setup: the `gpu` marker and import paths.

CPU tests (`-m "not gpu"`) pin the oracle, the golden fixtures, the host-side
logic and the C-ABI library's exports. GPU tests (`-m gpu`) are the parity
tests: the HIP kernels, called through the C ABI and the optimized/ package,
against the oracle on the same seeded inputs.
"""

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "distraction-optimizedtransformerlayer_amd")
for p in (REPO, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def kernels():
    """The loaded extension; fails (never skips) on a GPU box where it will not load."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import kernel_ext

    k = kernel_ext.get_kernels()
    if k is None:
        raise RuntimeError(f"libdotl_hip.so failed to load: {kernel_ext.load_error()}")
    return k
