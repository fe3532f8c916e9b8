"""Shared pytest setup: the `gpu` marker, import paths and session fixtures.

CPU tests (`-m "not gpu"`) exercise the oracle, the golden fixtures, the host
logic and the C ABI's exports / argument checks. GPU tests (`-m gpu`) run the
HIP kernels through the C ABI and compare them with the oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bonsai-ternary-fast_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs HIP kernels on an MI355X (gfx950)")


@pytest.fixture(scope="session")
def oracle():
    from btf_oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from btf_oracle import Ref, have_ref
    if not have_ref():
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    return Ref()


@pytest.fixture(scope="session")
def hip():
    """The HIP library on device 0 (kernels_init done)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this process")
    import btf_hip
    torch.cuda.init()
    btf_hip.kernels_init(0)
    return btf_hip
