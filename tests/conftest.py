"""Test configuration.

Two tiers:
  * ``-m "not gpu"`` -- runs anywhere: the oracle against upstream aten CPU
    kernels, golden vectors, closed forms and invariants; the planner and the
    magic-number divider against brute force; the C-ABI library's exports.
  * ``-m gpu`` -- parity of the HIP path (through the C ABI and through the
    PrivateUse1 dispatcher) against the oracle on an MI355X.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "torch-supa_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def supa():
    """The supa backend on a GPU box; fails loudly when the build is missing."""
    import torch
    import torch_supa  # noqa: F401

    assert torch.supa.is_available(), "no supa (HIP) device visible"
    return torch


@pytest.fixture
def no_fallback(supa):
    """Run a test with the CPU fallback disabled and check nothing used it."""
    supa.supa.set_cpu_fallback_enabled(False)
    supa.supa.reset_fallback_counts()
    yield
    counts = supa.supa.fallback_counts()
    supa.supa.set_cpu_fallback_enabled(True)
    assert counts == {}, f"ops went through the CPU fallback: {counts}"


@pytest.fixture
def fused_ce(supa):
    """Route cross_entropy through the fused kernels (every dtype) for one
    test, then restore the routing it found."""
    was = supa.supa.fused_cross_entropy_enabled()
    supa.supa.set_fused_cross_entropy_enabled(True)
    yield
    supa.supa.set_fused_cross_entropy_enabled(was)
