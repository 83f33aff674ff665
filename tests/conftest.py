"""Shared pytest setup: the package directory is put on sys.path so its flat modules (mxfp8, fused_mlp,
fused_linear, workloads) import the way the reference's scripts/ modules do; the repo root is on sys.path so
``oracle`` imports as a package."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "train-model-template_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def _fresh_cast_cache():
    """Each test starts a new 'training step': the per-step bf16 cast cache of fused_linear is keyed by id() of the
    parameters (fused_linear.py:55-69), so entries left by an earlier test could alias a new tensor at a recycled
    address.  The training loop clears it with new_step() at every step; so do the tests."""
    import fused_linear
    fused_linear.new_step()
    yield
