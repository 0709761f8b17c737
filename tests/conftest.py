"""Shared test setup: import paths, the ``gpu`` marker and tolerance helpers."""
import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "ictc-o3-hp-ascend_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

# fp32 relative tolerance of the hot path against the float64 oracle (north star: 1e-5).
RTOL = 1e-5
# forces (derivatives of a summed energy) are compared at 1e-4.
RTOL_FORCE = 1e-4


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built libictc_hip.so")


def max_rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    """max |a - b| / max |b| (0 for two empty tensors)."""
    a, b = actual.detach().double().cpu(), expected.detach().double().cpu()
    assert a.shape == b.shape, (a.shape, b.shape)
    if b.numel() == 0:
        return 0.0
    scale = b.abs().max().item()
    return (a - b).abs().max().item() / (scale if scale > 0 else 1.0)


def assert_rel(actual, expected, rtol=RTOL, what=""):
    err = max_rel_err(actual, expected)
    assert err <= rtol, f"{what}: relative error {err:.3e} > {rtol:.1e}"


@pytest.fixture(scope="session")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda", 0)
