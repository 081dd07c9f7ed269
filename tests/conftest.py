import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU and the built HIP library")


@pytest.fixture(scope="session")
def device():
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm device is visible")
    return torch.device("cuda:0")


def assert_close_rel(actual, expected, rtol=1e-2, atol_frac=1e-3, name=""):
    """|a-e| <= rtol*|e| + atol_frac*max|e| elementwise, in float64."""
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    assert a.shape == e.shape, (name, a.shape, e.shape)
    assert torch.isfinite(a).all(), f"{name}: non-finite values in actual"
    scale = e.abs().max().item()
    err = (a - e).abs()
    bound = rtol * e.abs() + atol_frac * scale
    bad = err > bound
    if bad.any():
        idx = torch.nonzero(bad)[0].tolist()
        raise AssertionError(
            f"{name}: {int(bad.sum())} of {bad.numel()} elements out of tolerance; "
            f"max err {err.max().item():.3e} (scale {scale:.3e}); first bad {idx}: "
            f"actual {a[tuple(idx)].item():.6e} expected {e[tuple(idx)].item():.6e}")
    return err.max().item() / max(scale, 1e-30)
