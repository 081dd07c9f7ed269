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


def assert_selection_gap_aware(scores, parents, tokens, keys, width, delta, name=""):
    """A top-``width`` selection judged against exact keys up to noise ``delta``.

    keys [B, Wp, V] float64 are the true candidate scores (log-softmax plus the
    parent score; -inf where masked); (scores, parents, tokens) [B, width] the
    selection under test.  Per request: the picks are distinct, sorted by score,
    each score within ``delta`` of its true key; every candidate whose key
    exceeds the width-th largest true key by more than ``delta`` is picked, and
    no pick lies more than ``delta`` below it.  Candidates inside that band are
    near-ties whose order the arithmetic's rounding may legitimately decide.
    Returns the number of picks that fell inside the band."""
    B, Wp, V = keys.shape
    s = scores.detach().double().cpu()
    p = parents.detach().long().cpu()
    t = tokens.detach().long().cpu()
    flat_keys = keys.reshape(B, -1)
    in_band = 0
    for b in range(B):
        flat = p[b] * V + t[b]
        assert len(set(flat.tolist())) == width, f"{name}: request {b} repeats a candidate"
        finite = torch.isfinite(s[b])
        assert bool((s[b][1:][finite[1:]] <= s[b][:-1][finite[1:]] + 1e-6).all()), \
            f"{name}: request {b} scores not in descending order"
        true = flat_keys[b].gather(0, flat)
        assert torch.equal(torch.isfinite(true), finite), f"{name}: validity differs"
        err = (s[b][finite] - true[finite]).abs()
        assert err.numel() == 0 or err.max().item() <= delta, \
            f"{name}: request {b} score error {err.max().item():.3e} > {delta}"
        kth = torch.topk(flat_keys[b], width).values[-1].item()
        if kth == -float("inf"):
            continue
        must = torch.nonzero(flat_keys[b] > kth + delta).squeeze(1)
        picked = set(flat.tolist())
        missing = [i for i in must.tolist() if i not in picked]
        assert not missing, f"{name}: request {b} misses {len(missing)} clear winners"
        low = true[finite] < kth - delta
        assert not bool(low.any()), f"{name}: request {b} picks {int(low.sum())} clear losers"
        in_band += int(((true - kth).abs() <= delta).sum())
    return in_band
