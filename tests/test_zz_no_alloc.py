"""kad_beam_select_noalloc (candidates in the library's own device array, no
allocation) against kad_beam_row_select + kad_beam_merge_select with caller
workspace: the same results bit for bit, on two calls in a row, the second
smaller than the first."""

import pytest
import torch

from kadllm_amd import _lib
from kadllm_amd.grbeam import select_level

pytestmark = pytest.mark.gpu


def _noalloc(logits, scores, width, mask=None):
    B, Wp, V = logits.shape
    dev = logits.device
    out_s = torch.empty(B, width, dtype=torch.float32, device=dev)
    out_p = torch.empty(B, width, dtype=torch.int64, device=dev)
    out_t = torch.empty(B, width, dtype=torch.int64, device=dev)
    out_v = torch.empty(B, width, dtype=torch.bool, device=dev)
    m = None if mask is None else mask.contiguous().view(torch.uint8)
    _lib.call("kad_beam_select_noalloc", _lib.ptr(logits), _lib.dtype_code(logits.dtype),
              logits.stride(1), _lib.ptr(m), V, _lib.ptr(scores), B, Wp, V, width,
              _lib.ptr(out_s), _lib.ptr(out_p), _lib.ptr(out_t), _lib.ptr(out_v),
              _lib.stream_of(logits))
    return out_s, out_p, out_t, out_v


def _case(device, B, Wp, V, width, dtype, masked, seed):
    g = torch.Generator().manual_seed(seed)
    logits = (torch.randn(B, Wp, V, generator=g) * 2).to(dtype).to(device)
    scores = (-torch.rand(B, Wp, generator=g) * 3).to(device)
    mask = (torch.rand(B, Wp, V, generator=g) > 0.3).to(device) if masked else None
    return logits, scores, mask


def test_noalloc_selection_matches_two_stage(device):
    cases = [dict(B=4, Wp=256, V=4096, width=256, dtype=torch.bfloat16, masked=False, seed=1),
             dict(B=2, Wp=16, V=1000, width=64, dtype=torch.float32, masked=True, seed=2)]
    for c in cases:
        logits, scores, mask = _case(device, c["B"], c["Wp"], c["V"], c["width"], c["dtype"],
                                     c["masked"], c["seed"])
        got = _noalloc(logits, scores, c["width"], mask)
        want = select_level(logits, scores, c["width"], mask)
        torch.cuda.synchronize()
        for a, b, name in zip(got, want, ("scores", "parents", "tokens", "valid")):
            assert torch.equal(a.cpu(), b.cpu()), f"{name} differ for {c}"


def test_noalloc_selection_full_vocabulary_level(device):
    """One decode level of 2 requests x 256 beams over 248,320 tokens."""
    logits, scores, _ = _case(device, 2, 256, 248320, 256, torch.bfloat16, False, 3)
    got = _noalloc(logits, scores, 256)
    want = select_level(logits, scores, 256)
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert torch.equal(a.cpu(), b.cpu())


def test_noalloc_selection_rejects_oversized_levels(device):
    logits = torch.zeros(64, 256, 512, dtype=torch.bfloat16, device=device)
    scores = torch.zeros(64, 256, device=device)
    with pytest.raises(_lib.KadLibraryError, match="at most 4194304 candidates"):
        _noalloc(logits, scores, 512)
