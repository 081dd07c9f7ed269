"""GRBeam: fixed-depth beam decoding with an immutable, request-sized prefix.

Drop-in for src/kadllm/grbeam.py: the same dataclasses, adapter protocol,
constraint type and ``grbeam_search`` signature, validation order and error
messages.  Selection runs on the GPU in the HIP kernels kad_beam_row_select /
kad_beam_merge_select / kad_beam_history (full-vocabulary log-softmax,
constraint mask, parent-score add and top-W without fp32 [W, V]
temporaries).  Ties are broken by the lower flat index (parent * V + token);
the reference's torch.topk leaves tie order unspecified (grbeam.py:95).
"""

import ctypes
import inspect
from collections.abc import Callable, Sequence
from dataclasses import dataclass
from typing import Any, Protocol

import torch

from . import _lib


@dataclass(frozen=True)
class PrefillResult:
    logits: torch.Tensor  # [B, vocabulary], predicts the first new token
    state: Any


class GRBeamAdapter(Protocol):
    def prefill(self, input_ids: torch.Tensor) -> PrefillResult:
        """Process [B, prompt_length] and save a request-sized prefix."""
        ...

    def decode(self, history: torch.Tensor, state: Any) -> torch.Tensor:
        """Replay [B, W, T] suffix tokens; return [B, W, vocabulary] logits.

        The prefix is read-only. No state from one beam may affect another.
        """
        ...


@dataclass(frozen=True)
class GRBeamResult:
    tokens: torch.Tensor  # [B, final_width, depth]
    scores: torch.Tensor  # unnormalized cumulative full-vocabulary log-prob
    valid: torch.Tensor  # False for unfilled slots under constraints


# Returns a bool mask shaped like logits; True allows a candidate; no renormalisation.
Constraint = Callable[[torch.Tensor, torch.Tensor], torch.Tensor]


# Widest level the merge kernel sorts in LDS (kad_beam_merge_select); wider
# levels take kad_beam_merge_select_wide, which sorts in workspace.
MAX_LDS_WIDTH = 16384


def select_level(logits, scores, width, mask=None):
    """One selection level on the GPU (src/kadllm/grbeam.py:89-104).

    logits [B, Wp, V] bf16, fp16 or fp32 (last dim contiguous; the key is
    computed in fp32 as the reference's .float().log_softmax), scores [B, Wp] fp32, mask
    [B, Wp, V] bool or None; a mask that is one [V] row broadcast to every beam
    row (an ``expand``-ed view, row stride 0) is read in place.  Returns
    (scores [B, width] fp32, parents, tokens [B, width] int64, valid [B, width]
    bool).
    """
    B, Wp, V = logits.shape
    if logits.dtype not in _lib.DTYPE_CODES:
        raise RuntimeError("HIP beam selection takes bf16, fp16 or fp32 logits")
    if not logits.is_cuda:
        raise RuntimeError("HIP beam selection needs logits on a ROCm device")
    if logits.stride(2) != 1 or logits.stride(0) != Wp * logits.stride(1):
        logits = logits.contiguous()
    dev = logits.device
    rows = B * Wp
    K = min(width, V)
    parent = scores.to(device=dev, dtype=torch.float32).contiguous()
    cand_key = torch.empty(rows, K, dtype=torch.float32, device=dev)
    cand_idx = torch.empty(rows, K, dtype=torch.int32, device=dev)
    m, ld_mask = None, V
    if mask is not None:
        if mask.shape != logits.shape or mask.dtype != torch.bool:
            raise ValueError("mask must be a bool tensor shaped like the logits")
        if mask.device != dev:
            raise ValueError("constraint mask must be on the logits' device")
        if mask.stride(2) == 1 and mask.stride(0) == Wp * mask.stride(1) and mask.is_cuda:
            m, ld_mask = mask.view(torch.uint8), mask.stride(1)
        else:
            m = mask.contiguous().view(torch.uint8)
    stream = _lib.stream_of(logits)
    _lib.call("kad_beam_row_select", _lib.ptr(logits), _lib.dtype_code(logits.dtype),
              logits.stride(1), _lib.ptr(m),
              ld_mask, _lib.ptr(parent), rows, Wp, V, K, _lib.ptr(cand_key), _lib.ptr(cand_idx),
              stream)
    new_scores = torch.empty(B, width, dtype=torch.float32, device=dev)
    parents = torch.empty(B, width, dtype=torch.int64, device=dev)
    tokens = torch.empty(B, width, dtype=torch.int64, device=dev)
    valid = torch.empty(B, width, dtype=torch.bool, device=dev)
    merge(cand_key, cand_idx, B, Wp * K, width, V, new_scores, parents, tokens, valid, stream)
    return new_scores, parents, tokens, valid


def merge(cand_key, cand_idx, B, ncand, width, V, scores, parents, tokens, valid, stream,
          wide=None):
    """The request-level stage of the selection: the LDS-sorting kernel up to
    MAX_LDS_WIDTH beams, the workspace-sorting one beyond (``wide`` forces
    either)."""
    if wide is None:
        wide = width > MAX_LDS_WIDTH
    if not wide:
        _lib.call("kad_beam_merge_select", _lib.ptr(cand_key), _lib.ptr(cand_idx), B, ncand,
                  width, V, _lib.ptr(scores), _lib.ptr(parents), _lib.ptr(tokens),
                  _lib.ptr(valid), stream)
        return
    nbytes = ctypes.c_int64()
    _lib.call("kad_beam_merge_select_wide_workspace_bytes", B, width, ctypes.byref(nbytes))
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=cand_key.device)
    _lib.call("kad_beam_merge_select_wide", _lib.ptr(cand_key), _lib.ptr(cand_idx), B, ncand,
              width, V, _lib.ptr(scores), _lib.ptr(parents), _lib.ptr(tokens), _lib.ptr(valid),
              _lib.ptr(ws), nbytes.value, stream)


def select_level_grouped(logits, scores, groups, width, mask=None):
    """Per-group selection: the Wp beam rows of each request form ``groups``
    contiguous groups of Wp / groups rows, and every group keeps its own
    ``width`` best candidates (ties to the lower (row, token) inside the group).
    Returns (scores, parents, tokens, valid), each [B, groups * width], beams
    ordered by group; parents index the request's Wp rows."""
    B, Wp, V = logits.shape
    if Wp % groups:
        raise ValueError("beam rows must split evenly into the groups")
    rpg = Wp // groups
    if logits.stride(2) != 1 or logits.stride(0) != Wp * logits.stride(1):
        logits = logits.contiguous()
    lg = logits.view(B * groups, rpg, V)
    sc = scores.reshape(B * groups, rpg)
    mk = None
    if mask is not None:
        if mask.shape != logits.shape or mask.dtype != torch.bool:
            raise ValueError("mask must be a bool tensor shaped like the logits")
        if mask.device != logits.device:
            raise ValueError("constraint mask must be on the logits' device")
        if mask.stride(2) == 1 and mask.stride(0) == Wp * mask.stride(1):
            mk = mask.as_strided((B * groups, rpg, V), (rpg * mask.stride(1), mask.stride(1), 1))
        else:
            mk = mask.contiguous().view(B * groups, rpg, V)
    s, p, t, v = select_level(lg, sc, width, mk)
    offset = torch.arange(groups, device=p.device, dtype=torch.int64)[:, None] * rpg
    parents = (p.view(B, groups, width) + offset).view(B, groups * width)
    return (s.view(B, groups * width), parents, t.view(B, groups * width),
            v.view(B, groups * width))


def extend_history(history, parents, tokens):
    """cat(history.gather(1, parents), tokens) on the GPU (src/kadllm/grbeam.py:102-104)."""
    B, Wp, step = history.shape
    W = parents.shape[1]
    out = torch.empty(B, W, step + 1, dtype=torch.int64, device=parents.device)
    h = history.to(torch.int64).contiguous() if step else None
    _lib.call("kad_beam_history", _lib.ptr(h), Wp, step, _lib.ptr(parents), _lib.ptr(tokens),
              _lib.ptr(out), B, W, _lib.stream_of(parents))
    return out


def _column_tokens(adapter, tokens):
    """Token ids of selected logits columns.  An adapter whose head projects to
    a sub-vocabulary (a SID-only head) names the token of each column in
    ``vocab_ids``; history and results then hold real token ids."""
    ids = getattr(adapter, "vocab_ids", None)
    if ids is None:
        return tokens
    return ids.index_select(0, tokens.reshape(-1)).view(tokens.shape)


def _incremental_decoder(adapter):
    """The adapter's decode_incremental as f(history, parents, state, cache,
    last), or None.  On a search's last level an adapter that takes
    ``keep_cache`` is told not to keep its suffix cache, which nothing would
    read (at B32 x W256 with 2-token suffixes it is ~5 GB of per-layer rows)."""
    fn = getattr(adapter, "decode_incremental", None)
    if fn is None:
        return None
    try:
        takes = "keep_cache" in inspect.signature(fn).parameters
    except (TypeError, ValueError):
        takes = False
    if takes:
        return lambda h, p, s, c, last: fn(h, p, s, c, keep_cache=not last)
    return lambda h, p, s, c, last: fn(h, p, s, c)


@torch.no_grad()
def grbeam_search(
    adapter: GRBeamAdapter,
    input_ids: torch.Tensor,
    widths: Sequence[int],
    *,
    allowed: Constraint | None = None,
) -> GRBeamResult:
    """Run GRBeam with a fixed token count and an explicit width per level.

    Call model.eval() first. EOS handling and length penalties are outside
    this fixed-depth API.  No CPU conversion of candidates is performed.
    Invalid constrained slots remain marked rather than invented.  With a
    SID-only head (``adapter.vocab_ids``), logits cover that sub-vocabulary and
    the softmax runs over it; selected columns become token ids.
    """
    if input_ids.ndim != 2 or min(input_ids.shape) < 1:
        raise ValueError("input_ids must be nonempty [B, prompt_length]")
    if not widths or any(
        not isinstance(w, int) or isinstance(w, bool) or w < 1 for w in widths
    ):
        raise ValueError("widths must contain positive integers")
    prefill = adapter.prefill(input_ids)
    B = input_ids.shape[0]
    if prefill.logits.ndim != 2 or prefill.logits.shape[0] != B:
        raise ValueError("prefill logits must have shape [B, vocabulary]")
    V = prefill.logits.shape[-1]
    if V < 1:
        raise ValueError("vocabulary must be nonempty")
    dev = prefill.logits.device
    history = torch.empty(B, 1, 0, dtype=torch.int64, device=dev)
    scores = torch.zeros(B, 1, device=dev)
    valid = None
    logits = prefill.logits[:, None, :]
    # An adapter that can extend the previous level's suffixes (keeping their
    # per-token state) gets the parents; its logits equal decode(history).
    incremental = _incremental_decoder(adapter)
    cache = parents = None
    for step, width in enumerate(widths):
        if step:
            if incremental is not None:
                logits, cache = incremental(history, parents, prefill.state, cache,
                                            step == len(widths) - 1)
            else:
                logits = adapter.decode(history, prefill.state)
        if logits.shape != (*history.shape[:2], V):
            raise ValueError("decode logits must be [B, current_width, vocabulary]")
        mask = None
        if allowed is not None:
            mask = allowed(history, logits)
            if mask.shape != logits.shape or mask.dtype != torch.bool:
                raise ValueError("constraint must return a bool mask matching logits")
            if mask.device != logits.device:
                raise ValueError("constraint mask must be on the logits' device")
        if width > history.shape[1] * V:
            raise ValueError("beam width exceeds the number of candidate slots")
        scores, parents, tokens, valid = select_level(logits, scores, width, mask)
        del logits, mask
        history = extend_history(history, parents, _column_tokens(adapter, tokens))
    return GRBeamResult(history, scores, valid)


@torch.no_grad()
def conditional_search(
    adapter: GRBeamAdapter,
    input_ids: torch.Tensor,
    coarse_widths: Sequence[int],
    fine_widths: Sequence[int],
    *,
    allowed: Constraint | None = None,
) -> GRBeamResult:
    """Two-level conditional search (semantic-ID generation with coarse and fine
    code levels): ``coarse_widths`` levels of ordinary GRBeam selection over the
    full vocabulary, then ``fine_widths`` levels in which every coarse beam
    keeps its own ``fine_widths[i]`` best descendants, so the level holds
    coarse_width * fine_widths[i] beams ordered by coarse beam.  Scores are
    cumulative full-vocabulary log-probabilities throughout; ``allowed`` masks
    candidates without renormalisation (src/kadllm/grbeam.py:41-42,80-84) and
    may return a [V] row broadcast to the logits' shape.  Each coarse beam's
    suffix is the shared prefix for its children: decoding reuses the request
    prefix state for every beam and extends cached suffixes by one token.
    Returns GRBeamResult(tokens [B, Wc * fine_widths[-1], depth], scores, valid).
    """
    for ws in (coarse_widths, fine_widths):
        if not ws or any(not isinstance(w, int) or isinstance(w, bool) or w < 1 for w in ws):
            raise ValueError("widths must contain positive integers")
    if input_ids.ndim != 2 or min(input_ids.shape) < 1:
        raise ValueError("input_ids must be nonempty [B, prompt_length]")
    prefill = adapter.prefill(input_ids)
    B = input_ids.shape[0]
    V = prefill.logits.shape[-1]
    dev = prefill.logits.device
    history = torch.empty(B, 1, 0, dtype=torch.int64, device=dev)
    scores = torch.zeros(B, 1, device=dev)
    logits = prefill.logits[:, None, :]
    incremental = _incremental_decoder(adapter)
    cache = parents = valid = None
    levels = [(w, None) for w in coarse_widths] + [(w, "fine") for w in fine_widths]
    groups = None
    for step, (width, kind) in enumerate(levels):
        if step:
            if incremental is not None:
                logits, cache = incremental(history, parents, prefill.state, cache,
                                            step == len(levels) - 1)
            else:
                logits = adapter.decode(history, prefill.state)
        if logits.shape != (*history.shape[:2], V):
            raise ValueError("decode logits must be [B, current_width, vocabulary]")
        mask = None
        if allowed is not None:
            mask = allowed(history, logits)
            if mask.dtype != torch.bool:
                raise ValueError("constraint must return a bool mask")
            if mask.device != logits.device:
                raise ValueError("constraint mask must be on the logits' device")
            mask = mask.expand(logits.shape)
        if kind is None:
            if width > history.shape[1] * V:
                raise ValueError("beam width exceeds the number of candidate slots")
            scores, parents, tokens, valid = select_level(logits, scores, width, mask)
        else:
            if groups is None:
                groups = history.shape[1]  # the coarse beams
            if width > (history.shape[1] // groups) * V:
                raise ValueError("fine width exceeds a coarse beam's candidate slots")
            scores, parents, tokens, valid = select_level_grouped(logits, scores, groups, width,
                                                                  mask)
        del logits, mask
        history = extend_history(history, parents, _column_tokens(adapter, tokens))
    return GRBeamResult(history, scores, valid)
