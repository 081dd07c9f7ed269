"""GRBeam: fixed-depth beam decoding with an immutable, request-sized prefix.

Drop-in for src/kadllm/grbeam.py: the same dataclasses, adapter protocol,
constraint type and ``grbeam_search`` signature, validation order and error
messages.  Selection runs on the GPU in the HIP kernels kad_beam_row_select /
kad_beam_merge_select / kad_beam_history (full-vocabulary log-softmax,
constraint mask, parent-score add and top-W without fp32 [W, V]
temporaries).  Ties are broken by the lower flat index (parent * V + token);
the reference's torch.topk leaves tie order unspecified (grbeam.py:95).
"""

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


def select_level(logits, scores, width, mask=None):
    """One selection level on the GPU (src/kadllm/grbeam.py:89-104).

    logits [B, Wp, V] bf16 (last dim contiguous), scores [B, Wp] fp32, mask
    [B, Wp, V] bool or None.  Returns (scores [B, width] fp32, parents,
    tokens [B, width] int64, valid [B, width] bool).
    """
    B, Wp, V = logits.shape
    if logits.dtype != torch.bfloat16:
        raise RuntimeError("HIP beam selection takes bf16 logits")
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
    m = None
    if mask is not None:
        m = mask.contiguous().view(torch.uint8)
    stream = _lib.stream_of(logits)
    _lib.call("kad_beam_row_select", _lib.ptr(logits), logits.stride(1), _lib.ptr(m),
              V, _lib.ptr(parent), rows, Wp, V, K, _lib.ptr(cand_key), _lib.ptr(cand_idx), stream)
    new_scores = torch.empty(B, width, dtype=torch.float32, device=dev)
    parents = torch.empty(B, width, dtype=torch.int64, device=dev)
    tokens = torch.empty(B, width, dtype=torch.int64, device=dev)
    valid = torch.empty(B, width, dtype=torch.bool, device=dev)
    _lib.call("kad_beam_merge_select", _lib.ptr(cand_key), _lib.ptr(cand_idx), B, Wp * K, width,
              V, _lib.ptr(new_scores), _lib.ptr(parents), _lib.ptr(tokens), _lib.ptr(valid), stream)
    return new_scores, parents, tokens, valid


def extend_history(history, parents, tokens):
    """cat(history.gather(1, parents), tokens) on the GPU (src/kadllm/grbeam.py:102-104)."""
    B, Wp, step = history.shape
    W = parents.shape[1]
    out = torch.empty(B, W, step + 1, dtype=torch.int64, device=parents.device)
    h = history.to(torch.int64).contiguous() if step else None
    _lib.call("kad_beam_history", _lib.ptr(h), Wp, step, _lib.ptr(parents), _lib.ptr(tokens),
              _lib.ptr(out), B, W, _lib.stream_of(parents))
    return out


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
    Invalid constrained slots remain marked rather than invented.
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
    incremental = getattr(adapter, "decode_incremental", None)
    cache = parents = None
    for step, width in enumerate(widths):
        if step:
            if incremental is not None:
                logits, cache = incremental(history, parents, prefill.state, cache)
            else:
                logits = adapter.decode(history, prefill.state)
        if logits.shape != (*history.shape[:2], V):
            raise ValueError("decode logits must be [B, current_width, vocabulary]")
        mask = None
        if allowed is not None:
            mask = allowed(history, logits)
            if mask.shape != logits.shape or mask.dtype != torch.bool:
                raise ValueError("constraint must return a bool mask matching logits")
        if width > history.shape[1] * V:
            raise ValueError("beam width exceeds the number of candidate slots")
        scores, parents, tokens, valid = select_level(logits, scores, width, mask)
        del logits, mask
        history = extend_history(history, parents, tokens)
    return GRBeamResult(history, scores, valid)
