"""Host-side argument checks that run before any kernel launch (CPU only)."""

import pytest
import torch

from kadllm_amd import conditional_search, grbeam_search
from kadllm_amd.grbeam import MAX_LDS_WIDTH, PrefillResult
from kadllm_amd.qwen35 import reject_biases


class _MetaAdapter:
    """Returns logits on the meta device (no data, no kernels) and counts calls."""

    def __init__(self, V=16):
        self.V = V
        self.prefills = 0

    def prefill(self, ids):
        self.prefills += 1
        return PrefillResult(torch.empty(ids.shape[0], self.V, device="meta"), None)

    def decode(self, history, state):
        raise AssertionError("decode must not be reached")


def test_width_beyond_candidate_slots_raises_before_selection():
    """Widths have no cap of their own (the reference's topk has none); a level
    wider than its candidate slots raises the reference's ValueError
    (src/kadllm/grbeam.py:85-86) before any selection kernel."""
    a = _MetaAdapter(V=16)
    ids = torch.zeros(1, 3, dtype=torch.int64)
    with pytest.raises(ValueError, match="exceeds the number of candidate slots"):
        grbeam_search(a, ids, [MAX_LDS_WIDTH + 1])
    with pytest.raises(ValueError, match="exceeds the number of candidate slots"):
        conditional_search(a, ids, [17], [2])
    assert a.prefills == 2


def test_constraint_mask_on_another_device_raises():
    """A mask on another device than the logits would hand the kernel a
    foreign pointer; it is refused before selection."""
    a = _MetaAdapter()
    ids = torch.zeros(2, 3, dtype=torch.int64)

    def allowed(history, logits):
        return torch.ones(logits.shape, dtype=torch.bool)  # CPU, logits are on meta

    with pytest.raises(ValueError, match="logits' device"):
        grbeam_search(a, ids, [2], allowed=allowed)
    with pytest.raises(ValueError, match="logits' device"):
        conditional_search(a, ids, [2], [2], allowed=allowed)


def test_checkpoint_biases_are_refused():
    sd = {"layers.0.self_attn.q_proj.weight": torch.zeros(1),
          "layers.0.self_attn.q_proj.bias": torch.zeros(1)}
    with pytest.raises(ValueError, match="no projection biases"):
        reject_biases(object(), sd)
    sd = {"layers.0.linear_attn.conv1d.bias": torch.zeros(1)}
    with pytest.raises(ValueError, match="no projection biases"):
        reject_biases(object(), sd)

    class Cfg:
        attention_bias = True

    with pytest.raises(ValueError, match="attention_bias"):
        reject_biases(Cfg(), {})
    reject_biases(object(), {"layers.0.input_layernorm.weight": torch.zeros(1)})


def test_last_level_cache_hint_only_for_adapters_that_take_it():
    """grbeam passes keep_cache=False on a search's last level, and only to a
    decode_incremental that declares the keyword."""
    from kadllm_amd.grbeam import _incremental_decoder

    calls = []

    class WithHint:
        def decode_incremental(self, history, parents, state, cache=None, *, keep_cache=True):
            calls.append(keep_cache)
            return "logits", None

    class WithoutHint:
        def decode_incremental(self, history, parents, state, cache=None):
            calls.append("plain")
            return "logits", cache

    f = _incremental_decoder(WithHint())
    f(None, None, None, None, False)
    f(None, None, None, None, True)
    g = _incremental_decoder(WithoutHint())
    g(None, None, None, None, True)
    assert calls == [True, False, "plain"]
    assert _incremental_decoder(object()) is None
