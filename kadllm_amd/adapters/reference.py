"""The reference's tiny hybrid example model, on the HIP operators.

Drop-in for ``ReferenceHybridLM`` (src/kadllm/adapters/reference.py:38-110):
the same constructor, submodule names (so state dicts load either way),
prefix type and prefill/decode contract, and the same layer math -- one
gated-delta mixer, one causal attention mixer with a shared prefix, a gated
MLP and an LM head.  The two GRBeam operators run the HIP kernels
(``kadllm_amd.ops.gated_delta`` / ``prefix_attention``); the toy model's own
linear layers, embedding and activations stay torch modules, as in the
reference.  Unlike the reference, the operators are inference-only and need
the model on a ROCm device (``ReferenceHybridLM(...).cuda().eval()``).
"""

from dataclasses import dataclass

import torch
from torch import nn
from torch.nn import functional as F

from ..grbeam import PrefillResult
from ..ops import gated_delta, prefix_attention


class GatedMLP(nn.Module):
    """down(silu(gate(x)) * up(x)) with biased projections."""

    def __init__(self, hidden_size, intermediate_size):
        super().__init__()
        self.intermediate_size = intermediate_size
        self.gate_proj = nn.Linear(hidden_size, intermediate_size)
        self.up_proj = nn.Linear(hidden_size, intermediate_size)
        self.down_proj = nn.Linear(intermediate_size, hidden_size)
        self.act_fn = F.silu

    def forward(self, x):
        return self.down_proj(self.act_fn(self.gate_proj(x)) * self.up_proj(x))


@dataclass(frozen=True)
class HybridPrefix:
    recurrent: torch.Tensor  # [B, heads, head_dim, head_dim] final GDN state
    keys: torch.Tensor       # [B, L, heads, head_dim]
    values: torch.Tensor


class ReferenceHybridLM(nn.Module):
    """A random GDN + attention + MLP model implementing the GRBeam adapter
    protocol.  Prompts are unpadded; heads = num_heads of hidden/num_heads."""

    def __init__(self, vocab_size=32, hidden_size=16, num_heads=2):
        super().__init__()
        if min(vocab_size, hidden_size, num_heads) < 1 or hidden_size % num_heads:
            raise ValueError(
                "positive dimensions and hidden_size divisible by num_heads required"
            )
        self.num_heads = num_heads
        self.head_dim = hidden_size // num_heads
        self.embedding = nn.Embedding(vocab_size, hidden_size)
        self.gdn_qkv = nn.Linear(hidden_size, 3 * hidden_size)
        self.gates = nn.Linear(hidden_size, 2 * num_heads)
        self.attention_qkv = nn.Linear(hidden_size, 3 * hidden_size)
        self.mlp = GatedMLP(hidden_size, hidden_size * 2)
        self.lm_head = nn.Linear(hidden_size, vocab_size, bias=False)

    def _heads(self, x):
        rows, T, _ = x.shape
        return x.reshape(rows, T, self.num_heads, self.head_dim)

    def _run(self, tokens, prefix=None, width=1):
        """Logits [rows, T, V] of token rows; prefill (prefix None) also
        returns the request prefix: the GDN final state and the prompt's K/V."""
        x = self.embedding(tokens)
        rows = x.shape[0]
        q, k, v = map(self._heads, self.gdn_qkv(x).chunk(3, dim=-1))
        decay_in, beta_in = self.gates(x).chunk(2, dim=-1)
        if prefix is None:
            state = x.new_zeros(rows, self.num_heads, self.head_dim, self.head_dim)
        else:
            state = prefix.recurrent
        mixed = gated_delta(q, k, v, -F.softplus(decay_in), beta_in.sigmoid(), state,
                            beam_width=width, backend="torch",
                            return_final_state=prefix is None)
        final = None
        if prefix is None:
            mixed, final = mixed
        x = x + mixed.reshape(x.shape)
        q, k, v = map(self._heads, self.attention_qkv(x).chunk(3, dim=-1))
        if prefix is None:   # the prompt is all suffix: an empty shared prefix
            pk, pv = k[:, :0], v[:, :0]
        else:
            pk, pv = prefix.keys, prefix.values
        x = x + prefix_attention(q, pk, pv, k, v, beam_width=width).reshape(x.shape)
        logits = self.lm_head(x + self.mlp(x))
        return logits, (HybridPrefix(final, k, v) if prefix is None else None)

    def forward(self, input_ids):
        return self._run(input_ids)[0]

    def prefill(self, input_ids):
        if self.training:
            raise RuntimeError("call eval() before beam decoding")
        logits, state = self._run(input_ids)
        return PrefillResult(logits[:, -1], state)

    def decode(self, history, state):
        if self.training:
            raise RuntimeError("call eval() before beam decoding")
        B, W, T = history.shape
        if B != state.recurrent.shape[0] or T < 1:
            raise ValueError(
                "history must match the prefix batch and have a nonempty suffix"
            )
        logits, _ = self._run(history.reshape(B * W, T), state, W)
        return logits[:, -1].reshape(B, W, -1)
