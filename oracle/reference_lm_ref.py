"""CPU restatement of the reference's toy hybrid model (oracle; tests only).

Follows src/kadllm/adapters/reference.py:56-110 (``ReferenceHybridLM._run``,
``prefill``, ``decode``) on a state dict in that module's naming, with the
operators of ``oracle.ops_ref`` in fp32: embedding; gated-delta mixer
(decay -softplus(a), beta sigmoid(b), zero initial state at prefill, the
final state kept as the prefix); causal attention whose shared prefix is the
prompt's K/V (empty at prefill); gated MLP added before the LM head.
Pinned by the reference's own outputs in tests/golden/reference_lm_fp32.npz.
"""

import torch
from torch.nn import functional as F

from . import ops_ref


class ReferenceLMOracle:
    """prefill(ids) -> (logits [B, V], prefix); decode(history, prefix) -> [B, W, V]."""

    def __init__(self, state_dict, num_heads):
        self.sd = {k: v.detach().to("cpu", torch.float32) for k, v in state_dict.items()}
        self.heads = num_heads

    def _linear(self, name, x):
        return F.linear(x, self.sd[name + ".weight"], self.sd.get(name + ".bias"))

    def _run(self, tokens, prefix=None, width=1):
        x = self.sd["embedding.weight"][tokens]
        rows, T, D = x.shape
        hd = D // self.heads

        def split(t):
            return [c.reshape(rows, T, self.heads, hd) for c in t.chunk(3, dim=-1)]

        q, k, v = split(self._linear("gdn_qkv", x))
        a, b = self._linear("gates", x).chunk(2, dim=-1)
        state = (torch.zeros(rows, self.heads, hd, hd) if prefix is None else prefix[0])
        res = ops_ref.gated_delta(q, k, v, -F.softplus(a), torch.sigmoid(b), state,
                                  beam_width=width, return_final_state=prefix is None)
        mixed, final = (res if prefix is None else (res, None))
        x = x + mixed.reshape(rows, T, D)
        q, k, v = split(self._linear("attention_qkv", x))
        pk, pv = (k[:, :0], v[:, :0]) if prefix is None else (prefix[1], prefix[2])
        x = x + ops_ref.prefix_attention(q, pk, pv, k, v, beam_width=width).reshape(rows, T, D)
        gate = self._linear("mlp.gate_proj", x)
        up = self._linear("mlp.up_proj", x)
        x = x + self._linear("mlp.down_proj", F.silu(gate) * up)
        logits = F.linear(x, self.sd["lm_head.weight"])
        return logits, ((final, k, v) if prefix is None else None)

    def prefill(self, input_ids):
        logits, prefix = self._run(input_ids)
        return logits[:, -1], prefix

    def decode(self, history, prefix):
        B, W, T = history.shape
        logits, _ = self._run(history.reshape(B * W, T), prefix, W)
        return logits[:, -1].reshape(B, W, -1)
