"""CPU restatement of the Qwen3.5 hybrid text model on the GRBeam path (oracle).

Prefill follows the native model forward the reference prefill calls
(src/kadllm/adapters/qwen3_5.py:106-133 -> transformers qwen3_5
Qwen3_5TextModel.forward, modeling_qwen3_5.py:1147-1214): embedding, per
layer pre-norm residual blocks (Gated DeltaNet :432-543 or gated attention
:656-701) with a SwiGLU MLP (:704-717), final RMSNorm; logits of the last
prompt token.  The prefix snapshot matches qwen3_5.py:113-129: per GDN layer
(conv state = last kernel-size pre-conv inputs [B,C,4], recurrent state
fp32 [B,HV,K,V]); per attention layer (K post-norm post-RoPE, V), exposed as
[B,L,HK,D] views of [B,HK,L,D] storage.  The prompt's attention is the
causal SDPA call the transformers forward makes with
attn_implementation="sdpa" (the reference's runner, benchmarks/grbeam.py:213).
Pinned bit for bit in bf16 and to 1e-5 in fp32 against the reference's own
search outputs (tests/golden/grbeam_tiny_*.npz).

Decode follows Qwen35GRBeamAdapter.decode/_linear/_attention
(src/kadllm/adapters/qwen3_5.py:144-235) with the oracle operators of
``ops_ref``.

Weights are a dict in the transformers Qwen3_5TextModel state-dict naming
(``embed_tokens.weight``, ``layers.{i}.linear_attn.in_proj_qkv.weight``, ...)
plus ``lm_head.weight`` (absent = tied to the embedding).  ``cfg`` is any
object with the Qwen3_5TextConfig attribute names used below.
"""

from dataclasses import dataclass

import torch
from torch.nn import functional as F

from . import ops_ref


def rms_norm(x, w, eps):
    """Qwen3_5RMSNorm (modeling_qwen3_5.py:720-734): fp32 norm, (1+w), one rounding."""
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (y * (1.0 + w.float())).type_as(x)


def rms_norm_gated(x, z, w, eps):
    """Qwen3_5RMSNormGated (modeling_qwen3_5.py:168-184): w*norm(x) rounded, then *silu(z)."""
    dt = x.dtype
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    y = w * y.to(dt)
    y = y * F.silu(z.float())
    return y.to(dt)


def rope_inv_freq(cfg):
    """Default RoPE inverse frequencies over the rotary part of a head.

    modeling_qwen3_5.py:104-120: dim = head_dim * partial_rotary_factor.
    """
    dim = int(cfg.head_dim * cfg.partial_rotary_factor)
    return 1.0 / (cfg.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.float) / dim))


def rope_cos_sin(cfg, positions, dtype):
    """cos/sin tables [N, P, rot] for integer positions [N, P] (text-only MRoPE == RoPE).

    modeling_qwen3_5.py:122-147: fp32 freqs = pos * inv_freq, duplicated,
    cos/sin cast to the activation dtype.
    """
    inv = rope_inv_freq(cfg)
    freqs = positions.float()[..., None] * inv
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def apply_rope(x, cos, sin):
    """Rotate-half RoPE on the first rot dims (modeling_qwen3_5.py:554-589).

    x [..., P, D] with cos/sin broadcastable [..., P, rot]; bf16 ops round per op.
    """
    rot = cos.shape[-1]
    xr, xp = x[..., :rot], x[..., rot:]
    half = rot // 2
    rotated = torch.cat((-xr[..., half:], xr[..., :half]), dim=-1)
    return torch.cat(((xr * cos) + (rotated * sin), xp), dim=-1)


@dataclass(frozen=True)
class OraclePrefix:
    length: int
    batch: int
    layers: tuple


class Qwen35Oracle:
    """Hybrid GDN / gated-attention model on CPU tensors (weights in model dtype)."""

    def __init__(self, cfg, weights):
        self.cfg = cfg
        self.w = weights
        self.dtype = weights["embed_tokens.weight"].dtype

    # -- helpers -----------------------------------------------------------
    def _p(self, name):
        return self.w[name]

    def lm_head_weight(self):
        return self.w.get("lm_head.weight", self.w["embed_tokens.weight"])

    def _mlp(self, i, x):
        p = f"layers.{i}.mlp."
        g = F.linear(x, self._p(p + "gate_proj.weight"))
        u = F.linear(x, self._p(p + "up_proj.weight"))
        return F.linear(F.silu(g) * u, self._p(p + "down_proj.weight"))

    def _gdn_projections(self, i, n):
        cfg = self.cfg
        p = f"layers.{i}.linear_attn."
        qkv = F.linear(n, self._p(p + "in_proj_qkv.weight"))
        z = F.linear(n, self._p(p + "in_proj_z.weight"))
        b = F.linear(n, self._p(p + "in_proj_b.weight"))
        a = F.linear(n, self._p(p + "in_proj_a.weight"))
        beta = b.sigmoid()
        g = -self._p(p + "A_log").float().exp() * F.softplus(a.float() + self._p(p + "dt_bias"))
        return qkv, z, beta, g

    def _gdn_finish(self, i, o, z, rows, length):
        cfg = self.cfg
        p = f"layers.{i}.linear_attn."
        dv = cfg.linear_value_head_dim
        y = rms_norm_gated(o.reshape(-1, dv), z.reshape(-1, dv), self._p(p + "norm.weight"),
                           cfg.rms_norm_eps)
        y = y.reshape(rows, length, cfg.linear_num_value_heads * dv)
        return F.linear(y, self._p(p + "out_proj.weight"))

    def _split_qkv(self, mixed, rows, length):
        cfg = self.cfg
        kd = cfg.linear_num_key_heads * cfg.linear_key_head_dim
        q, k, v = mixed.split((kd, kd, cfg.linear_num_value_heads * cfg.linear_value_head_dim), -1)
        q = q.reshape(rows, length, cfg.linear_num_key_heads, cfg.linear_key_head_dim)
        k = k.reshape_as(q)
        v = v.reshape(rows, length, cfg.linear_num_value_heads, cfg.linear_value_head_dim)
        return q, k, v

    def _attn_projections(self, i, n, cos, sin):
        cfg = self.cfg
        p = f"layers.{i}.self_attn."
        rows, length = n.shape[:2]
        hd = cfg.head_dim
        qg = F.linear(n, self._p(p + "q_proj.weight")).reshape(rows, length, -1, 2 * hd)
        q, gate = qg.chunk(2, dim=-1)
        q = rms_norm(q, self._p(p + "q_norm.weight"), cfg.rms_norm_eps).transpose(1, 2)
        k = F.linear(n, self._p(p + "k_proj.weight")).reshape(rows, length, -1, hd)
        k = rms_norm(k, self._p(p + "k_norm.weight"), cfg.rms_norm_eps).transpose(1, 2)
        v = F.linear(n, self._p(p + "v_proj.weight")).reshape(rows, length, -1, hd)
        q = apply_rope(q, cos[:, None], sin[:, None])
        k = apply_rope(k, cos[:, None], sin[:, None])
        return q, k, v, gate.reshape(rows, length, -1)

    # -- full forward / prefill --------------------------------------------
    def forward_layer(self, i, x, cos, sin):
        """Layer i of the full causal forward on x [B,L,H]: (x after the layer,
        its prefix snapshot (conv state, S) or (K, V))."""
        cfg = self.cfg
        B, L = x.shape[:2]
        kind = cfg.layer_types[i]
        n = rms_norm(x, self._p(f"layers.{i}.input_layernorm.weight"), cfg.rms_norm_eps)
        if kind == "linear_attention":
            qkv, z, beta, g = self._gdn_projections(i, n)
            pre = qkv.transpose(1, 2)                                   # [B,C,L]
            ks = cfg.linear_conv_kernel_dim
            padded = F.pad(pre, (max(0, ks - L), 0)) if L < ks else pre
            conv_state = padded[..., -ks:].clone()
            wconv = self._p(f"layers.{i}.linear_attn.conv1d.weight")    # [C,1,ks]
            y = F.conv1d(pre.to(wconv.dtype), wconv, None, padding=ks - 1,
                         groups=pre.shape[1])[..., :L]
            y = F.silu(y).to(pre.dtype).transpose(1, 2)
            q, k, v = self._split_qkv(y, B, L)
            rep = cfg.linear_num_value_heads // cfg.linear_num_key_heads
            if rep > 1:
                q = q.repeat_interleave(rep, dim=2)
                k = k.repeat_interleave(rep, dim=2)
            o, S = ops_ref.chunk_gated_delta(q, k, v, g, beta)
            mixed = self._gdn_finish(i, o, z, B, L)
            snap = (conv_state, S)
        else:
            q, k, v, gate = self._attn_projections(i, n, cos, sin)
            vt = v.transpose(1, 2)                                      # [B,HK,L,D]
            rep = cfg.num_attention_heads // cfg.num_key_value_heads
            # the causal SDPA call of the transformers forward the reference
            # runs (attn_implementation="sdpa", benchmarks/grbeam.py:213;
            # HF-q35 682-695), in the model dtype: its internal rounding is
            # part of the reference's bf16 prefill
            a = F.scaled_dot_product_attention(q, k.repeat_interleave(rep, dim=1),
                                               vt.repeat_interleave(rep, dim=1), is_causal=True,
                                               scale=cfg.head_dim ** -0.5)   # [B,H,L,D]
            a = a.transpose(1, 2).reshape(B, L, -1) * gate.sigmoid()
            mixed = F.linear(a, self._p(f"layers.{i}.self_attn.o_proj.weight"))
            snap = (k.transpose(1, 2), vt.transpose(1, 2))             # [B,L,HK,D] views
        x = x + mixed
        n2 = rms_norm(x, self._p(f"layers.{i}.post_attention_layernorm.weight"),
                      cfg.rms_norm_eps)
        return x + self._mlp(i, n2), snap

    def prompt_rope(self, B, L, dtype):
        pos = torch.arange(L)[None].expand(B, L)
        return rope_cos_sin(self.cfg, pos, dtype)

    def forward(self, input_ids):
        """Full causal forward.  Returns (final-normed hidden [B,L,H], snapshot)."""
        cfg = self.cfg
        B, L = input_ids.shape
        x = F.embedding(input_ids, self._p("embed_tokens.weight"))
        cos, sin = self.prompt_rope(B, L, x.dtype)
        snap = []
        for i in range(len(cfg.layer_types)):
            x, s = self.forward_layer(i, x, cos, sin)
            snap.append(s)
        x = rms_norm(x, self._p("norm.weight"), cfg.rms_norm_eps)
        return x, tuple(snap)

    def full_logits(self, input_ids):
        """Logits at every position of a full forward [B,L,V]."""
        h, _ = self.forward(input_ids)
        return F.linear(h, self.lm_head_weight())

    def prefill(self, input_ids):
        """Reference prefill (qwen3_5.py:106-133): logits [B,V] and the request-sized prefix."""
        h, snap = self.forward(input_ids)
        logits = F.linear(h[:, -1], self.lm_head_weight())
        return logits, OraclePrefix(input_ids.shape[1], input_ids.shape[0], snap)

    # -- suffix replay ------------------------------------------------------
    def suffix_rope(self, rows, length, T, dtype):
        pos = torch.arange(length, length + T)[None].expand(rows, T)
        return rope_cos_sin(self.cfg, pos, dtype)

    def decode_layer(self, i, x, cached, W, cos, sin):
        """Layer i of the suffix replay on x [B*W,T,H] against the prefix entry
        ``cached`` of that layer; returns x after the layer."""
        cfg = self.cfg
        rows, T = x.shape[:2]
        kind = cfg.layer_types[i]
        n = rms_norm(x, self._p(f"layers.{i}.input_layernorm.weight"), cfg.rms_norm_eps)
        if kind == "linear_attention":
            qkv, z, beta, g = self._gdn_projections(i, n)
            wconv = self._p(f"layers.{i}.linear_attn.conv1d.weight").squeeze(1)
            mixed = ops_ref.causal_conv1d(qkv.transpose(1, 2), cached[0], wconv,
                                          beam_width=W).transpose(1, 2)
            q, k, v = self._split_qkv(mixed, rows, T)
            o = ops_ref.gated_delta(q, k, v, g, beta, cached[1], beam_width=W)
            mixed = self._gdn_finish(i, o, z, rows, T)
        else:
            q, k, v, gate = self._attn_projections(i, n, cos, sin)
            o = ops_ref.prefix_attention(q.transpose(1, 2), cached[0], cached[1],
                                         k.transpose(1, 2), v, beam_width=W,
                                         scale=cfg.head_dim ** -0.5)
            o = o.reshape(rows, T, -1) * gate.sigmoid()
            mixed = F.linear(o, self._p(f"layers.{i}.self_attn.o_proj.weight"))
        x = x + mixed
        n2 = rms_norm(x, self._p(f"layers.{i}.post_attention_layernorm.weight"),
                      cfg.rms_norm_eps)
        return x + self._mlp(i, n2)

    def head(self, h):
        """Final RMSNorm and LM head of hidden rows [..., H]."""
        h = rms_norm(h, self._p("norm.weight"), self.cfg.rms_norm_eps)
        return F.linear(h, self.lm_head_weight())

    def decode(self, history, state):
        """Reference decode (qwen3_5.py:204-235): replay [B,W,T] suffixes -> [B,W,V]."""
        B, W, T = history.shape
        rows = B * W
        x = F.embedding(history.reshape(rows, T), self._p("embed_tokens.weight"))
        cos, sin = self.suffix_rope(rows, state.length, T, x.dtype)
        for i, cached in enumerate(state.layers):
            x = self.decode_layer(i, x, cached, W, cos, sin)
        return self.head(x[:, -1]).reshape(B, W, -1)
