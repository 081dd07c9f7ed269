"""Native Qwen3.5 hybrid text model on the HIP kernels: prefill and suffix replay.

The layer math is the one the reference path runs: prefill = the transformers
Qwen3_5TextModel forward (src/kadllm/adapters/qwen3_5.py:106-133),
decode = Qwen35GRBeamAdapter.decode/_linear/_attention (qwen3_5.py:144-235).
Each step maps onto a few fused kernels:

  GDN layer   rmsnorm -> GEMM [qkv | z | a | b] -> conv4 (prefill: whole
              prompt; decode: prefix taps + suffix) -> gates -> chunked GDN
              (prefill) / factored suffix replay (decode) -> gated rmsnorm ->
              GEMM out_proj + residual
  attention   rmsnorm -> GEMM [q+gate | k | v] -> q/k norm + partial RoPE ->
              causal attention (prefill) / prefix-shared attention (decode),
              sigmoid gate fused -> GEMM o_proj + residual
  MLP         rmsnorm -> GEMM [gate | up] with SwiGLU epilogue -> GEMM down + residual
  head        final rmsnorm on the last token of each row -> GEMM lm_head

Weights are packed once per model into bf16 device buffers; activations are
bf16 with the reference's rounding points.  Nothing here falls back to a
non-HIP implementation: every numeric step is a libkadllm_hip entry point.
"""

import ctypes
from dataclasses import dataclass

import torch

from . import _lib, layers
from .attention import attention_prefill, prefix_attention_decode
from .ops import REPLAY_MAX_T

_BLOCK = 32  # gate/up interleave granularity of the SwiGLU epilogue


def _round_up(x, m):
    return (x + m - 1) // m * m


def reject_biases(cfg, state_dict):
    """The packed projections carry no bias.  Qwen3.5 has none
    (attention_bias=False, bias-free GDN projections and conv); a checkpoint
    that holds one would be applied by the reference adapter's modules
    (src/kadllm/adapters/qwen3_5.py:146,181-188,202 and the conv1d.bias it
    passes to causal_conv1d), so it is refused here rather than dropped."""
    if getattr(cfg, "attention_bias", False):
        raise ValueError("attention_bias=True checkpoints are not supported by the HIP runner")
    biased = sorted(k for k in state_dict
                    if k.endswith(".bias") and (".self_attn." in k or ".linear_attn." in k
                                                or ".mlp." in k))
    if biased:
        raise ValueError(f"the HIP runner has no projection biases; checkpoint holds {biased[:3]}")


@dataclass
class _GdnLayer:
    input_norm: torch.Tensor
    post_norm: torch.Tensor
    w_in: torch.Tensor        # [qkv | z, H]
    w_ab: torch.Tensor        # [a | b, H]
    conv_w: torch.Tensor      # [C, 4]
    A_log: torch.Tensor
    dt_bias: torch.Tensor
    norm_w: torch.Tensor      # [dv]
    w_out: torch.Tensor       # [H, Vd]
    w_gu: torch.Tensor        # [2F, H] interleaved
    w_down: torch.Tensor      # [H, F]


@dataclass
class _AttnLayer:
    input_norm: torch.Tensor
    post_norm: torch.Tensor
    w_qkv: torch.Tensor       # [(2 nh hd) | nkv hd | nkv hd, H]
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    w_o: torch.Tensor         # [H, nh hd]
    w_gu: torch.Tensor
    w_down: torch.Tensor


def interleave_gate_up(gate, up):
    """[F, H] gate and up -> [2F, H] in [gate 32 | up 32] row blocks."""
    F_, H = gate.shape
    if F_ % _BLOCK:
        raise ValueError(f"intermediate size must be a multiple of {_BLOCK}")
    g = gate.reshape(F_ // _BLOCK, _BLOCK, H)
    u = up.reshape(F_ // _BLOCK, _BLOCK, H)
    return torch.stack((g, u), dim=1).reshape(2 * F_, H).contiguous()


def pack_mlp(gate, up, down):
    """(w_gu, w_down) for the SwiGLU GEMM pair.  Any FFN width works (e.g. the
    wider MLPs that WideTuning's to_dense merges, src/kadllm/widetuning.py:96-127):
    the width is zero-padded to a multiple of 64, which adds exact zeros --
    silu(0) * 0 = 0 through padded gate/up rows, and zero down-projection
    columns."""
    F_, H = gate.shape
    pad = (-F_) % 64
    if pad:
        gate = torch.cat((gate, gate.new_zeros(pad, H)), 0)
        up = torch.cat((up, up.new_zeros(pad, H)), 0)
        down = torch.cat((down, down.new_zeros(down.shape[0], pad)), 1)
    return interleave_gate_up(gate, up), down.contiguous()


class Qwen35Runner:
    """Packed bf16 weights of one Qwen3.5 text model plus its forward passes.

    ``head_tokens`` (optional int64 token ids) gives a SID-only head: the LM
    head projects only to those tokens (README.md:164, the production head that
    projects to the semantic-ID tokens), logits column c is token
    head_tokens[c], and the softmax of a search runs over that sub-vocabulary.
    """

    dtype = torch.bfloat16

    def __init__(self, cfg, state_dict, lm_head_weight=None, device=None, head_tokens=None):
        self.cfg = cfg
        self.device = torch.device(device) if device is not None else \
            state_dict["embed_tokens.weight"].device
        if self.device.type != "cuda":
            raise RuntimeError("the native Qwen3.5 path runs on a ROCm device")
        bf = torch.bfloat16

        def get(name):
            return state_dict[name].detach().to(device=self.device, dtype=bf).contiguous()

        H = cfg.hidden_size
        if H % 64:
            raise ValueError("hidden size must be a multiple of 64 for the GEMM kernels")
        reject_biases(cfg, state_dict)
        self.embed = get("embed_tokens.weight")
        head = lm_head_weight if lm_head_weight is not None else state_dict.get("lm_head.weight")
        self.lm_head = (self.embed if head is None else
                        head.detach().to(device=self.device, dtype=bf).contiguous())
        self.head_ids = None
        if head_tokens is not None:
            ids = torch.as_tensor(head_tokens, dtype=torch.int64, device=self.device)
            if ids.ndim != 1 or ids.numel() < 1 or int(ids.min()) < 0 or \
                    int(ids.max()) >= self.lm_head.shape[0]:
                raise ValueError("head_tokens must be a nonempty 1-D list of vocabulary ids")
            self.head_ids = ids.contiguous()
            self.lm_head = self.lm_head.index_select(0, self.head_ids).contiguous()
        self.norm_w = get("norm.weight")
        self.kd = cfg.linear_num_key_heads * cfg.linear_key_head_dim
        self.vd = cfg.linear_num_value_heads * cfg.linear_value_head_dim
        self.conv_dim = 2 * self.kd + self.vd
        hv = cfg.linear_num_value_heads
        self.gdn_cols = _round_up(self.conv_dim + self.vd + 2 * hv, 64)
        self.attn_cols = (2 * cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * cfg.head_dim
        self.layers = []
        for i, kind in enumerate(cfg.layer_types):
            p = f"layers.{i}."
            w_gu, w_down = pack_mlp(get(p + "mlp.gate_proj.weight"), get(p + "mlp.up_proj.weight"),
                                    get(p + "mlp.down_proj.weight"))
            common = dict(input_norm=get(p + "input_layernorm.weight"),
                          post_norm=get(p + "post_attention_layernorm.weight"),
                          w_gu=w_gu, w_down=w_down)
            if kind == "linear_attention":
                a = p + "linear_attn."
                # two GEMMs fill one projection row [qkv | z | a | b | pad]: the
                # wide [qkv | z] one keeps its N a multiple of the 256-column
                # tile (the 32 gate columns would add a nearly empty column
                # of tiles to it)
                w_in = torch.cat((get(a + "in_proj_qkv.weight"), get(a + "in_proj_z.weight")),
                                 0).contiguous()
                w_ab = torch.cat((get(a + "in_proj_a.weight"), get(a + "in_proj_b.weight")),
                                 0).contiguous()
                if cfg.linear_conv_kernel_dim != 4:
                    raise ValueError("the conv kernels are specialised for width 4")
                self.layers.append(_GdnLayer(
                    w_in=w_in, w_ab=w_ab, conv_w=get(a + "conv1d.weight").reshape(self.conv_dim, 4).contiguous(),
                    A_log=get(a + "A_log"), dt_bias=get(a + "dt_bias"), norm_w=get(a + "norm.weight"),
                    w_out=get(a + "out_proj.weight"), **common))
            else:
                a = p + "self_attn."
                w_qkv = torch.cat((get(a + "q_proj.weight"), get(a + "k_proj.weight"),
                                   get(a + "v_proj.weight")), 0).contiguous()
                self.layers.append(_AttnLayer(w_qkv=w_qkv, q_norm=get(a + "q_norm.weight"),
                                              k_norm=get(a + "k_norm.weight"),
                                              w_o=get(a + "o_proj.weight"), **common))
        # optional observer: trace(phase, layer, x) after each layer with a copy
        # of the residual stream rows (the last position only past a pruned
        # last layer); phase is "prefill", "decode" or "step"
        self.trace = None
        rot = int(cfg.head_dim * cfg.partial_rotary_factor)
        self.rot = rot
        self.inv_freq = (1.0 / (cfg.rope_theta ** (torch.arange(0, rot, 2, dtype=torch.float) / rot))
                         ).to(self.device)

    # ------------------------------------------------------------------
    def _mlp(self, lyr, x, rows, prefetch=False):
        cfg = self.cfg
        if prefetch:
            layers.cache_prefetch(lyr.w_gu, lyr.w_down)
        n2 = layers.rmsnorm(x, lyr.post_norm, cfg.rms_norm_eps)
        h = layers.gemm(n2, lyr.w_gu, epilogue=layers.EPI_SWIGLU)
        layers.gemm(h, lyr.w_down, out=x, epilogue=layers.EPI_RESIDUAL, residual=x)

    def _gdn_proj(self, lyr, n, out=None):
        """[rows, gdn_cols] projection row [qkv | z | a | b | pad] of n (or into out)."""
        if out is None:
            out = torch.empty(n.shape[0], self.gdn_cols, dtype=torch.bfloat16, device=n.device)
        c = self.conv_dim + self.vd
        # the 32-column gate projection first, while n is still in the caches
        # the large projection's output then sweeps out
        layers.gemm(n, lyr.w_ab, out=out[:, c:c + lyr.w_ab.shape[0]])
        layers.gemm(n, lyr.w_in, out=out[:, :c])
        return out

    def _gdn_proj_conv(self, lyr, n, B, L, conv_state):
        """The prefill's projection rows and the causal conv (+ SiLU) of their
        q | k | v channels: (proj [rows, gdn_cols], conv) with conv the rows
        holding the conv outputs in columns [0, conv_dim).  Where the shape
        allows, one call (kad_gemm_bf16_conv) writes the conv outputs straight
        into proj's q | k | v columns (the same bits), and conv is proj;
        otherwise the plain projection and kad_causal_conv_prefill into a
        buffer of its own.  conv_state receives each prompt's last 4 inputs."""
        rows = n.shape[0]
        C = self.conv_dim
        c = C + self.vd
        dev = n.device
        stream = _lib.stream_of(n)
        w_in = lyr.w_in
        if (L % 128 == 0 and rows % 256 == 0 and c % 256 == 0 and C % 256 == 0
                and n.shape[1] % 64 == 0 and lyr.conv_w.is_contiguous()
                and lyr.conv_w.data_ptr() % 16 == 0):
            proj = torch.empty(rows, self.gdn_cols, dtype=torch.bfloat16, device=dev)
            layers.gemm(n, lyr.w_ab, out=proj[:, c:c + lyr.w_ab.shape[0]])
            nb = ctypes.c_int64(0)
            _lib.call("kad_gemm_bf16_conv_workspace_bytes", rows, C, ctypes.byref(nb))
            ws = torch.empty(nb.value, dtype=torch.uint8, device=dev)
            _lib.call("kad_gemm_bf16_conv", _lib.ptr(n), n.stride(0), _lib.ptr(w_in),
                      w_in.stride(0), _lib.ptr(proj), proj.stride(0), rows, c, n.shape[1], C,
                      _lib.ptr(lyr.conv_w), L, _lib.ptr(conv_state), _lib.ptr(ws), ws.numel(),
                      stream)
            return proj, proj
        proj = self._gdn_proj(lyr, n)
        conv = torch.empty(rows, C, dtype=torch.bfloat16, device=dev)
        _lib.call("kad_causal_conv_prefill", _lib.ptr(proj), proj.stride(0), _lib.ptr(lyr.conv_w),
                  _lib.ptr(conv), conv.stride(0), _lib.ptr(conv_state), n.shape[0] // L, L, C, 1,
                  stream)
        return proj, conv

    def _gdn_gates(self, lyr, proj):
        hv = self.cfg.linear_num_value_heads
        o = self.conv_dim + self.vd
        return layers.gdn_gates(proj[:, o:o + hv], proj[:, o + hv:o + 2 * hv], lyr.A_log,
                                lyr.dt_bias)

    def _gdn_replay(self, conv, g, beta, S, o, B, W, T):
        """Each beam's T suffix tokens applied to its request's prefix state S
        (q, k, v are column ranges of the conv output rows).  Up to 8 tokens
        the factored MFMA replay, whose arithmetic for a token does not depend
        on how many follow it (so a cached suffix extended by one token gives
        the stateless replay's bits); longer suffixes the per-token recurrence
        (kad_gdn_recurrent), the reference torch path's arithmetic in fp32."""
        cfg = self.cfg
        H_, HV = cfg.linear_num_key_heads, cfg.linear_num_value_heads
        dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
        C = self.conv_dim
        base, es = conv.data_ptr(), conv.element_size()
        args = (_lib.ptr(conv), _lib.ptr_at(base + self.kd * es), _lib.ptr_at(base + 2 * self.kd * es),
                C, C, 0, _lib.ptr(g), 2, _lib.ptr(beta), 0, HV, _lib.ptr(S),
                _lib.dtype_code(S.dtype))
        if T <= REPLAY_MAX_T:
            _lib.call("kad_gdn_suffix_replay", *args, _lib.ptr(o), self.vd, B, W, T, H_, HV, dk,
                      dv, float(dk ** -0.5), _lib.stream_of(conv))
        else:
            _lib.call("kad_gdn_recurrent", *args, W, _lib.ptr(o), self.vd, None, B * W, T, H_, HV,
                      dk, dv, float(dk ** -0.5), _lib.stream_of(conv))

    def _mixer_fusable(self, lyr, W):
        """Whether the fused decode mixer takes this layer's shapes (besides
        the suffix length and row alignment, checked where it is called)."""
        cfg = self.cfg
        return (W % 16 == 0 and cfg.linear_key_head_dim == 128
                and cfg.linear_value_head_dim == 128 and self.gdn_cols % 8 == 0
                and lyr.conv_w.is_contiguous() and lyr.conv_w.data_ptr() % 8 == 0
                and lyr.norm_w.data_ptr() % 8 == 0
                and cfg.linear_num_value_heads % 2 == 0)

    def _gdn_mix_parents(self, lyr, n, prev, parents, cached, B, W, Wp, T):
        """_gdn_mix for the search's last level (last token only, T = 2) with
        the earlier token's projection rows read in place from the parent
        level's cache (kad_gdn_suffix_replay_conv_gated_parents): only the new
        token's rows are projected, and only the parents' gate inputs (a | b,
        64 bytes a row) are gathered.  The same bits as gathering the rows."""
        cfg = self.cfg
        H_, HV = cfg.linear_num_key_heads, cfg.linear_num_value_heads
        dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
        C = self.conv_dim
        c = C + self.vd
        cols = self.gdn_cols
        BW = B * W
        dev = n.device
        stream = _lib.stream_of(n)
        nab = lyr.w_ab.shape[0]
        ab = torch.empty(BW * T, nab, dtype=torch.bfloat16, device=dev)
        _lib.call("kad_gather_beam_rows", _lib.ptr_at(prev.data_ptr() + c * 2), cols * 2, T - 1,
                  _lib.ptr(ab), nab * 2, T, T - 1, nab * 2, _lib.ptr(parents), B, W, Wp, stream)
        cur = torch.empty(BW, cols, dtype=torch.bfloat16, device=dev)
        layers.gemm(n, lyr.w_ab, out=ab.view(BW, T, nab)[:, T - 1])
        layers.gemm(n, lyr.w_in, out=cur[:, :c])
        g, beta = layers.gdn_gates(ab[:, :HV], ab[:, HV:2 * HV], lyr.A_log, lyr.dt_bias)
        cs, S = cached
        z = cur[:, C:C + self.vd]
        y = torch.empty(BW, self.vd, dtype=torch.bfloat16, device=dev)
        _lib.call("kad_gdn_suffix_replay_conv_gated_parents", _lib.ptr(prev), cols,
                  _lib.ptr(parents), Wp, _lib.ptr(cur), cols, _lib.ptr(cs), *cs.stride(),
                  cs.shape[-1], _lib.ptr(lyr.conv_w), _lib.ptr(g), 2, _lib.ptr(beta), 0,
                  g.stride(0), _lib.ptr(S), _lib.dtype_code(S.dtype), _lib.ptr(z), cols,
                  _lib.ptr(lyr.norm_w), cfg.rms_norm_eps, _lib.ptr(y), self.vd, B, W, T, H_, HV,
                  dk, dv, float(dk ** -0.5), stream)
        return y

    def _gdn_mix(self, lyr, proj, T, cached, B, W, last_only):
        """A GDN layer's suffix mixer up to out_proj: conv of the projection
        rows' q | k | v channels, replay against the prefix state, gated
        RMSNorm.  Returns the normed rows [B*W, vd] (each beam's last token,
        last_only) or [B*W*T, vd].  One fused call
        (kad_gdn_suffix_replay_conv_gated, the same bits) where it takes the
        shape, else kad_causal_conv_suffix into a buffer, _gdn_replay and
        kad_rmsnorm_gated.  proj: [B*W*T, cols] rows, token-major per beam."""
        cfg = self.cfg
        H_, HV = cfg.linear_num_key_heads, cfg.linear_num_value_heads
        dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
        C = self.conv_dim
        BW = B * W
        ld = proj.stride(0)
        dev = proj.device
        stream = _lib.stream_of(proj)
        cs, S = cached
        g, beta = self._gdn_gates(lyr, proj)
        z = proj[:, C:C + self.vd]
        if (T <= 2 and W % 16 == 0 and dk == 128 and dv == 128 and g.stride(0) % 2 == 0
                and ld % 8 == 0 and proj.data_ptr() % 16 == 0 and lyr.conv_w.is_contiguous()
                and lyr.conv_w.data_ptr() % 8 == 0 and lyr.norm_w.data_ptr() % 8 == 0):
            y = torch.empty(BW if last_only else BW * T, self.vd, dtype=torch.bfloat16,
                            device=dev)
            _lib.call("kad_gdn_suffix_replay_conv_gated", _lib.ptr(proj), ld, _lib.ptr(cs),
                      *cs.stride(), cs.shape[-1], _lib.ptr(lyr.conv_w), _lib.ptr(g), 2,
                      _lib.ptr(beta), 0, g.stride(0), _lib.ptr(S), _lib.dtype_code(S.dtype),
                      _lib.ptr(z), ld, _lib.ptr(lyr.norm_w), cfg.rms_norm_eps,
                      1 if last_only else 0, _lib.ptr(y), self.vd, B, W, T, H_, HV, dk, dv,
                      float(dk ** -0.5), stream)
            return y
        conv = torch.empty(proj.shape[0], C, dtype=torch.bfloat16, device=dev)
        _lib.call("kad_causal_conv_suffix", _lib.ptr(proj), T * ld, 1, ld, _lib.ptr(cs),
                  *cs.stride(), cs.shape[-1], _lib.ptr(lyr.conv_w), 4, None,
                  _lib.ptr(conv), T * C, 1, C, B, W, C, T, 0, 1, stream)
        o = torch.empty(BW * T, self.vd, dtype=torch.bfloat16, device=dev)
        self._gdn_replay(conv, g, beta, S, o, B, W, T)
        if last_only:
            o, z = o.view(BW, T, -1)[:, -1], proj.view(BW, T, -1)[:, -1, C:C + self.vd]
        return layers.rmsnorm_gated(o, z, lyr.norm_w, cfg.rms_norm_eps, HV)

    def _gdn_finish(self, lyr, o, proj, x):
        cfg = self.cfg
        z = proj[:, self.conv_dim:self.conv_dim + self.vd]
        y = layers.rmsnorm_gated(o, z, lyr.norm_w, cfg.rms_norm_eps, cfg.linear_num_value_heads)
        layers.gemm(y, lyr.w_out, out=x, epilogue=layers.EPI_RESIDUAL, residual=x)

    def _attn_terminal(self, lyr, n, x_last, B, L):
        """Last-layer attention of the prefill: K/V for every position (the
        prefix), the query, attention, gate and o_proj for the last position
        only (added into x_last).  Returns the layer's (K, V) prefix views."""
        cfg = self.cfg
        nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        rows = n.shape[0]
        dev = n.device
        qcols = 2 * nh * hd
        kv = layers.gemm(n, lyr.w_qkv[qcols:])                  # [rows, k | v]
        ld = kv.stride(0)
        kc = torch.empty(B, nkv, L, hd, dtype=torch.bfloat16, device=dev)
        vc = torch.empty(B, nkv, L, hd, dtype=torch.bfloat16, device=dev)
        kv_strides = (nkv * L * hd, hd, L * hd)
        layers.qk_norm_rope(kv, ld, hd, nkv, lyr.k_norm, kc, kv_strides, L, rows, hd, self.rot,
                            self.inv_freq, 0, L, cfg.rms_norm_eps)
        layers.scatter_heads(kv[:, nkv * hd:], ld, nkv, hd, vc, kv_strides, L, rows)
        qg = layers.gemm(n.view(B, L, -1)[:, -1], lyr.w_qkv[:qcols])   # [B, q | gate per head]
        q = torch.empty(B, 1, nh, hd, dtype=torch.bfloat16, device=dev)
        layers.qk_norm_rope(qg, qg.stride(0), 2 * hd, nh, lyr.q_norm, q, (nh * hd, nh * hd, hd),
                            1, B, hd, self.rot, self.inv_freq, L - 1, 1, cfg.rms_norm_eps)
        k_all, v_all = kc.transpose(1, 2), vc.transpose(1, 2)  # [B, L, nkv, hd]
        att = prefix_attention_decode(q, k_all[:, :L - 1], v_all[:, :L - 1], k_all[:, L - 1:],
                                      v_all[:, L - 1:], 1, None, hd ** -0.5, gate=qg[:, hd:],
                                      gate_strides=(qg.stride(0), qg.stride(0), 2 * hd))
        layers.gemm(att.view(B, nh * hd), lyr.w_o, out=x_last, epilogue=layers.EPI_RESIDUAL,
                    residual=x_last)
        return k_all, v_all

    # ------------------------------------------------------------------
    @torch.no_grad()
    def prefill(self, input_ids):
        """Full prompt forward.  Returns (logits [B, V] bf16, per-layer prefix tuple)."""
        cfg = self.cfg
        B, L = input_ids.shape
        rows = B * L
        dev = self.device
        x = layers.embedding(input_ids, self.embed)
        H_, HV = cfg.linear_num_key_heads, cfg.linear_num_value_heads
        dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
        nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        snap = []
        # Terminal pruning: past the last layer's token mixer only the last
        # position of each prompt is used (its logits); the prefix needs that
        # layer's state or K/V for every position, but not its outputs.
        x_last = x.view(B, L, -1)[:, -1]
        for li, lyr in enumerate(self.layers):
            terminal = li == len(self.layers) - 1
            n = layers.rmsnorm(x, lyr.input_norm, cfg.rms_norm_eps)
            if isinstance(lyr, _GdnLayer):
                conv_state = torch.empty(B, self.conv_dim, 4, dtype=torch.bfloat16, device=dev)
                proj, conv = self._gdn_proj_conv(lyr, n, B, L, conv_state)
                g, beta = self._gdn_gates(lyr, proj)
                o = torch.empty(rows, self.vd, dtype=torch.bfloat16, device=dev)
                S = torch.empty(B, HV, dk, dv, dtype=torch.float32, device=dev)
                base = conv.data_ptr()
                es = conv.element_size()
                ws = _lib.gdn_chunk_workspace(B, L, HV, dk, dev)
                ldc = conv.stride(0)
                args = (_lib.ptr(conv), _lib.ptr_at(base + self.kd * es),
                        _lib.ptr_at(base + 2 * self.kd * es), ldc, ldc, 0,
                        _lib.ptr(g), 2, _lib.ptr(beta), 0, HV, None, 2, 1, _lib.ptr(o), self.vd,
                        _lib.ptr(S), _lib.ptr(ws), ws.numel(), B, L, H_, HV, dk, dv,
                        float(dk ** -0.5))
                if terminal:
                    _lib.call("kad_gdn_chunk", *args, 1, _lib.stream_of(x))
                    self._gdn_finish(lyr, o.view(B, L, -1)[:, -1], proj.view(B, L, -1)[:, -1],
                                     x_last)
                else:
                    # the chunk rule with the gated RMSNorm on its output rows
                    # (the same bits as kad_gdn_chunk then kad_rmsnorm_gated)
                    z = proj[:, self.conv_dim:self.conv_dim + self.vd]
                    _lib.call("kad_gdn_chunk_gated", *args, _lib.ptr(z), z.stride(0),
                              _lib.ptr(lyr.norm_w), float(cfg.rms_norm_eps), _lib.stream_of(x))
                    layers.gemm(o, lyr.w_out, out=x, epilogue=layers.EPI_RESIDUAL, residual=x)
                snap.append((conv_state, S))
            elif terminal:
                snap.append(self._attn_terminal(lyr, n, x_last, B, L))
            else:
                proj = layers.gemm(n, lyr.w_qkv)
                ld = proj.stride(0)
                q = torch.empty(B, L, nh, hd, dtype=torch.bfloat16, device=dev)
                kc = torch.empty(B, nkv, L, hd, dtype=torch.bfloat16, device=dev)
                vc = torch.empty(B, nkv, L, hd, dtype=torch.bfloat16, device=dev)
                layers.qk_norm_rope(proj, ld, 2 * hd, nh, lyr.q_norm, q, (0, nh * hd, hd), rows,
                                    rows, hd, self.rot, self.inv_freq, 0, L, cfg.rms_norm_eps)
                kv_strides = (nkv * L * hd, hd, L * hd)
                kp = proj[:, 2 * nh * hd:]
                layers.qk_norm_rope(kp, ld, hd, nkv, lyr.k_norm, kc, kv_strides, L, rows, hd,
                                    self.rot, self.inv_freq, 0, L, cfg.rms_norm_eps)
                layers.scatter_heads(proj[:, (2 * nh + nkv) * hd:], ld, nkv, hd, vc, kv_strides,
                                     L, rows)
                att = torch.empty(B, L, nh, hd, dtype=torch.bfloat16, device=dev)
                gate = proj[:, hd:]
                attention_prefill(q, kc.transpose(1, 2), vc.transpose(1, 2), hd ** -0.5,
                                  gate=gate, gate_strides=(L * ld, ld, 2 * hd), out=att)
                layers.gemm(att.view(rows, nh * hd), lyr.w_o, out=x,
                            epilogue=layers.EPI_RESIDUAL, residual=x)
                snap.append((kc.transpose(1, 2), vc.transpose(1, 2)))
            if terminal:
                self._mlp(lyr, x_last, B)
            else:
                self._mlp(lyr, x, rows)
            if self.trace is not None:
                self.trace("prefill", li, (x_last if terminal else x).clone())
        hN = layers.rmsnorm(x_last, self.norm_w, cfg.rms_norm_eps)
        logits = layers.gemm(hN, self.lm_head)
        return logits, tuple(snap)

    # ------------------------------------------------------------------
    @torch.no_grad()
    def decode(self, history, prefix_layers, prefix_length):
        """Replay [B, W, T] suffixes against the prefix; returns logits [B, W, V] bf16."""
        cfg = self.cfg
        B, W, T = history.shape
        BW = B * W
        R = BW * T
        dev = self.device
        x = layers.embedding(history, self.embed)
        H_, HV = cfg.linear_num_key_heads, cfg.linear_num_value_heads
        dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
        nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        C = self.conv_dim
        # terminal pruning: the logits read only each beam's last token, so the
        # last layer's mixer output, o_proj/out_proj and MLP run on those rows
        # (its K/V or conv/state inputs still cover the whole suffix)
        x_last = x.view(BW, T, -1)[:, -1]
        for li, (lyr, cached) in enumerate(zip(self.layers, prefix_layers)):
            terminal = li == len(self.layers) - 1 and T > 1
            n = layers.rmsnorm(x, lyr.input_norm, cfg.rms_norm_eps)
            if isinstance(lyr, _GdnLayer):
                proj = self._gdn_proj(lyr, n)
                y = self._gdn_mix(lyr, proj, T, cached, B, W, last_only=terminal)
                xo = x_last if terminal else x
                layers.gemm(y, lyr.w_out, out=xo, epilogue=layers.EPI_RESIDUAL, residual=xo)
            elif terminal:
                proj = layers.gemm(n, lyr.w_qkv)
                ld = proj.stride(0)
                # queries of the last token only (position prefix + T - 1), keys and
                # values of the whole suffix
                q = torch.empty(BW, 1, nh, hd, dtype=torch.bfloat16, device=dev)
                k = torch.empty(BW, T, nkv, hd, dtype=torch.bfloat16, device=dev)
                last_rows = proj.view(BW, T, -1)[:, -1]
                layers.qk_norm_rope(last_rows, T * ld, 2 * hd, nh, lyr.q_norm, q, (0, nh * hd, hd),
                                    BW, BW, hd, self.rot, self.inv_freq, prefix_length + T - 1, 1,
                                    cfg.rms_norm_eps)
                layers.qk_norm_rope(proj[:, 2 * nh * hd:], ld, hd, nkv, lyr.k_norm, k,
                                    (0, nkv * hd, hd), R, R, hd, self.rot, self.inv_freq,
                                    prefix_length, T, cfg.rms_norm_eps)
                v = proj[:, (2 * nh + nkv) * hd:].as_strided((BW, T, nkv, hd), (T * ld, ld, hd, 1))
                att = prefix_attention_decode(q, cached[0], cached[1], k, v, W, None,
                                              hd ** -0.5, gate=last_rows[:, hd:],
                                              gate_strides=(T * ld, T * ld, 2 * hd))
                layers.gemm(att.view(BW, nh * hd), lyr.w_o, out=x_last,
                            epilogue=layers.EPI_RESIDUAL, residual=x_last)
            else:
                proj = layers.gemm(n, lyr.w_qkv)
                ld = proj.stride(0)
                q = torch.empty(BW, T, nh, hd, dtype=torch.bfloat16, device=dev)
                k = torch.empty(BW, T, nkv, hd, dtype=torch.bfloat16, device=dev)
                layers.qk_norm_rope(proj, ld, 2 * hd, nh, lyr.q_norm, q, (0, nh * hd, hd), R, R,
                                    hd, self.rot, self.inv_freq, prefix_length, T,
                                    cfg.rms_norm_eps)
                layers.qk_norm_rope(proj[:, 2 * nh * hd:], ld, hd, nkv, lyr.k_norm, k,
                                    (0, nkv * hd, hd), R, R, hd, self.rot, self.inv_freq,
                                    prefix_length, T, cfg.rms_norm_eps)
                v = proj[:, (2 * nh + nkv) * hd:].as_strided((BW, T, nkv, hd), (T * ld, ld, hd, 1))
                att = prefix_attention_decode(q, cached[0], cached[1], k, v, W, None,
                                              hd ** -0.5, gate=proj[:, hd:],
                                              gate_strides=(T * ld, ld, 2 * hd))
                layers.gemm(att.view(R, nh * hd), lyr.w_o, out=x,
                            epilogue=layers.EPI_RESIDUAL, residual=x)
            if terminal:
                self._mlp(lyr, x_last, BW)
            else:
                self._mlp(lyr, x, R)
            if self.trace is not None:
                self.trace("decode", li, (x_last if terminal else x).clone())
        hN = layers.rmsnorm(x_last, self.norm_w, cfg.rms_norm_eps)
        logits = layers.gemm(hN, self.lm_head)
        return logits.view(B, W, -1)

    # ------------------------------------------------------------------
    @torch.no_grad()
    def decode_step(self, tokens, parents, prefix_layers, prefix_length, cache=None,
                    keep_cache=True):
        """One search level that extends each parent beam's suffix by one token.

        tokens [B, W] int64 are the new tokens, parents [B, W] int64 the
        indices of the previous level's beams they extend (ignored for the
        first level, ``cache=None``, whose parent is the prefix itself), and
        ``cache`` the DecodeCache the previous level returned.  Returns
        (logits [B, W, V] bf16, DecodeCache), the cache None with
        ``keep_cache=False`` (nothing keeps the layers' per-token rows then).

        The logits equal ``decode(history)`` for history = the parents'
        suffixes followed by ``tokens``: every per-token quantity of the cached
        tokens (GDN projection rows, attention K/V after norm and RoPE) is what
        the parent level computed for the same token at the same position, and
        every kernel's per-row arithmetic is independent of the batch, so only
        the new token's rows go through the projections, norms and MLP; the
        conv and the GDN replay run over the whole suffix and attention takes
        the new token's queries only.  The reference replays the whole suffix
        at every level (src/kadllm/adapters/qwen3_5.py:216; README.md:252).
        """
        cfg = self.cfg
        B, W = tokens.shape
        BW = B * W
        T = 1 if cache is None else cache.T + 1
        Wp = 1 if cache is None else cache.W
        dev = self.device
        parents = parents.to(torch.int64).contiguous() if cache is not None else None
        x = layers.embedding(tokens, self.embed)
        H_, HV = cfg.linear_num_key_heads, cfg.linear_num_value_heads
        dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
        nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        C = self.conv_dim
        pos = prefix_length + T - 1
        stream = _lib.stream_of(x)

        def follow(src, dst, rows_per_beam_src, row_bytes, ld_src, ld_dst):
            _lib.call("kad_gather_beam_rows", _lib.ptr(src), ld_src, rows_per_beam_src,
                      _lib.ptr(dst), ld_dst, T, T - 1, row_bytes, _lib.ptr(parents), B, W, Wp,
                      stream)

        # Weights arrive cold from HBM at every level (a layer's ~40 MB are long
        # gone from the 256 MB last-level cache by the next level), which costs
        # the 8,192-row GEMMs far more than their bytes: measured alone, the
        # SwiGLU projection took 128 against 110 us with only its weight cold,
        # QKV 99 against 83, down 66 against 61.  Reading the MLP weights (22
        # MB) before the post-mixer norm and an attention layer's QKV weight
        # before its input norm takes a few microseconds and restores the warm
        # times.  The prefill's 32,768-row GEMMs lose only 2-3 us cold, less
        # than the prefetch costs, and a GEMM of few rows reads its weight
        # once at HBM rate whether or not it was prefetched.
        prefetch = 2048 <= BW <= 16384
        new_layers = []
        for li, (lyr, cached) in enumerate(zip(self.layers, prefix_layers)):
            if prefetch and not isinstance(lyr, _GdnLayer):
                layers.cache_prefetch(lyr.w_qkv)
            n = layers.rmsnorm(x, lyr.input_norm, cfg.rms_norm_eps)
            if isinstance(lyr, _GdnLayer):
                cols = self.gdn_cols
                if T == 2 and not keep_cache and self._mixer_fusable(lyr, W):
                    # the last level reads the earlier token's rows from the
                    # parents' cache in place: no row gather
                    y = self._gdn_mix_parents(lyr, n, cache.layers[li], parents, cached, B, W,
                                              Wp, T)
                else:
                    proj = torch.empty(BW * T, cols, dtype=torch.bfloat16, device=dev)
                    pv = proj.view(BW, T, cols)
                    if T > 1:
                        follow(cache.layers[li], proj, T - 1, cols * 2, cols * 2, cols * 2)
                    self._gdn_proj(lyr, n, out=pv[:, T - 1])
                    y = self._gdn_mix(lyr, proj, T, cached, B, W, last_only=True)
                    if keep_cache:
                        new_layers.append(proj)
                layers.gemm(y, lyr.w_out, out=x, epilogue=layers.EPI_RESIDUAL, residual=x)
            else:
                proj = layers.gemm(n, lyr.w_qkv)
                ld = proj.stride(0)
                q = torch.empty(BW, 1, nh, hd, dtype=torch.bfloat16, device=dev)
                k_all = torch.empty(BW, T, nkv, hd, dtype=torch.bfloat16, device=dev)
                v_all = torch.empty(BW, T, nkv, hd, dtype=torch.bfloat16, device=dev)
                if T > 1:
                    kp, vp = cache.layers[li]
                    rb = nkv * hd * 2
                    follow(kp, k_all, T - 1, rb, rb, rb)
                    follow(vp, v_all, T - 1, rb, rb, rb)
                layers.qk_norm_rope(proj, ld, 2 * hd, nh, lyr.q_norm, q, (0, nh * hd, hd), BW, BW,
                                    hd, self.rot, self.inv_freq, pos, 1, cfg.rms_norm_eps)
                tok = (0, T * nkv * hd, hd)
                layers.qk_norm_rope(proj[:, 2 * nh * hd:], ld, hd, nkv, lyr.k_norm, k_all[:, T - 1],
                                    tok, BW, BW, hd, self.rot, self.inv_freq, pos, 1,
                                    cfg.rms_norm_eps)
                layers.scatter_heads(proj[:, (2 * nh + nkv) * hd:], ld, nkv, hd, v_all[:, T - 1],
                                     tok, BW, BW)
                att = prefix_attention_decode(q, cached[0], cached[1], k_all, v_all, W, None,
                                              hd ** -0.5, gate=proj[:, hd:],
                                              gate_strides=(ld, ld, 2 * hd))
                layers.gemm(att.view(BW, nh * hd), lyr.w_o, out=x, epilogue=layers.EPI_RESIDUAL,
                            residual=x)
                if keep_cache:
                    new_layers.append((k_all, v_all))
            self._mlp(lyr, x, BW, prefetch)
            if self.trace is not None:
                self.trace("step", li, x.clone())
        hN = layers.rmsnorm(x, self.norm_w, cfg.rms_norm_eps)
        logits = layers.gemm(hN, self.lm_head)
        return logits.view(B, W, -1), (DecodeCache(T, W, tuple(new_layers)) if keep_cache else None)


@dataclass
class DecodeCache:
    """Per-layer rows of the suffixes of one search level's beams.

    GDN layers: the fused input projection rows [B*W*T, cols] (token-major
    within each beam); attention layers: (K, V) [B*W, T, HK, D] after norm and
    RoPE.  Read by the next level through each beam's parent."""

    T: int
    W: int
    layers: tuple


class Qwen35TextModel:
    """Weights + config of a Qwen3.5 text model without transformers.

    Holds a state dict in the transformers Qwen3_5TextModel naming; accepted
    by Qwen35GRBeamAdapter wherever a transformers Qwen3_5TextModel is.
    """

    def __init__(self, config, state_dict):
        self.config = config
        self._sd = dict(state_dict)
        self.training = False

    def state_dict(self):
        return dict(self._sd)

    def parameters(self):
        return iter(self._sd.values())

    def eval(self):
        self.training = False
        return self

    def train(self, mode=True):
        self.training = mode
        return self


class LMHead:
    """A bias-free output projection holding ``weight`` [V, H] (tied or not)."""

    def __init__(self, weight):
        self.weight = weight
        self.training = False

    def parameters(self):
        return iter((self.weight,))

    def eval(self):
        self.training = False
        return self
