"""fp32 Qwen3.5 hybrid text model on the HIP kernels: prefill and suffix replay.

The reference adapter wraps a transformers model in whatever float dtype it
was loaded in (src/kadllm/adapters/qwen3_5.py:40-104); with an fp32 model
every step of its prefill (the transformers forward, qwen3_5.py:111) and of
its decode (qwen3_5.py:204-235) is fp32 arithmetic.  This runner is that
model on the GPU with no rounding anywhere: projections on the fp32 MFMA
GEMM (kad_gemm_f32), fp32 row-wise kernels (kad_rmsnorm_f32,
kad_rmsnorm_gated_f32, kad_gdn_gates_f32, kad_qk_norm_rope_f32,
kad_embedding_f32), the depthwise conv (kad_causal_conv_suffix, the prompt
with zero history at prefill), the token-by-token gated delta rule with the
fp32 state (kad_gdn_recurrent; at prefill from a zero state, keeping the
final state as the prefix) and one softmax over prefix and causal suffix keys
(kad_attention_general; a prompt is an all-suffix query with no prefix).
Decode is the stateless replay of the whole suffix, as in the reference.
"""

import torch

from . import _lib
from .attention import prefix_attention_general
from .qwen35 import pack_mlp, reject_biases

EPI_STORE, EPI_RESIDUAL, EPI_SWIGLU = 0, 1, 2


def gemm(a, w, out=None, *, epilogue=EPI_STORE, residual=None):
    """out = epilogue(a @ w^T) in fp32; a, w, out row-strided 2-D views."""
    M, K = a.shape
    N = w.shape[0]
    n_out = N // 2 if epilogue == EPI_SWIGLU else N
    if out is None:
        out = torch.empty(M, n_out, dtype=torch.float32, device=a.device)
    r = residual
    _lib.call("kad_gemm_f32", _lib.ptr(a), a.stride(0), _lib.ptr(w), w.stride(0), _lib.ptr(out),
              out.stride(0), _lib.ptr(r), r.stride(0) if r is not None else 0, M, N, K, epilogue,
              _lib.stream_of(a))
    return out


def rmsnorm(x, w, eps, w_offset=1.0):
    rows, D = x.shape
    out = torch.empty(rows, D, dtype=torch.float32, device=x.device)
    _lib.call("kad_rmsnorm_f32", _lib.ptr(x), x.stride(0), _lib.ptr(w), float(w_offset),
              _lib.ptr(out), out.stride(0), rows, D, float(eps), _lib.stream_of(x))
    return out


class Qwen35RunnerF32:
    """fp32 weights of one Qwen3.5 text model and its forward passes on the GPU.

    The same interface as the bf16 ``Qwen35Runner`` for prefill/decode (and
    ``head_tokens`` for a SID-only head); there is no incremental decode."""

    dtype = torch.float32

    def __init__(self, cfg, state_dict, lm_head_weight=None, device=None, head_tokens=None):
        self.cfg = cfg
        self.device = torch.device(device) if device is not None else \
            state_dict["embed_tokens.weight"].device
        if self.device.type != "cuda":
            raise RuntimeError("the native Qwen3.5 path runs on a ROCm device")
        reject_biases(cfg, state_dict)
        f32 = torch.float32

        def get(name):
            return state_dict[name].detach().to(device=self.device, dtype=f32).contiguous()

        self.embed = get("embed_tokens.weight")
        head = lm_head_weight if lm_head_weight is not None else state_dict.get("lm_head.weight")
        self.lm_head = self.embed if head is None else \
            head.detach().to(device=self.device, dtype=f32).contiguous()
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
        self.ks = cfg.linear_conv_kernel_dim
        self.layers = []
        for i, kind in enumerate(cfg.layer_types):
            p = f"layers.{i}."
            w_gu, w_down = pack_mlp(get(p + "mlp.gate_proj.weight"), get(p + "mlp.up_proj.weight"),
                                    get(p + "mlp.down_proj.weight"))
            lyr = dict(kind=kind, input_norm=get(p + "input_layernorm.weight"),
                       post_norm=get(p + "post_attention_layernorm.weight"), w_gu=w_gu,
                       w_down=w_down)
            if kind == "linear_attention":
                a = p + "linear_attn."
                # one projection row [qkv | z | a | b]
                lyr.update(
                    w_in=torch.cat([get(a + n + ".weight") for n in
                                    ("in_proj_qkv", "in_proj_z", "in_proj_a", "in_proj_b")],
                                   0).contiguous(),
                    conv_w=get(a + "conv1d.weight").reshape(self.conv_dim, self.ks).contiguous(),
                    A_log=get(a + "A_log"), dt_bias=get(a + "dt_bias"),
                    norm_w=get(a + "norm.weight"), w_out=get(a + "out_proj.weight"))
            else:
                a = p + "self_attn."
                lyr.update(w_qkv=torch.cat([get(a + n + ".weight") for n in
                                            ("q_proj", "k_proj", "v_proj")], 0).contiguous(),
                           q_norm=get(a + "q_norm.weight"), k_norm=get(a + "k_norm.weight"),
                           w_o=get(a + "o_proj.weight"))
            self.layers.append(lyr)
        self.rot = int(cfg.head_dim * cfg.partial_rotary_factor)
        self.inv_freq = (1.0 / (cfg.rope_theta ** (
            torch.arange(0, self.rot, 2, dtype=torch.float) / self.rot))).to(self.device)

    # ------------------------------------------------------------------
    def _mlp(self, lyr, x):
        n2 = rmsnorm(x, lyr["post_norm"], self.cfg.rms_norm_eps)
        h = gemm(n2, lyr["w_gu"], epilogue=EPI_SWIGLU)
        gemm(h, lyr["w_down"], out=x, epilogue=EPI_RESIDUAL, residual=x)

    def _gates(self, lyr, proj):
        hv = self.cfg.linear_num_value_heads
        o = self.conv_dim + self.vd
        a, b = proj[:, o:o + hv], proj[:, o + hv:o + 2 * hv]
        rows = proj.shape[0]
        g = torch.empty(rows, hv, dtype=torch.float32, device=proj.device)
        beta = torch.empty_like(g)
        _lib.call("kad_gdn_gates_f32", _lib.ptr(a), a.stride(0), _lib.ptr(b), b.stride(0),
                  _lib.ptr(lyr["A_log"]), _lib.ptr(lyr["dt_bias"]), _lib.ptr(g), _lib.ptr(beta),
                  rows, hv, _lib.stream_of(proj))
        return g, beta

    def _gdn(self, lyr, proj, conv, N, T, state, beams_per_state, want_final):
        """Gates, the recurrence over conv's q/k/v columns, the gated norm with
        z; returns (y [N*T, vd], final state or None)."""
        cfg = self.cfg
        H_, HV = cfg.linear_num_key_heads, cfg.linear_num_value_heads
        dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
        C = self.conv_dim
        g, beta = self._gates(lyr, proj)
        o = torch.empty(N * T, self.vd, dtype=torch.float32, device=proj.device)
        final = torch.empty(N, HV, dk, dv, dtype=torch.float32, device=proj.device) \
            if want_final else None
        base, es = conv.data_ptr(), conv.element_size()
        _lib.call("kad_gdn_recurrent", _lib.ptr(conv), _lib.ptr_at(base + self.kd * es),
                  _lib.ptr_at(base + 2 * self.kd * es), C, C, 2, _lib.ptr(g), 2, _lib.ptr(beta), 2,
                  HV, _lib.ptr(state), 2, beams_per_state, _lib.ptr(o), self.vd, _lib.ptr(final),
                  N, T, H_, HV, dk, dv, float(dk ** -0.5), _lib.stream_of(proj))
        z = proj[:, C:C + self.vd]
        y = torch.empty(N * T, self.vd, dtype=torch.float32, device=proj.device)
        _lib.call("kad_rmsnorm_gated_f32", _lib.ptr(o), o.stride(0), _lib.ptr(z), z.stride(0),
                  _lib.ptr(lyr["norm_w"]), _lib.ptr(y), y.stride(0), N * T, HV, dv,
                  float(cfg.rms_norm_eps), _lib.stream_of(proj))
        return y, final

    def _conv(self, lyr, proj, state, B, W, T, history):
        """SiLU(conv) of every row's qkv columns over [state taps || suffix]."""
        C = self.conv_dim
        ld = proj.stride(0)
        out = torch.empty(B * W * T, C, dtype=torch.float32, device=proj.device)
        _lib.call("kad_causal_conv_suffix", _lib.ptr(proj), T * ld, 1, ld, _lib.ptr(state),
                  *state.stride(), history, _lib.ptr(lyr["conv_w"]), self.ks, None, _lib.ptr(out),
                  T * C, 1, C, B, W, C, T, 2, 1, _lib.stream_of(proj))
        return out

    def _qk(self, src, ld, head_stride, heads, w, dst, rows, pos0, period):
        """Per-head RMSNorm(1+w) and RoPE of `rows` tokens into dst [rows, heads, D]."""
        cfg = self.cfg
        D = cfg.head_dim
        _lib.call("kad_qk_norm_rope_f32", _lib.ptr(src), ld, head_stride, heads, _lib.ptr(w),
                  _lib.ptr(dst), rows, 0, heads * D, D, rows, D, self.rot,
                  _lib.ptr(self.inv_freq), pos0, period, float(cfg.rms_norm_eps), 1,
                  _lib.stream_of(src))

    def _attention(self, lyr, n, N, T, prefix_k, prefix_v, W, pos0):
        """q/k norm + RoPE, attention over [prefix || causal suffix] with the
        sigmoid gate; returns (attention rows [N*T, nh*hd], suffix K, V)."""
        cfg = self.cfg
        nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        proj = gemm(n, lyr["w_qkv"])
        ld = proj.stride(0)
        rows = N * T
        q = torch.empty(N, T, nh, hd, dtype=torch.float32, device=n.device)
        k = torch.empty(N, T, nkv, hd, dtype=torch.float32, device=n.device)
        self._qk(proj, ld, 2 * hd, nh, lyr["q_norm"], q, rows, pos0, T)
        self._qk(proj[:, 2 * nh * hd:], ld, hd, nkv, lyr["k_norm"], k, rows, pos0, T)
        v = proj[:, (2 * nh + nkv) * hd:].as_strided((N, T, nkv, hd), (T * ld, ld, hd, 1))
        att = prefix_attention_general(q, prefix_k, prefix_v, k, v, W, None, hd ** -0.5,
                                       gate=proj[:, hd:], gate_strides=(T * ld, ld, 2 * hd))
        return att.view(rows, nh * hd), k, v.contiguous()

    # ------------------------------------------------------------------
    @torch.no_grad()
    def prefill(self, input_ids):
        """Full prompt forward: (logits [B, V] fp32, per-layer prefix tuple)."""
        cfg = self.cfg
        B, L = input_ids.shape
        dev = self.device
        x = self._embed(input_ids)
        C, ks = self.conv_dim, self.ks
        nkv, hd = cfg.num_key_value_heads, cfg.head_dim
        snap = []
        for lyr in self.layers:
            n = rmsnorm(x, lyr["input_norm"], cfg.rms_norm_eps)
            if lyr["kind"] == "linear_attention":
                proj = gemm(n, lyr["w_in"])
                zero = torch.zeros(B, C, ks - 1, dtype=torch.float32, device=dev)
                conv = self._conv(lyr, proj, zero, B, 1, L, ks - 1)
                # conv state: the last ks pre-conv inputs, zeros before the prompt
                conv_state = torch.zeros(B, C, ks, dtype=torch.float32, device=dev)
                take = min(L, ks)
                conv_state[:, :, ks - take:] = proj.view(B, L, -1)[:, L - take:, :C].transpose(1, 2)
                y, S = self._gdn(lyr, proj, conv, B, L, None, 1, True)
                gemm(y, lyr["w_out"], out=x, epilogue=EPI_RESIDUAL, residual=x)
                snap.append((conv_state, S))
            else:
                empty = torch.empty(B, 0, nkv, hd, dtype=torch.float32, device=dev)
                att, k, v = self._attention(lyr, n, B, L, empty, empty, 1, 0)
                gemm(att, lyr["w_o"], out=x, epilogue=EPI_RESIDUAL, residual=x)
                snap.append((k, v))
            self._mlp(lyr, x)
        hN = rmsnorm(x.view(B, L, -1)[:, -1], self.norm_w, cfg.rms_norm_eps)
        return gemm(hN, self.lm_head), tuple(snap)

    @torch.no_grad()
    def decode(self, history, prefix_layers, prefix_length):
        """Replay [B, W, T] suffixes against the prefix: logits [B, W, V] fp32."""
        cfg = self.cfg
        B, W, T = history.shape
        BW = B * W
        x = self._embed(history)
        for lyr, cached in zip(self.layers, prefix_layers):
            n = rmsnorm(x, lyr["input_norm"], cfg.rms_norm_eps)
            if lyr["kind"] == "linear_attention":
                proj = gemm(n, lyr["w_in"])
                conv = self._conv(lyr, proj, cached[0], B, W, T, cached[0].shape[-1])
                y, _ = self._gdn(lyr, proj, conv, BW, T, cached[1], W, False)
                gemm(y, lyr["w_out"], out=x, epilogue=EPI_RESIDUAL, residual=x)
            else:
                att, _, _ = self._attention(lyr, n, BW, T, cached[0], cached[1], W, prefix_length)
                gemm(att, lyr["w_o"], out=x, epilogue=EPI_RESIDUAL, residual=x)
            self._mlp(lyr, x)
        hN = rmsnorm(x.view(BW, T, -1)[:, -1], self.norm_w, cfg.rms_norm_eps)
        return gemm(hN, self.lm_head).view(B, W, -1)

    def _embed(self, ids):
        ids = ids.reshape(-1).to(torch.int64).contiguous()
        D = self.embed.shape[1]
        out = torch.empty(ids.numel(), D, dtype=torch.float32, device=self.device)
        _lib.call("kad_embedding_f32", _lib.ptr(ids), _lib.ptr(self.embed), _lib.ptr(out),
                  ids.numel(), D, self.embed.shape[0], _lib.stream_of(out))
        return out


class Qwen35RunnerF16(Qwen35RunnerF32):
    """fp16 models (the reference adapter wraps a model in any float dtype,
    src/kadllm/adapters/qwen3_5.py:40-104) on the fp32 kernels above: the
    weights are widened once, at construction, and every step runs in fp32,
    which carries the fp16 model's arithmetic more accurately than fp16
    rounding would.  Logits and the prefix are fp32, as for an fp32 model."""

    source_dtype = torch.float16
