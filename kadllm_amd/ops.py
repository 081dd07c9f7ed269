"""GRBeam shared-prefix operators on MI355X (drop-in for ``kadllm.ops``).

Same names, arguments, layouts, validation order, exception types and
messages as the reference operators (src/kadllm/ops.py:17-341).  Execution
differs in one respect only: there is exactly one implementation per
operator, the HIP kernels of libkadllm_hip.so.  The reference's backend
strings are still accepted and validated -- "auto", "torch" and "triton" for
gated_delta / causal_conv1d, "torch" and "flash_attn" for prefix_attention --
and all of them run the HIP kernel.  Tensors must live on a ROCm device;
CPU tensors and requested gradients raise RuntimeError (inference only).

The persistent prefix (``shared_state``, ``prefix_k``/``prefix_v``) is
request-sized, read through const pointers and never written.
"""

import math

import torch

from . import _lib


def _backend(name, tensors):
    """Validate a backend string (src/kadllm/ops.py:17-38) and require the HIP path."""
    if name not in ("auto", "torch", "triton"):
        raise ValueError("backend must be auto, torch, or triton")
    _require_device(tensors)
    return name


def _require_device(tensors):
    gradients = torch.is_grad_enabled() and any(t.requires_grad for t in tensors)
    if gradients:
        raise RuntimeError("kadllm_amd operators are inference-only; disable gradients")
    if not all(t.is_cuda for t in tensors):
        raise RuntimeError(
            "kadllm_amd operators run on ROCm devices only; move tensors to the GPU")
    if any(t.dtype not in (torch.bfloat16, torch.float16, torch.float32) for t in tensors):
        raise RuntimeError("HIP operators require fp16/bf16/fp32 tensors")


def _same_device(tensors):
    if len({t.device for t in tensors}) != 1:
        raise ValueError("all tensors must be on the same device")
    if not all(t.is_floating_point() for t in tensors):
        raise TypeError("operator inputs must be floating-point tensors")


def _width(width):
    if not isinstance(width, int) or isinstance(width, bool) or width <= 0:
        raise ValueError("beam_width must be a positive integer")


def _gdn_launch(config):
    """Validate a launch tuple exactly as src/kadllm/ops.py:53-67.

    (tile_v, num_warps, num_stages[, beam_group]).  The HIP kernel chooses
    its own tiling; a beam_group value is accepted as a hint and the kernel
    always shares one state load across all beams of a request-head block.
    """
    if config is None:
        return
    if (
        not isinstance(config, tuple)
        or len(config) not in (3, 4)
        or any(type(value) is not int for value in config)
        or config[0] not in (8, 16, 32, 64, 128)
        or config[1] not in (1, 2, 4, 8)
        or config[2] not in (1, 2, 3)
        or (len(config) == 4 and config[3] not in (1, 2, 4, 8, 16))
    ):
        raise ValueError(
            "triton_config must be (tile_v, num_warps, num_stages[, beam_group])"
        )


# longest suffix of the factored replay kernel (kad_gdn_suffix_replay)
REPLAY_MAX_T = 8


def gated_delta(q, k, v, log_decay, beta, shared_state, *, beam_width: int = 1,
                scale: float | None = None, backend: str = "auto",
                return_final_state: bool = False,
                triton_config: tuple[int, ...] | None = None):
    """Gated delta recurrence starting from a shared prefix (src/kadllm/ops.py:70-163).

    q,k: [B*W,T,H,K]; v: [B*W,T,HV,V]; gates: [B*W,T,HV]; shared_state:
    [B,HV,K,V]; HV divisible by H.  q/k are L2-normalised (eps 1e-6), q scaled
    by ``scale`` (default K**-0.5); decay is in natural-log space.  Returns
    [B*W,T,HV,V] in v's dtype; with ``return_final_state`` also the per-beam
    final state [B*W,HV,K,V] fp32 (use W=1 to build a shared prefix).

    Key and value dims of 64 or 128 run the specialised kernels: suffixes of
    up to 8 tokens the factored replay (kad_gdn_suffix_replay), longer bf16
    ones and final-state requests the chunked kernel (kad_gdn_chunk).  Every
    other shape and dtype (fp16, fp32 beyond the replay, head dims up to 256)
    runs the token-by-token recurrence kernel (kad_gdn_recurrent).
    """
    _width(beam_width)
    _gdn_launch(triton_config)
    tensors = (q, k, v, log_decay, beta, shared_state)
    _same_device(tensors)
    if q.ndim != 4 or k.shape != q.shape or v.ndim != 4 or shared_state.ndim != 4:
        raise ValueError("invalid q/k/v/state ranks or shapes")
    BW, T, H, K = q.shape
    HV, V = v.shape[-2:]
    if min(BW, T, H, K, HV, V) <= 0 or HV % H or BW % beam_width:
        raise ValueError("empty dimensions or incompatible beam/head counts")
    if (
        v.shape[:2] != (BW, T)
        or log_decay.shape != (BW, T, HV)
        or beta.shape != log_decay.shape
        or shared_state.shape != (BW // beam_width, HV, K, V)
    ):
        raise ValueError("incompatible state, value, or gate shape")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q/k/v must have the same dtype")
    scale = K**-0.5 if scale is None else scale
    _backend(backend, tensors)
    if return_final_state and backend == "triton":
        raise ValueError("Triton decode does not return a final state")
    if triton_config is not None and (backend == "torch" or return_final_state):
        raise ValueError("triton_config requires the Triton execution path")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    log_decay, beta = log_decay.contiguous(), beta.contiguous()
    shared_state = shared_state.contiguous()
    B = BW // beam_width
    specialised = K in (64, 128) and V in (64, 128)
    if not specialised or q.dtype == torch.float16 or (
            q.dtype == torch.float32 and (T > REPLAY_MAX_T or return_final_state)):
        return gdn_recurrent(q, k, v, log_decay, beta, shared_state, beam_width=beam_width,
                             scale=scale, want_final=return_final_state)
    if T <= REPLAY_MAX_T and not return_final_state:
        out = torch.empty_like(v)
        _lib.call("kad_gdn_suffix_replay", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), H * K, HV * V,
                  _lib.dtype_code(q.dtype), _lib.ptr(log_decay), _lib.dtype_code(log_decay.dtype),
                  _lib.ptr(beta), _lib.dtype_code(beta.dtype), HV, _lib.ptr(shared_state),
                  _lib.dtype_code(shared_state.dtype), _lib.ptr(out), HV * V, B, beam_width, T,
                  H, HV, K, V, float(scale), _lib.stream_of(q))
        return out
    from .prefill import gdn_chunk
    out, final = gdn_chunk(q, k, v, log_decay, beta, shared_state, beam_width=beam_width,
                           scale=scale, want_final=return_final_state)
    return (out, final) if return_final_state else out


def gdn_recurrent(q, k, v, log_decay, beta, shared_state, *, beam_width=1, scale=None,
                  want_final=False):
    """The per-token gated delta rule of src/kadllm/ops.py:139-163 on the GPU
    (kad_gdn_recurrent) for contiguous q, k [N,T,H,K], v [N,T,HV,V], gates
    [N,T,HV], shared_state [N/beam_width,HV,K,V] or None (zeros).  Returns out
    [N,T,HV,V] in v's dtype, or (out, final fp32 [N,HV,K,V]) with want_final."""
    N, T, H, K = q.shape
    HV, V = v.shape[-2:]
    scale = K ** -0.5 if scale is None else scale
    out = torch.empty_like(v)
    final = torch.empty(N, HV, K, V, dtype=torch.float32, device=v.device) if want_final else None
    st = shared_state
    _lib.call("kad_gdn_recurrent", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), H * K, HV * V,
              _lib.dtype_code(q.dtype), _lib.ptr(log_decay), _lib.dtype_code(log_decay.dtype),
              _lib.ptr(beta), _lib.dtype_code(beta.dtype), HV, _lib.ptr(st),
              _lib.dtype_code(st.dtype) if st is not None else 2, beam_width, _lib.ptr(out),
              HV * V, _lib.ptr(final), N, T, H, HV, K, V, float(scale), _lib.stream_of(v))
    return (out, final) if want_final else out


def causal_conv1d(x, shared_state, weight, *, beam_width: int = 1, bias=None,
                  activation: str | None = "silu", backend: str = "auto"):
    """Stateless depthwise short convolution (src/kadllm/ops.py:166-226).

    x: [B*W,C,T] (any strides); shared_state: [B,C,history]; weight:
    [C,width].  Only the last width-1 prefix taps are consumed.  Returns
    [B*W,C,T].  shared_state is never written.
    """
    _width(beam_width)
    tensors = (x, shared_state, weight) + (() if bias is None else (bias,))
    _same_device(tensors)
    if x.ndim != 3 or shared_state.ndim != 3 or weight.ndim != 2:
        raise ValueError("invalid convolution input ranks")
    BW, C, T = x.shape
    width = weight.shape[-1]
    if (
        min(BW, C, T, width) < 1
        or BW % beam_width
        or shared_state.shape[:2] != (BW // beam_width, C)
        or shared_state.shape[-1] < width - 1
        or weight.shape[0] != C
    ):
        raise ValueError("incompatible convolution shapes")
    if len({t.dtype for t in tensors}) != 1:
        raise ValueError("convolution inputs must have the same dtype")
    if bias is not None and bias.shape != (C,):
        raise ValueError("bias must have shape [C]")
    if activation not in (None, "silu"):
        raise ValueError("activation must be None or silu")
    _backend(backend, tensors)
    if (width != 4 or bias is not None or activation != "silu") and backend == "triton":
        raise ValueError("Triton short-conv requires width=4, SiLU, and no bias")
    weight = weight.contiguous()
    bias = None if bias is None else bias.contiguous()
    # [BW, C, T] in x's layout: token-major x (channels contiguous, as a
    # projection's rows give it) gets a token-major result
    if x.stride() == (T * C, 1, C):
        out = torch.empty(BW, T, C, dtype=x.dtype, device=x.device).transpose(1, 2)
    else:
        out = torch.empty(BW, C, T, dtype=x.dtype, device=x.device)
    _lib.call("kad_causal_conv_suffix", _lib.ptr(x), *x.stride(), _lib.ptr(shared_state),
              *shared_state.stride(), shared_state.shape[-1], _lib.ptr(weight), width,
              _lib.ptr(bias), _lib.ptr(out), *out.stride(), BW // beam_width, beam_width, C, T,
              _lib.dtype_code(x.dtype), int(activation == "silu"), _lib.stream_of(x))
    return out


def merge_attention(prefix_out, prefix_lse, suffix_out, suffix_lse):
    """Merge two independently normalized attention partitions using LSE.

    src/kadllm/ops.py:243-249.  Elementwise torch arithmetic on the caller's
    tensors (the fused attention kernel performs this merge internally).
    """
    total = torch.logaddexp(prefix_lse, suffix_lse)
    return (
        prefix_out * (prefix_lse - total).exp()[..., None]
        + suffix_out * (suffix_lse - total).exp()[..., None]
    )


def prefix_attention(q, prefix_k, prefix_v, suffix_k, suffix_v, *, beam_width: int = 1,
                     prefix_mask: torch.Tensor | None = None, scale: float | None = None,
                     backend: str = "torch", gate: torch.Tensor | None = None):
    """Shared-prefix attention plus a causal replay suffix, GQA (src/kadllm/ops.py:252-341).

    Layout: q [B*W,T,H,D], prefix K/V [B,L,HK,D] (any strides), suffix K/V
    [B*W,T,HK,D].  prefix_mask [B,L] is True for valid keys.  Returns
    [B*W,T,H,D] in q's dtype.  ``gate`` (an extension, [B*W,T,H*D]) multiplies
    the output by sigmoid(gate) inside the kernel, the gated-attention output
    of Qwen3.5 (src/kadllm/adapters/qwen3_5.py:199-201).
    """
    _width(beam_width)
    tensors = (q, prefix_k, prefix_v, suffix_k, suffix_v)
    _same_device(tensors)
    if any(t.ndim != 4 for t in tensors):
        raise ValueError("attention inputs must all have rank 4")
    BW, T, H, D = q.shape
    B, L, HK, DK = prefix_k.shape
    if (
        min(BW, T, H, D, B, HK) < 1
        or BW != B * beam_width
        or H % HK
        or DK != D
        or prefix_v.shape != prefix_k.shape
        or suffix_k.shape != (BW, T, HK, D)
        or suffix_v.shape != suffix_k.shape
    ):
        raise ValueError("incompatible attention shapes")
    if len({t.dtype for t in tensors}) != 1:
        raise ValueError("attention inputs must have the same dtype")
    if prefix_mask is not None and (
        prefix_mask.shape != (B, L)
        or prefix_mask.dtype != torch.bool
        or prefix_mask.device != q.device
    ):
        raise ValueError("prefix_mask must be bool [B,L] on the query device")
    scale = 1 / math.sqrt(D) if scale is None else scale
    if backend not in ("torch", "flash_attn"):
        raise ValueError("attention backend must be torch or flash_attn")
    _require_device(tensors)
    from .attention import prefix_attention_decode

    return prefix_attention_decode(q, prefix_k, prefix_v, suffix_k, suffix_v, beam_width,
                                   prefix_mask, scale, gate)
