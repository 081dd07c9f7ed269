"""Host wrappers of the HIP attention kernels (decode with shared prefix; causal prefill)."""

import torch

from . import _lib

# longest per-beam suffix the MFMA decode kernel folds in (kad_prefix_attention_decode_ex)
MFMA_MAX_SUFFIX = 8


def _inner_contiguous(t):
    """Return t if its last dim is contiguous and its other strides are multiples of 8."""
    if t.stride(-1) == 1 and all(s % 8 == 0 for s in t.stride()[:-1]) and t.data_ptr() % 16 == 0:
        return t
    return t.contiguous()


def prefix_attention_decode(q, prefix_k, prefix_v, suffix_k, suffix_v, beam_width, prefix_mask,
                            scale, gate=None, out=None, gate_strides=None):
    """q [B*W,T,H,D]; prefix K/V [B,L,HK,D] (strided views allowed); suffix K/V
    [B*W,Tk,HK,D] with Tk >= T (the queries are the last T of the Tk suffix
    tokens; Tk = T is the reference operator); optional bool prefix_mask [B,L];
    optional gate [B*W,T,H*D] (output multiplied by sigmoid(gate)), or any
    tensor whose data pointer is head 0's gate with element strides
    ``gate_strides`` = (beam, token, head).  Returns [B*W,T,H,D] in q's dtype.
    bf16 with head dims 64/128/256 and suffixes of at most 8 tokens run the
    MFMA kernel (kad_prefix_attention_decode_ex); every other shape and dtype
    the general kernel (kad_attention_general)."""
    BW, T, H, D = q.shape
    Tk = suffix_k.shape[1]
    B, L, HK, _ = prefix_k.shape
    if q.dtype != torch.bfloat16 or D not in (64, 128, 256) or Tk > MFMA_MAX_SUFFIX:
        return prefix_attention_general(q, prefix_k, prefix_v, suffix_k, suffix_v, beam_width,
                                        prefix_mask, scale, gate, out, gate_strides)
    q = _inner_contiguous(q)
    suffix_k = _inner_contiguous(suffix_k)
    if L:
        prefix_k = _inner_contiguous(prefix_k)
        prefix_v = _inner_contiguous(prefix_v)
        if prefix_k.stride() != prefix_v.stride():
            prefix_k, prefix_v = prefix_k.contiguous(), prefix_v.contiguous()
    if suffix_v.stride(-1) != 1 or any(s % 4 for s in suffix_v.stride()[:-1]):
        suffix_v = suffix_v.contiguous()
    mask = None
    if prefix_mask is not None:
        mask = prefix_mask.contiguous().view(torch.uint8)
    if gate is not None and gate_strides is not None:
        g_strides = tuple(gate_strides)
    elif gate is not None:
        if gate.shape != (BW, T, H * D) or gate.dtype != torch.bfloat16:
            raise ValueError("gate must be bf16 [B*W, T, H*D]")
        if gate.stride(-1) != 1 or any(s % 4 for s in gate.stride()[:-1]):
            gate = gate.contiguous()
        g_strides = (gate.stride(0), gate.stride(1), D)
    else:
        g_strides = (0, 0, 0)
    if out is None:
        out = torch.empty(BW, T, H, D, dtype=q.dtype, device=q.device)
    pk_strides = (prefix_k.stride(0), prefix_k.stride(1), prefix_k.stride(2)) if L else (0, 0, 0)
    _lib.call("kad_prefix_attention_decode_ex", _lib.ptr(q), *q.stride()[:3],
              _lib.ptr(prefix_k if L else None), _lib.ptr(prefix_v if L else None), *pk_strides,
              _lib.ptr(suffix_k), *suffix_k.stride()[:3], _lib.ptr(suffix_v),
              *suffix_v.stride()[:3], _lib.ptr(mask), _lib.ptr(gate), *g_strides,
              _lib.ptr(out), *out.stride()[:3], B, beam_width, T, Tk, H, HK, L, D, float(scale),
              _lib.stream_of(q))
    return out


def prefix_attention_general(q, prefix_k, prefix_v, suffix_k, suffix_v, beam_width, prefix_mask,
                             scale, gate=None, out=None, gate_strides=None):
    """The contract of prefix_attention_decode for every shape and dtype the
    specialised kernel does not take (kad_attention_general): any head dim up
    to 256, any suffix length, bf16/fp16/fp32.  Strides are passed through;
    prefix K and V must share theirs (copied otherwise)."""
    BW, T, H, D = q.shape
    Tk = suffix_k.shape[1]
    B, L, HK, _ = prefix_k.shape
    if L and prefix_k.stride() != prefix_v.stride():
        prefix_k, prefix_v = prefix_k.contiguous(), prefix_v.contiguous()
    mask = prefix_mask.contiguous().view(torch.uint8) if prefix_mask is not None else None
    if gate is not None and gate_strides is not None:
        g_strides = tuple(gate_strides)
    elif gate is not None:
        if gate.shape != (BW, T, H * D) or gate.dtype != q.dtype:
            raise ValueError("gate must be [B*W, T, H*D] in the query dtype")
        if gate.stride(-1) != 1:
            gate = gate.contiguous()
        g_strides = (gate.stride(0), gate.stride(1), D)
    else:
        g_strides = (0, 0, 0)
    if out is None:
        out = torch.empty(BW, T, H, D, dtype=q.dtype, device=q.device)
    for t in (q, suffix_k, suffix_v, out) + ((prefix_k,) if L else ()):
        if t.stride(-1) != 1:
            raise ValueError("attention tensors need a contiguous last dimension")
    pk_strides = prefix_k.stride()[:3] if L else (0, 0, 0)
    _lib.call("kad_attention_general", _lib.ptr(q), *q.stride()[:3],
              _lib.ptr(prefix_k if L else None), _lib.ptr(prefix_v if L else None), *pk_strides,
              _lib.ptr(suffix_k), *suffix_k.stride()[:3], _lib.ptr(suffix_v),
              *suffix_v.stride()[:3], _lib.ptr(mask), _lib.ptr(gate), *g_strides,
              _lib.ptr(out), *out.stride()[:3], B, beam_width, T, Tk, H, HK, L, D,
              _lib.dtype_code(q.dtype), float(scale), _lib.stream_of(q))
    return out


def attention_prefill(q, k, v, scale, gate=None, gate_strides=None, out=None):
    """Causal GQA attention.  q [B,L,H,D]-strided; k, v [B,L,HK,D]-strided; optional
    gate with (b, l, h) strides ``gate_strides``.  Returns out [B,L,H,D] bf16."""
    B, L, H, D = q.shape
    HK = k.shape[2]
    if out is None:
        out = torch.empty(B, L, H, D, dtype=q.dtype, device=q.device)
    gs = gate_strides if gate is not None else (0, 0, 0)
    if k.stride() != v.stride():
        raise ValueError("k and v must share strides")
    _lib.call("kad_attention_prefill", _lib.ptr(q), *q.stride()[:3], _lib.ptr(k), _lib.ptr(v),
              *k.stride()[:3], _lib.ptr(gate), *gs, _lib.ptr(out), *out.stride()[:3], B, L, H,
              HK, D, float(scale), _lib.stream_of(q))
    return out
