"""Host wrappers of the prefill-side HIP kernels (chunked gated delta, conv prefill)."""

import torch

from . import _lib


def gdn_chunk(q, k, v, log_decay, beta, shared_state, *, beam_width=1, scale=None,
              want_final=False, transformers_l2norm=False, out=None):
    """Chunked gated delta over [N, T] sequences (kad_gdn_chunk).

    q, k [N,T,H,K], v [N,T,HV,V] bf16 (contiguous, or row-strided via the
    ``*_ld`` layout of the C ABI through views with contiguous heads);
    log_decay, beta [N,T,HV]; shared_state [N/beam_width,HV,K,V] or None.
    Returns (out [N,T,HV,V] bf16, final fp32 [N,HV,K,V] or None).
    """
    N, T, H, K = q.shape
    HV, V = v.shape[-2:]
    if q.dtype != torch.bfloat16:
        raise RuntimeError("the chunked gated-delta kernel takes bf16 q/k/v")
    scale = K ** -0.5 if scale is None else scale
    if out is None:
        out = torch.empty(N, T, HV, V, dtype=v.dtype, device=v.device)
    final = (torch.empty(N, HV, K, V, dtype=torch.float32, device=v.device)
             if want_final else None)
    st = shared_state
    ws = _lib.gdn_chunk_workspace(N, T, HV, K, v.device)
    _lib.call("kad_gdn_chunk", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), q.stride(1), v.stride(1),
              _lib.dtype_code(q.dtype), _lib.ptr(log_decay), _lib.dtype_code(log_decay.dtype),
              _lib.ptr(beta), _lib.dtype_code(beta.dtype), log_decay.stride(1), _lib.ptr(st),
              _lib.dtype_code(st.dtype) if st is not None else 2, beam_width, _lib.ptr(out),
              out.stride(1), _lib.ptr(final), _lib.ptr(ws), ws.numel(), N, T, H, HV, K, V,
              float(scale), int(transformers_l2norm), _lib.stream_of(v))
    return out, final


def conv_prefill(x, weight, out, state, B, L, C, silu=True):
    """Causal conv4 (+SiLU) over [B*L, C] rows; writes conv state [B, C, 4]."""
    _lib.call("kad_causal_conv_prefill", _lib.ptr(x), x.stride(0), _lib.ptr(weight), _lib.ptr(out),
              out.stride(0), _lib.ptr(state), B, L, C, int(silu), _lib.stream_of(x))
    return out
