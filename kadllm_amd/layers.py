"""Thin host wrappers of the HIP layer kernels (GEMM, norms, gates, RoPE, gathers).

Every function enqueues one kernel on torch's current stream for the
tensors' device and returns without synchronising.  Shapes and strides are
checked by the C ABI, which raises KadLibraryError on a violation.
"""

import torch

from . import _lib

EPI_STORE, EPI_RESIDUAL, EPI_SWIGLU = 0, 1, 2

def gemm(a, w, out=None, *, epilogue=EPI_STORE, residual=None):
    """out[M, N'] = epilogue(a[M, K] @ w[N, K]^T) (bf16, fp32 accumulate).

    a, w, out may be row-strided 2-D views (last dim contiguous).  For the
    SwiGLU epilogue N' = N/2; for the residual epilogue ``residual`` [M, N]
    is added (it may be ``out`` itself).
    """
    M, K = a.shape
    N = w.shape[0]
    n_out = N // 2 if epilogue == EPI_SWIGLU else N
    if out is None:
        out = torch.empty(M, n_out, dtype=torch.bfloat16, device=a.device)
    r = residual
    _lib.call("kad_gemm_bf16", _lib.ptr(a), a.stride(0), _lib.ptr(w), w.stride(0), _lib.ptr(out),
              out.stride(0), _lib.ptr(r), r.stride(0) if r is not None else 0, M, N, K, epilogue,
              _lib.stream_of(a))
    return out


def rmsnorm(x, w, eps, out=None, *, w_offset=1.0):
    """Qwen3_5RMSNorm over the last dim of a 2-D (row-strided) x."""
    rows, D = x.shape
    if out is None:
        out = torch.empty(rows, D, dtype=x.dtype, device=x.device)
    _lib.call("kad_rmsnorm", _lib.ptr(x), x.stride(0), _lib.ptr(w), float(w_offset),
              _lib.ptr(out), out.stride(0), rows, D, float(eps), _lib.stream_of(x))
    return out


def rmsnorm_gated(x, z, w, eps, heads, out=None):
    """Qwen3_5RMSNormGated per head: x, z are [rows, heads*D] row-strided views."""
    rows = x.shape[0]
    D = w.shape[0]
    if out is None:
        out = torch.empty(rows, heads * D, dtype=x.dtype, device=x.device)
    _lib.call("kad_rmsnorm_gated", _lib.ptr(x), x.stride(0), _lib.ptr(z), z.stride(0),
              _lib.ptr(w), _lib.ptr(out), out.stride(0), rows, heads, D, float(eps),
              _lib.stream_of(x))
    return out


def gdn_gates(a, b, A_log, dt_bias, g_out=None, beta_out=None):
    """g = -exp(A_log) softplus(a + dt_bias) fp32; beta = sigmoid(b) bf16; a, b [rows, HV]."""
    rows, HV = a.shape
    if g_out is None:
        g_out = torch.empty(rows, HV, dtype=torch.float32, device=a.device)
    if beta_out is None:
        beta_out = torch.empty(rows, HV, dtype=torch.bfloat16, device=a.device)
    _lib.call("kad_gdn_gates", _lib.ptr(a), a.stride(0), _lib.ptr(b), b.stride(0), _lib.ptr(A_log),
              _lib.ptr(dt_bias), _lib.ptr(g_out), _lib.ptr(beta_out), rows, HV, _lib.stream_of(a))
    return g_out, beta_out


def qk_norm_rope(src, ld_src, head_stride, heads, w, dst, dst_strides, period, rows, D, rot,
                 inv_freq, pos0, pos_period, eps, do_norm=True):
    """Per-head RMSNorm(1+w) + partial RoPE from a strided source into a strided destination.

    Token r reads src[r*ld_src + head*head_stride : +D] and writes
    dst[(r // period)*s_b + (r % period)*s_t + head*s_h : +D] with
    (s_b, s_t, s_h) = dst_strides; its position is pos0 + r % pos_period.
    """
    s_b, s_t, s_h = dst_strides
    _lib.call("kad_qk_norm_rope", _lib.ptr(src), ld_src, head_stride, heads, _lib.ptr(w),
              _lib.ptr(dst), period, s_b, s_t, s_h, rows, D, rot, _lib.ptr(inv_freq), pos0,
              pos_period, float(eps), int(do_norm), _lib.stream_of(src))


def scatter_heads(src, ld_src, heads, D, dst, dst_strides, period, rows):
    s_b, s_t, s_h = dst_strides
    _lib.call("kad_scatter_heads", _lib.ptr(src), ld_src, heads, D, _lib.ptr(dst), period, s_b, s_t,
              s_h, rows, _lib.stream_of(src))


def embedding(ids, table, out=None):
    """out[r] = table[ids[r]]; ids int64 (any shape, flattened)."""
    ids = ids.reshape(-1)
    if ids.dtype != torch.int64:
        ids = ids.to(torch.int64)
    ids = ids.contiguous()
    rows = ids.numel()
    D = table.shape[1]
    if out is None:
        out = torch.empty(rows, D, dtype=table.dtype, device=table.device)
    _lib.call("kad_embedding", _lib.ptr(ids), _lib.ptr(table), _lib.ptr(out), rows, D,
              table.shape[0], _lib.stream_of(table))
    return out


def cache_prefetch(t0, t1=None):
    """Read one or two (contiguous) tensors into the last-level cache ahead of
    the kernels that use them; computes nothing."""
    b1 = t1.numel() * t1.element_size() if t1 is not None else 0
    _lib.call("kad_cache_prefetch", _lib.ptr(t0), t0.numel() * t0.element_size(),
              _lib.ptr(t1) if t1 is not None else None, b1, _lib.stream_of(t0))
