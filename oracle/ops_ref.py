"""CPU restatement of the GRBeam shared-prefix operators (oracle; tests only).

Reference semantics followed:
  gated_delta        src/kadllm/ops.py:70-163  (torch path :139-163)
  causal_conv1d      src/kadllm/ops.py:166-226 (torch path :215-226)
  prefix_attention   src/kadllm/ops.py:229-341 (torch path :311-341)
  chunked prefill    transformers qwen3_5 torch_chunk_gated_delta_rule
                     (modeling_qwen3_5.py:249-327 of transformers 5.15.0), the
                     third-party routine the reference prefill calls.

The functions take and return torch CPU tensors.  ``compute`` selects the
internal float type (float32 as in the reference, or float64 for brute-force
pins).  Nothing here is optimised; loops mirror the reference's loops.
"""

import math

import torch
from torch.nn import functional as F


def _l2_normalise(x, eps=1e-6):
    # ops.py:147-148: x / sqrt(sum(x^2) + eps), in the compute type.
    return x / (x.square().sum(-1, keepdim=True) + eps).sqrt()


def gated_delta(q, k, v, log_decay, beta, shared_state, *, beam_width=1,
                scale=None, return_final_state=False, compute=None):
    """Gated delta recurrence from a request-shared initial state.

    Follows src/kadllm/ops.py:139-163.  Layout: q,k [BW,T,H,K]; v [BW,T,HV,V];
    log_decay, beta [BW,T,HV]; shared_state [B,HV,K,V].  Per request and per
    token: S <- S*exp(g); u = beta*(v - S^T k); S <- S + k u^T; o = S^T q,
    with q and k L2-normalised (eps 1e-6) and q scaled by ``scale``
    (default K**-0.5).  Output has v's dtype.
    """
    BW, T, H, K = q.shape
    HV, V = v.shape[-2:]
    B = shared_state.shape[0]
    W = beam_width
    assert BW == B * W and HV % H == 0
    scale = K ** -0.5 if scale is None else scale
    if compute is None:
        compute = torch.float64 if q.dtype == torch.float64 else torch.float32
    group = HV // H
    out = torch.empty(BW, T, HV, V, dtype=compute)
    finals = []
    for r in range(B):
        rows = slice(r * W, (r + 1) * W)
        S = shared_state[r].to(compute).unsqueeze(0).expand(W, HV, K, V).clone()
        qn = _l2_normalise(q[rows].to(compute)) * scale
        kn = _l2_normalise(k[rows].to(compute))
        qn = qn.repeat_interleave(group, dim=2)  # ops.py:149-150 head mapping
        kn = kn.repeat_interleave(group, dim=2)
        for t in range(T):
            decay = log_decay[rows, t].to(compute).exp()          # [W,HV]
            S = S * decay[..., None, None]
            # reductions as broadcast-multiply then sum over K (ops.py:155,158),
            # so bf16 outputs round from the same fp32 sums
            recalled = (S * kn[:, t, :, :, None]).sum(-2)
            u = beta[rows, t].to(compute)[..., None] * (v[rows, t].to(compute) - recalled)
            S = S + kn[:, t, :, :, None] * u[:, :, None, :]
            out[rows, t] = (S * qn[:, t, :, :, None]).sum(-2)
        finals.append(S)
    out = out.to(v.dtype)
    if return_final_state:
        return out, torch.cat(finals)
    return out


def gated_delta_grouped_terminal(q, k, v, log_decay, beta, shared_state, *,
                                 beam_width=1, scale=None):
    """Grouped-kernel semantics with the factored terminal readout.

    Follows src/kadllm/kernels/gated_delta.py:114-142: the last token's output
    is o = (S*e^g)^T q + delta * (k.q) with no final state update.  float64.
    """
    BW, T, H, K = q.shape
    HV, V = v.shape[-2:]
    W = beam_width
    scale = K ** -0.5 if scale is None else scale
    group = HV // H
    out = torch.empty(BW, T, HV, V, dtype=torch.float64)
    for n in range(BW):
        for hv in range(HV):
            h = hv // group
            S = shared_state[n // W, hv].double().clone()
            for t in range(T):
                qt = q[n, t, h].double()
                kt = k[n, t, h].double()
                qt = qt * torch.rsqrt((qt * qt).sum() + 1e-6) * scale
                kt = kt * torch.rsqrt((kt * kt).sum() + 1e-6)
                S = S * math.exp(float(log_decay[n, t, hv]))
                delta = float(beta[n, t, hv]) * (v[n, t, hv].double() - S.T @ kt)
                if t == T - 1:
                    out[n, t, hv] = S.T @ qt + delta * (kt @ qt)
                else:
                    S = S + torch.outer(kt, delta)
                    out[n, t, hv] = S.T @ qt
    return out


def causal_conv1d(x, shared_state, weight, *, beam_width=1, bias=None,
                  activation="silu"):
    """Stateless depthwise causal conv over [prefix taps || suffix].

    Follows src/kadllm/ops.py:215-226: per request, the last width-1 columns of
    shared_state [B,C,history] are prepended to each beam's x [BW,C,T]; a
    grouped conv1d (no padding) gives [BW,C,T]; SiLU is applied to the conv
    output in the tensor's dtype (two roundings for bf16, as torch does).
    """
    BW, C, T = x.shape
    width = weight.shape[-1]
    W = beam_width
    outs = []
    for r in range(BW // W):
        if width > 1:
            taps = shared_state[r:r + 1, :, -(width - 1):]
        else:
            taps = shared_state[r:r + 1, :, :0]
        window = torch.cat((taps.expand(W, -1, -1), x[r * W:(r + 1) * W]), dim=-1)
        y = F.conv1d(window, weight[:, None, :], bias, groups=C)
        outs.append(F.silu(y) if activation == "silu" else y)
    return torch.cat(outs)


def attention_part(scores, values):
    """One attention partition with its log-sum-exp.

    Follows src/kadllm/ops.py:229-240: an empty partition or a fully masked row
    gives a zero output and -inf LSE instead of NaN.
    """
    if scores.shape[-1] == 0:
        return (scores.new_zeros(*scores.shape[:-1], values.shape[-1]),
                scores.new_full(scores.shape[:-1], -torch.inf))
    live = torch.isfinite(scores).any(-1, keepdim=True)
    safe = torch.where(live, scores, torch.zeros_like(scores))
    p = torch.softmax(safe, dim=-1) * live
    lse = torch.where(live.squeeze(-1), safe.logsumexp(-1), -torch.inf)
    return p @ values, lse


def merge_attention(prefix_out, prefix_lse, suffix_out, suffix_lse):
    """LSE merge of two normalised partitions (src/kadllm/ops.py:243-249)."""
    total = torch.logaddexp(prefix_lse, suffix_lse)
    return (prefix_out * (prefix_lse - total).exp()[..., None]
            + suffix_out * (suffix_lse - total).exp()[..., None])


def prefix_attention(q, prefix_k, prefix_v, suffix_k, suffix_v, *, beam_width=1,
                     prefix_mask=None, scale=None, compute=None):
    """Shared-prefix attention plus a causal per-beam suffix, GQA.

    Follows src/kadllm/ops.py:311-341: beams are folded into the query rows of
    the prefix partition, the suffix partition is causal over T, and the two
    are merged by LSE.  Output is q's dtype.
    """
    BW, T, H, D = q.shape
    B, L, HK, _ = prefix_k.shape
    W = beam_width
    group = H // HK
    scale = 1 / math.sqrt(D) if scale is None else scale
    if compute is None:
        compute = torch.float64 if q.dtype == torch.float64 else torch.float32
    qry = q.to(compute).reshape(B, W, T, H, D).permute(0, 1, 3, 2, 4)     # B,W,H,T,D
    pk = prefix_k.to(compute).repeat_interleave(group, 2).permute(0, 2, 1, 3)  # B,H,L,D
    pv = prefix_v.to(compute).repeat_interleave(group, 2).permute(0, 2, 1, 3)
    folded = qry.permute(0, 2, 1, 3, 4).reshape(B, H, W * T, D)
    s_pre = folded @ pk.transpose(-1, -2) * scale
    if prefix_mask is not None:
        s_pre = s_pre.masked_fill(~prefix_mask[:, None, None, :], -torch.inf)
    o_pre, l_pre = attention_part(s_pre, pv)
    o_pre = o_pre.reshape(B, H, W, T, D).permute(0, 2, 1, 3, 4)
    l_pre = l_pre.reshape(B, H, W, T).permute(0, 2, 1, 3)

    def per_beam(x):
        return (x.to(compute).repeat_interleave(group, 2)
                .reshape(B, W, T, H, D).permute(0, 1, 3, 2, 4))

    sk, sv = per_beam(suffix_k), per_beam(suffix_v)
    causal = torch.ones(T, T, dtype=torch.bool).tril()
    s_suf = (qry @ sk.transpose(-1, -2) * scale).masked_fill(~causal, -torch.inf)
    o_suf, l_suf = attention_part(s_suf, sv)
    out = merge_attention(o_pre, l_pre, o_suf, l_suf)
    return out.permute(0, 1, 3, 2, 4).reshape(BW, T, H, D).to(q.dtype)


# ---------------------------------------------------------------------------
# Chunked gated delta rule used by prefill.


def _bf16_like_l2norm(x, eps=1e-6):
    """l2norm evaluated in x's own dtype, as the prefill routine does.

    transformers qwen3_5 l2norm (modeling_qwen3_5.py:242-246): x * rsqrt(sum(x*x)+eps)
    computed in the input dtype (bf16 rounding after each op for bf16 input).
    """
    return x * torch.rsqrt((x * x).sum(dim=-1, keepdim=True) + eps)


def chunk_gated_delta(q, k, v, g, beta, *, chunk_size=64, initial_state=None,
                      use_qk_l2norm=True):
    """Chunked (WY/UT) gated delta rule over full sequences.

    Restates the algorithm of transformers' torch_chunk_gated_delta_rule
    (modeling_qwen3_5.py:249-327), which the reference prefill calls
    (src/kadllm/adapters/qwen3_5.py:111 -> HF Qwen3_5GatedDeltaNet).
    Layout: q,k [B,L,H,K]; v [B,L,H,V]; g,beta [B,L,H] (heads already
    repeated).  Returns (o [B,L,H,V] in q's dtype, final state [B,H,K,V] fp32).

    Per chunk c with cumulative log decays G (within the chunk):
      T = (I + L)^-1 with L[i,j] = beta_i (k_i.k_j) exp(G_i-G_j) for j<i,
      obtained by forward substitution on A = -L;
      U = T (beta v);  Wk = T (beta k exp(G));
      v_new = U - Wk S;  o = (q exp(G)) S + tril(q k^T exp(G_i-G_j)) v_new;
      S <- exp(G_last) S + (k exp(G_last-G))^T v_new.
    """
    out_dtype = q.dtype
    if use_qk_l2norm:
        q = _bf16_like_l2norm(q)
        k = _bf16_like_l2norm(k)
    f32 = torch.float32
    q, k, v, beta, g = (x.transpose(1, 2).contiguous().to(f32) for x in (q, k, v, beta, g))
    B, H, L, K = k.shape
    V = v.shape[-1]
    C = chunk_size
    pad = (-L) % C
    if pad:
        q, k, v = (F.pad(x, (0, 0, 0, pad)) for x in (q, k, v))
        beta, g = (F.pad(x, (0, pad)) for x in (beta, g))
    n_chunks = (L + pad) // C
    q = q * (K ** -0.5)
    S = (torch.zeros(B, H, K, V, dtype=f32) if initial_state is None
         else initial_state.to(f32).clone())
    out = torch.zeros(B, H, L + pad, V, dtype=f32)
    strict_upper_incl = torch.triu(torch.ones(C, C, dtype=torch.bool), 0)
    strict_upper = torch.triu(torch.ones(C, C, dtype=torch.bool), 1)
    for c in range(n_chunks):
        sl = slice(c * C, (c + 1) * C)
        qc, kc, vc = q[:, :, sl], k[:, :, sl], v[:, :, sl]
        bc = beta[:, :, sl]
        G = g[:, :, sl].cumsum(-1)                                   # [B,H,C]
        decay = (G[..., :, None] - G[..., None, :]).tril().exp().tril()
        kb = kc * bc[..., None]
        A = -((kb @ kc.transpose(-1, -2)) * decay).masked_fill(strict_upper_incl, 0)
        # forward substitution, row by row (the routine's 63-step loop)
        for i in range(1, C):
            row = A[..., i, :i].clone()
            A[..., i, :i] = row + (row[..., None] * A[..., :i, :i]).sum(-2)
        Tm = A + torch.eye(C, dtype=f32)
        U = Tm @ (vc * bc[..., None])
        Wk = Tm @ (kb * G.exp()[..., None])
        v_new = U - Wk @ S
        intra = (qc @ kc.transpose(-1, -2) * decay).masked_fill(strict_upper, 0)
        out[:, :, sl] = (qc * G.exp()[..., None]) @ S + intra @ v_new
        tail = (G[..., -1:] - G).exp()                               # [B,H,C]
        S = S * G[..., -1, None, None].exp() + (kc * tail[..., None]).transpose(-1, -2) @ v_new
    out = out[:, :, :L].transpose(1, 2).contiguous().to(out_dtype)
    return out, S


def recurrent_gated_delta_full(q, k, v, g, beta, *, initial_state=None,
                               use_qk_l2norm=True, compute=torch.float32):
    """Token-by-token gated delta over full sequences (W=1 special case).

    Equivalent to transformers' torch_recurrent_gated_delta_rule
    (modeling_qwen3_5.py:331-380) and to src/kadllm/ops.py:152-158 at W=1.
    Layout as chunk_gated_delta.  Returns (o in q's dtype, final state).
    """
    out_dtype = q.dtype
    if use_qk_l2norm:
        q = _bf16_like_l2norm(q)
        k = _bf16_like_l2norm(k)
    q, k, v, beta, g = (x.transpose(1, 2).to(compute) for x in (q, k, v, beta, g))
    B, H, L, K = k.shape
    V = v.shape[-1]
    q = q * (K ** -0.5)
    S = (torch.zeros(B, H, K, V, dtype=compute) if initial_state is None
         else initial_state.to(compute).clone())
    out = torch.empty(B, H, L, V, dtype=compute)
    for t in range(L):
        S = S * g[:, :, t].exp()[..., None, None]
        u = (v[:, :, t] - torch.einsum("bhkv,bhk->bhv", S, k[:, :, t])) * beta[:, :, t, None]
        S = S + k[:, :, t, :, None] * u[:, :, None, :]
        out[:, :, t] = torch.einsum("bhkv,bhk->bhv", S, q[:, :, t])
    return out.transpose(1, 2).contiguous().to(out_dtype), S
