"""Pins for the oracle operators (CPU).

Each oracle function is checked against something independent of its own
formula: transformers' gated-delta routines (the third-party library the
reference prefill calls), torch's conv1d / scaled_dot_product_attention on
the unfactored problem, closed forms, float64 brute force, invariances, and
the golden vectors written by the reference implementation itself.
"""

import pytest
import torch
from torch.nn import functional as F

from _fixtures import bf16_from_bits, conv_inputs, gdn_inputs, load_npz
from conftest import assert_close_rel
from oracle import ops_ref

hf = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")


# --------------------------------------------------------------------------
# gated delta


def test_gated_delta_w1_matches_transformers_recurrent():
    B, L, H, K = 3, 6, 2, 32
    q, k, v, g, beta, S = gdn_inputs(B, 1, L, H, H, K, K, dtype=torch.float32, seed=1,
                                     state_std=0.3)
    ours, ours_state = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=1,
                                           return_final_state=True)
    theirs, their_state = hf.torch_recurrent_gated_delta_rule(
        q, k, v, g=g, beta=beta, initial_state=S, output_final_state=True,
        use_qk_l2norm_in_kernel=True)
    assert_close_rel(ours, theirs, rtol=1e-5, atol_frac=1e-6, name="o")
    assert_close_rel(ours_state, their_state, rtol=1e-5, atol_frac=1e-6, name="state")


def test_gated_delta_beta_zero_closed_form():
    B, W, T, H, K = 2, 3, 3, 2, 16
    q, k, v, g, beta, S = gdn_inputs(B, W, T, H, H, K, K, dtype=torch.float64, seed=2,
                                     state_dtype=torch.float64)
    beta = torch.zeros_like(beta)
    out = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=W)
    qn = q / (q.square().sum(-1, keepdim=True) + 1e-6).sqrt() * K ** -0.5
    gam = g.double().cumsum(1).exp()
    expected = torch.einsum("nhkv,nthk->nthv", S.repeat_interleave(W, 0), qn) * gam[..., None]
    assert torch.allclose(out, expected, rtol=1e-12, atol=1e-14)


def test_gated_delta_delta_rule_overwrite():
    """g=0, beta=1, unit k: after a step the state maps k_t exactly to v_t."""
    B, W, T, H, K = 1, 2, 3, 1, 8
    q, k, v, g, beta, S = gdn_inputs(B, W, T, H, H, K, K, dtype=torch.float64, seed=3,
                                     state_dtype=torch.float64)
    g = torch.zeros_like(g)
    beta = torch.ones_like(beta)
    k = k / k.norm(dim=-1, keepdim=True)
    _, final = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=W, return_final_state=True)
    recalled = torch.einsum("nhkv,nhk->nhv", final, k[:, -1] / (1 + 1e-6) ** 0.5)
    assert torch.allclose(recalled, v[:, -1], atol=1e-5)


def test_gated_delta_terminal_factoring_identity():
    B, W, T, H, HV, K = 2, 3, 3, 1, 2, 16
    q, k, v, g, beta, S = gdn_inputs(B, W, T, H, HV, K, K, dtype=torch.float64, seed=4,
                                     state_dtype=torch.float64)
    a = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=W, compute=torch.float64)
    b = ops_ref.gated_delta_grouped_terminal(q, k, v, g, beta, S, beam_width=W)
    assert torch.allclose(a, b, rtol=1e-10, atol=1e-12)


def test_gated_delta_beam_permutation_and_request_independence():
    B, W, T, H, K = 2, 4, 2, 2, 16
    q, k, v, g, beta, S = gdn_inputs(B, W, T, H, H, K, K, dtype=torch.float64, seed=5,
                                     state_dtype=torch.float64)
    out = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=W)
    perm = torch.tensor([2, 0, 3, 1, 4, 5, 6, 7])
    out_p = ops_ref.gated_delta(q[perm], k[perm], v[perm], g[perm], beta[perm], S, beam_width=W)
    assert torch.allclose(out_p, out[perm])
    S2 = S.clone()
    S2[1] += 1.0
    out2 = ops_ref.gated_delta(q, k, v, g, beta, S2, beam_width=W)
    assert torch.equal(out2[:W], out[:W]) and not torch.allclose(out2[W:], out[W:])


def test_gated_delta_golden_bf16():
    f = load_npz("ops_bf16.npz")
    q, k, v = (bf16_from_bits(f[n]) for n in ("gdn_q", "gdn_k", "gdn_v"))
    out = ops_ref.gated_delta(q, k, v, torch.from_numpy(f["gdn_g"]),
                              bf16_from_bits(f["gdn_beta"]), torch.from_numpy(f["gdn_state"]),
                              beam_width=3)
    assert torch.equal(out, bf16_from_bits(f["gdn_out"]))


# --------------------------------------------------------------------------
# chunked prefill rule


@pytest.mark.parametrize("L", [1, 37, 64, 130])
def test_chunk_rule_matches_transformers_chunk(L):
    B, H, K = 2, 2, 32
    q, k, v, g, beta, _ = gdn_inputs(B, 1, L, H, H, K, K, dtype=torch.float32, seed=L)
    q, k, v = q.reshape(B, L, H, K), k.reshape(B, L, H, K), v.reshape(B, L, H, K)
    g, beta = g.reshape(B, L, H), beta.reshape(B, L, H)
    ours, s1 = ops_ref.chunk_gated_delta(q, k, v, g, beta)
    theirs, s2 = hf.torch_chunk_gated_delta_rule(q, k, v, g=g, beta=beta, output_final_state=True,
                                                 use_qk_l2norm_in_kernel=True)
    assert_close_rel(ours, theirs, rtol=1e-5, atol_frac=1e-6, name="chunk o")
    assert_close_rel(s1, s2, rtol=1e-5, atol_frac=1e-6, name="chunk state")


def test_chunk_rule_equals_recurrence_and_is_chunk_size_invariant():
    B, L, H, K, V = 1, 100, 2, 16, 24
    g0 = torch.Generator().manual_seed(8)
    q, k = torch.randn(B, L, H, K, generator=g0), torch.randn(B, L, H, K, generator=g0)
    v = torch.randn(B, L, H, V, generator=g0)
    g = -F.softplus(torch.randn(B, L, H, generator=g0))
    beta = torch.rand(B, L, H, generator=g0)
    S0 = torch.randn(B, H, K, V, generator=g0) * 0.1
    rec, srec = ops_ref.recurrent_gated_delta_full(q.double(), k.double(), v.double(), g.double(),
                                                   beta.double(), initial_state=S0.double(),
                                                   compute=torch.float64)
    for C in (16, 32, 64):
        o, s = ops_ref.chunk_gated_delta(q, k, v, g, beta, chunk_size=C, initial_state=S0)
        assert_close_rel(o, rec.float(), rtol=1e-4, atol_frac=1e-5, name=f"chunk {C} o")
        assert_close_rel(s, srec.float(), rtol=1e-4, atol_frac=1e-5, name=f"chunk {C} S")


# --------------------------------------------------------------------------
# causal conv1d


def test_conv_equals_full_sequence_conv():
    B, W, C, T = 2, 3, 10, 3
    x, st, w = conv_inputs(B, W, C, T, dtype=torch.float64, history=5)
    out = ops_ref.causal_conv1d(x, st, w, beam_width=W)
    for n in range(B * W):
        seq = torch.cat((st[n // W], x[n]), dim=-1)[None]            # [1,C,5+T]
        full = F.silu(F.conv1d(seq, w[:, None, :], groups=C))        # outputs for t>=3
        assert torch.allclose(out[n], full[0, :, -T:], rtol=1e-12, atol=1e-14)


def test_conv_golden_bf16():
    f = load_npz("ops_bf16.npz")
    x, st, w = (bf16_from_bits(f[n]) for n in ("conv_x", "conv_state", "conv_w"))
    out = ops_ref.causal_conv1d(x, st, w, beam_width=3)
    assert torch.equal(out, bf16_from_bits(f["conv_out"]))


# --------------------------------------------------------------------------
# prefix attention


def _sdpa_reference(q, pk, pv, sk, sv, W, mask=None, scale=None):
    """One softmax over [prefix keys || own causal suffix keys], by torch SDPA."""
    BW, T, H, D = q.shape
    B, L, HK, _ = pk.shape
    rep = H // HK
    out = torch.empty(BW, T, H, D, dtype=torch.float64)
    for n in range(BW):
        b = n // W
        keys = torch.cat((pk[b], sk[n]), 0).double().repeat_interleave(rep, 1)   # [L+T,H,D]
        vals = torch.cat((pv[b], sv[n]), 0).double().repeat_interleave(rep, 1)
        allowed = torch.zeros(T, L + T, dtype=torch.bool)
        allowed[:, :L] = True if mask is None else mask[b]
        allowed[:, L:] = torch.ones(T, T, dtype=torch.bool).tril()
        o = F.scaled_dot_product_attention(q[n].double().transpose(0, 1), keys.transpose(0, 1),
                                           vals.transpose(0, 1), attn_mask=allowed, scale=scale)
        out[n] = o.transpose(0, 1)
    return out


@pytest.mark.parametrize("L", [0, 1, 7])
def test_prefix_attention_equals_single_softmax(L):
    B, W, T, H, HK, D = 2, 3, 3, 4, 2, 16
    g = torch.Generator().manual_seed(L)
    q = torch.randn(B * W, T, H, D, generator=g, dtype=torch.float64)
    pk, pv = (torch.randn(B, L, HK, D, generator=g, dtype=torch.float64) for _ in range(2))
    sk, sv = (torch.randn(B * W, T, HK, D, generator=g, dtype=torch.float64) for _ in range(2))
    out = ops_ref.prefix_attention(q, pk, pv, sk, sv, beam_width=W)
    assert torch.allclose(out, _sdpa_reference(q, pk, pv, sk, sv, W), rtol=1e-10, atol=1e-12)


def test_prefix_attention_masked_rows():
    B, W, T, H, HK, D, L = 2, 2, 2, 2, 1, 8, 4
    g = torch.Generator().manual_seed(3)
    q = torch.randn(B * W, T, H, D, generator=g, dtype=torch.float64)
    pk, pv = (torch.randn(B, L, HK, D, generator=g, dtype=torch.float64) for _ in range(2))
    sk, sv = (torch.randn(B * W, T, HK, D, generator=g, dtype=torch.float64) for _ in range(2))
    mask = torch.tensor([[True, False, True, False], [False, False, False, False]])
    out = ops_ref.prefix_attention(q, pk, pv, sk, sv, beam_width=W, prefix_mask=mask)
    assert torch.allclose(out, _sdpa_reference(q, pk, pv, sk, sv, W, mask), rtol=1e-10,
                          atol=1e-12)


def test_prefix_attention_golden_bf16():
    f = load_npz("ops_bf16.npz")
    q, pk, pv, sk, sv = (bf16_from_bits(f[n]) for n in ("att_q", "att_pk", "att_pv", "att_sk",
                                                         "att_sv"))
    out = ops_ref.prefix_attention(q, pk, pv, sk, sv, beam_width=3)
    assert torch.equal(out, bf16_from_bits(f["att_out"]))
    mask = torch.from_numpy(f["att_mask"])
    outm = ops_ref.prefix_attention(q, pk, pv, sk, sv, beam_width=3, prefix_mask=mask)
    assert torch.equal(outm, bf16_from_bits(f["att_out_masked"]))
