"""HIP beam selection, chunked GDN / conv prefill kernels against the oracle."""

import pytest
import torch
from torch.nn import functional as F

from _fixtures import gdn_inputs
from conftest import assert_close_rel
from kadllm_amd import _lib, layers, ops
from kadllm_amd.grbeam import extend_history, select_level
from oracle import grbeam_ref, ops_ref

pytestmark = pytest.mark.gpu


def _check_selection(logits, scores, width, mask=None):
    dev = logits.device
    s, p, t, valid = select_level(logits, scores, width, mask)
    torch.cuda.synchronize()
    rs, rp, rt = grbeam_ref.level_select(logits.cpu(), scores.cpu(),
                                         width, None if mask is None else mask.cpu())
    assert torch.equal(p.cpu(), rp), "parents differ"
    assert torch.equal(t.cpu(), rt), "tokens differ"
    finite = torch.isfinite(rs)
    assert torch.equal(valid.cpu(), finite)
    assert torch.equal(torch.isfinite(s.cpu()), finite)
    # Scores against fp64 log-softmax at the selected (parent, token): torch's
    # fp32 CPU log_softmax itself drifts by ~3e-5 over 248k near-equal terms.
    logp = logits.cpu().double().log_softmax(-1) + scores.cpu().double()[..., None]
    flat = rp.clamp(min=0) * logits.shape[-1] + rt.clamp(min=0)
    s64 = logp.reshape(logp.shape[0], -1).gather(1, flat)
    assert torch.allclose(s.cpu()[finite].double(), s64[finite], rtol=0, atol=1e-5)
    assert torch.allclose(s.cpu()[finite], rs[finite], rtol=0, atol=1e-4)
    return s, p, t


@pytest.mark.parametrize("B,Wp,V,W", [(3, 5, 1000, 7), (2, 1, 4096, 8), (2, 8, 33, 200),
                                      (1, 3, 64, 192), (2, 4, 60000, 300), (2, 3, 60000, 500)])
def test_select_level_matches_oracle(device, B, Wp, V, W):
    g = torch.Generator().manual_seed(V + W)
    logits = torch.randn(B, Wp, V, generator=g).bfloat16()   # bf16 rounding creates ties
    scores = -torch.rand(B, Wp, generator=g) * 3
    _check_selection(logits.to(device), scores.to(device), W)


def test_select_level_exact_ties_lower_index_first(device):
    B, Wp, V, W = 2, 4, 50, 9
    logits = torch.zeros(B, Wp, V, dtype=torch.bfloat16)
    logits[:, :, 7] = 1.0                     # many exact ties at the top
    scores = torch.zeros(B, Wp)
    s, p, t = _check_selection(logits.to(device), scores.to(device), W)
    assert t[0, :4].tolist() == [7, 7, 7, 7] and p[0, :4].tolist() == [0, 1, 2, 3]


def test_select_level_with_mask(device):
    B, Wp, V, W = 2, 3, 300, 20
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(B, Wp, V, generator=g).bfloat16()
    scores = -torch.rand(B, Wp, generator=g)
    mask = torch.rand(B, Wp, V, generator=g) > 0.7
    mask[1] = False
    mask[1, 0, :5] = True                      # request 1: only 5 allowed -> 15 invalid slots
    _check_selection(logits.to(device), scores.to(device), W, mask.to(device))


def test_select_level_full_vocab_shape(device):
    """One decode level at the workload shape: 256 beams x 248320 tokens, 2 requests."""
    B, Wp, V, W = 2, 256, 248320, 256
    gen = torch.Generator(device=device).manual_seed(3)
    logits = (torch.randn(B, Wp, V, generator=gen, device=device) * 2).bfloat16()
    scores = -torch.rand(B, Wp, generator=gen, device=device) * 4
    _check_selection(logits, scores, W)


def test_select_level_unsampled_outlier(device):
    """A logit far above everything the row sample sees (line 1 of the row is
    not sampled): the log-sum-exp is taken again against the true max."""
    B, Wp, V, W = 1, 4, 248320, 64
    gen = torch.Generator(device=device).manual_seed(8)
    logits = torch.randn(B, Wp, V, generator=gen, device=device).bfloat16()
    logits[0, 0, 65] = 90.0
    logits[0, 2, 70] = 75.0
    scores = -torch.rand(B, Wp, generator=gen, device=device)
    _check_selection(logits, scores, W)


def test_history_update(device):
    B, Wp, step, W = 2, 3, 2, 5
    hist = torch.arange(B * Wp * step).reshape(B, Wp, step)
    parents = torch.tensor([[2, 0, 1, 1, 2], [0, 0, 2, 1, 0]])
    tokens = torch.arange(10).reshape(B, W) + 100
    out = extend_history(hist.to(device), parents.to(device), tokens.to(device))
    torch.cuda.synchronize()
    ref = torch.cat((hist.gather(1, parents[..., None].expand(B, W, step)), tokens[..., None]), -1)
    assert torch.equal(out.cpu(), ref)
    out0 = extend_history(torch.empty(B, 1, 0, dtype=torch.int64, device=device),
                          torch.zeros(B, W, dtype=torch.int64, device=device), tokens.to(device))
    torch.cuda.synchronize()
    assert torch.equal(out0.cpu(), tokens[..., None])


# --------------------------------------------------------------------------
# chunked gated delta


@pytest.mark.parametrize("B,W,T,H,HV,K,V", [(2, 3, 9, 2, 4, 64, 64), (1, 2, 70, 4, 4, 128, 128),
                                            (2, 1, 130, 2, 2, 128, 64)])
def test_gdn_long_suffix_uses_chunk_kernel(device, B, W, T, H, HV, K, V):
    q, k, v, g, beta, S = gdn_inputs(B, W, T, H, HV, K, V, seed=T, state_std=0.1)
    expected = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=W)
    out = ops.gated_delta(*(t.to(device) for t in (q, k, v, g, beta, S)), beam_width=W)
    torch.cuda.synchronize()
    assert_close_rel(out.cpu(), expected, rtol=1e-2, atol_frac=3e-3, name="chunk ops path")


def test_gdn_return_final_state(device):
    B, W, T, H, HV, K, V = 2, 2, 5, 2, 2, 64, 128
    q, k, v, g, beta, S = gdn_inputs(B, W, T, H, HV, K, V, seed=2, state_std=0.1)
    eo, es = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=W, return_final_state=True)
    o, s = ops.gated_delta(*(t.to(device) for t in (q, k, v, g, beta, S)), beam_width=W,
                           return_final_state=True)
    torch.cuda.synchronize()
    assert s.shape == (B * W, HV, K, V) and s.dtype == torch.float32
    assert_close_rel(o.cpu(), eo, rtol=1e-2, atol_frac=3e-3, name="o")
    assert_close_rel(s.cpu(), es, rtol=1e-4, atol_frac=1e-5, name="final state")


@pytest.mark.parametrize("L", [37, 64, 200, 1024])
def test_prefill_chunk_matches_transformers_semantics(device, L):
    """Prefill mode (bf16-rounded l2norm) against the oracle restatement of the
    transformers chunk routine, including the final fp32 state."""
    B, H, K = 2, 4, 128
    q, k, v, g, beta, _ = gdn_inputs(B, 1, L, H, H, K, K, seed=L)
    q, k, v = (t.reshape(B, L, H, K) for t in (q, k, v))
    g, beta = g.reshape(B, L, H), beta.reshape(B, L, H)
    eo, es = ops_ref.chunk_gated_delta(q, k, v, g, beta)
    dev = [t.to(device).contiguous() for t in (q, k, v, g, beta)]
    o = torch.empty(B, L, H, K, dtype=torch.bfloat16, device=device)
    s = torch.empty(B, H, K, K, dtype=torch.float32, device=device)
    ws = _lib.gdn_chunk_workspace(B, L, H, K, device)
    _lib.call("kad_gdn_chunk", _lib.ptr(dev[0]), _lib.ptr(dev[1]), _lib.ptr(dev[2]), H * K, H * K,
              0, _lib.ptr(dev[3]), 2, _lib.ptr(dev[4]), 0, H, None, 2, 1, _lib.ptr(o), H * K,
              _lib.ptr(s), _lib.ptr(ws), ws.numel(), B, L, H, H, K, K, float(K ** -0.5), 1,
              _lib.stream_of(o))
    torch.cuda.synchronize()
    assert_close_rel(o.cpu(), eo, rtol=1e-2, atol_frac=3e-3, name="prefill o")
    assert_close_rel(s.cpu(), es, rtol=1e-3, atol_frac=1e-4, name="prefill state")


@pytest.mark.parametrize("L,K", [(37, 128), (200, 128), (100, 64)])
def test_prefill_chunk_gated_equals_chunk_then_norm(device, L, K):
    """kad_gdn_chunk_gated against kad_gdn_chunk followed by kad_rmsnorm_gated,
    bit for bit (output and final state), with a gate row stride wider than
    the value heads and a partial last chunk."""
    B, H = 2, 4
    q, k, v, g, beta, _ = gdn_inputs(B, 1, L, H, H, K, K, seed=300 + L)
    dev = [t.to(device).contiguous() for t in (q, k, v, g, beta)]
    gen = torch.Generator().manual_seed(301 + L)
    zpad = torch.randn(B * L, H * K + 40, generator=gen).bfloat16().to(device)
    z = zpad[:, 8:8 + H * K]
    w = (1.0 + 0.1 * torch.randn(K, generator=gen)).bfloat16().to(device)
    eps = 1e-6
    ws = _lib.gdn_chunk_workspace(B, L, H, K, device)
    args = (_lib.ptr(dev[0]), _lib.ptr(dev[1]), _lib.ptr(dev[2]), H * K, H * K, 0,
            _lib.ptr(dev[3]), 2, _lib.ptr(dev[4]), 0, H, None, 2, 1)
    o = torch.empty(B * L, H * K, dtype=torch.bfloat16, device=device)
    s1 = torch.empty(B, H, K, K, dtype=torch.float32, device=device)
    _lib.call("kad_gdn_chunk", *args, _lib.ptr(o), H * K, _lib.ptr(s1), _lib.ptr(ws), ws.numel(),
              B, L, H, H, K, K, float(K ** -0.5), 1, _lib.stream_of(o))
    y1 = layers.rmsnorm_gated(o, z, w, eps, H)
    y2 = torch.full((B * L, H * K), 7.0, dtype=torch.bfloat16, device=device)
    s2 = torch.empty(B, H, K, K, dtype=torch.float32, device=device)
    _lib.call("kad_gdn_chunk_gated", *args, _lib.ptr(y2), H * K, _lib.ptr(s2), _lib.ptr(ws),
              ws.numel(), B, L, H, H, K, K, float(K ** -0.5), _lib.ptr(z), z.stride(0),
              _lib.ptr(w), eps, _lib.stream_of(o))
    torch.cuda.synchronize()
    assert torch.equal(y2.cpu(), y1.cpu()), "gated chunk output differs from chunk + norm"
    assert torch.equal(s2.cpu(), s1.cpu()), "gated chunk final state differs"


@pytest.mark.parametrize("L", [1, 3, 50])
def test_conv_prefill_and_state(device, L):
    B, C = 2, 64
    g = torch.Generator().manual_seed(L)
    x = torch.randn(B, L, C, generator=g).bfloat16()
    w = (torch.rand(C, 4, generator=g) - 0.5).bfloat16()
    xd = x.to(device).reshape(B * L, C)
    out = torch.empty(B * L, C, dtype=torch.bfloat16, device=device)
    st = torch.empty(B, C, 4, dtype=torch.bfloat16, device=device)
    wd = w.to(device)   # held until the kernel has read it
    _lib.call("kad_causal_conv_prefill", _lib.ptr(xd), C, _lib.ptr(wd), _lib.ptr(out), C,
              _lib.ptr(st), B, L, C, 1, _lib.stream_of(xd))
    torch.cuda.synchronize()
    pre = x.transpose(1, 2)
    ref = F.silu(F.conv1d(pre, w[:, None, :], padding=3, groups=C)[..., :L]).transpose(1, 2)
    a, e = out.cpu().float().reshape(B, L, C), ref.float()
    assert ((a - e).abs() <= e.abs() * 2 ** -7 + 1e-6).all()
    ref_state = F.pad(pre, (max(0, 4 - L), 0))[..., -4:]
    assert torch.equal(st.cpu(), ref_state)


def test_select_level_masked_fast_path(device):
    B, Wp, V, W = 2, 4, 4096, 16
    g = torch.Generator().manual_seed(12)
    logits = torch.randn(B, Wp, V, generator=g).bfloat16()
    scores = -torch.rand(B, Wp, generator=g)
    mask = torch.rand(B, Wp, V, generator=g) > 0.3
    _check_selection(logits.to(device), scores.to(device), W, mask.to(device))


def test_select_level_candidate_overflow_falls_back_exactly(device):
    """Near-constant rows put far more than the candidate capacity at the sampled
    threshold; the exact histogram path must take over with the same answer."""
    B, Wp, V, W = 1, 3, 248320, 64
    g = torch.Generator().manual_seed(13)
    logits = torch.randint(0, 10, (B, Wp, V), generator=g).float() / 10   # 10 levels, huge ties
    logits[0, 1, 12345] = 3.0
    logits = logits.bfloat16()
    scores = -torch.rand(B, Wp, generator=g)
    _check_selection(logits.to(device), scores.to(device), W)


def test_select_level_grouped_with_shared_mask(device):
    """Per-group quotas with one allowed-token row broadcast to every beam row
    (read in place, row stride 0): exactly the oracle's grouped selection."""
    from kadllm_amd.grbeam import select_level_grouped
    B, G, rpg, V, W = 2, 4, 3, 5000, 6
    g = torch.Generator().manual_seed(31)
    logits = torch.randn(B, G * rpg, V, generator=g).bfloat16()
    scores = -torch.rand(B, G * rpg, generator=g) * 2
    sub = torch.zeros(V, dtype=torch.bool)
    sub[torch.randperm(V, generator=g)[:700]] = True
    mask = sub.to(device).expand(B, G * rpg, V)
    s, p, t, valid = select_level_grouped(logits.to(device), scores.to(device), G, W, mask)
    torch.cuda.synchronize()
    rs, rp, rt = grbeam_ref.level_select_grouped(logits, scores, G, W, sub.expand(B, G * rpg, V))
    assert torch.equal(p.cpu(), rp) and torch.equal(t.cpu(), rt)
    assert torch.allclose(s.cpu(), rs, rtol=0, atol=1e-4) and bool(valid.all())
    assert bool(sub[t.cpu()].all()), "a disallowed token was selected"
    # the same mask materialised gives the same answer
    s2, p2, t2, _ = select_level_grouped(logits.to(device), scores.to(device), G, W,
                                         mask.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(p2, p) and torch.equal(t2, t) and torch.equal(s2, s)


def test_conditional_search_teacher_forced(device):
    """Two-level conditional search on the tiny model: coarse [4, 4], fine [3, 2]
    with an allowed-token subset on the fine levels; each level's selection is
    the oracle's (grouped) selection applied to the GPU's own logits."""
    from kadllm_amd import conditional_search
    from kadllm_amd.adapters import Qwen35GRBeamAdapter, native_model
    from kadllm_amd.config import tiny_hybrid_config
    from kadllm_amd.weights import random_state_dict
    cfg = tiny_hybrid_config()
    sd = random_state_dict(cfg, seed=2, dtype=torch.bfloat16, device=device)
    adapter = Qwen35GRBeamAdapter(*native_model(cfg, sd))
    V = cfg.vocab_size
    sub = torch.zeros(V, dtype=torch.bool)
    sub[torch.randperm(V, generator=torch.Generator().manual_seed(4))[:300]] = True
    subd = sub.to(device)
    coarse, fine = [4, 4], [3, 2]

    def allowed(history, logits):
        if history.shape[2] < len(coarse):
            return torch.ones(V, dtype=torch.bool, device=logits.device)
        return subd

    ids = torch.randint(0, V, (2, 40), generator=torch.Generator().manual_seed(5)).to(device)
    res = conditional_search(adapter, ids, coarse, fine, allowed=allowed)
    torch.cuda.synchronize()
    B = 2
    assert res.tokens.shape == (B, coarse[-1] * fine[-1], 4) and bool(res.valid.all())
    assert bool(sub[res.tokens[:, :, 2:].cpu()].all())
    # teacher forcing through the oracle selection rules; every level's logits
    # against the oracle model (GPU error to the fp32 evaluation within 1.5x the
    # bf16 oracle's own, +0.2%)
    from oracle.qwen35_ref import Qwen35Oracle
    cpu_sd = {k: v.cpu() for k, v in sd.items()}
    oracle = Qwen35Oracle(cfg, cpu_sd)
    truth = Qwen35Oracle(cfg, {k: v.float() for k, v in cpu_sd.items()})
    b_logits, b_state = oracle.prefill(ids.cpu())
    t_logits, t_state = truth.prefill(ids.cpu())

    def rel(a, e):
        return ((a.float() - e.float()).norm() / e.float().norm()).item()

    pre = adapter.prefill(ids)
    history = torch.empty(B, 1, 0, dtype=torch.int64)
    scores = torch.zeros(B, 1)
    logits = pre.logits.cpu()[:, None]
    for step, (w, is_fine) in enumerate([(w, False) for w in coarse] + [(w, True) for w in fine]):
        if step:
            logits = adapter.decode(history.to(device), pre.state).cpu()
            ref, exact = oracle.decode(history, b_state), truth.decode(history, t_state)
        else:
            ref, exact = b_logits[:, None], t_logits[:, None]
        assert rel(logits, exact) <= 1.5 * rel(ref, exact) + 2e-3, f"level {step} logits"
        m = allowed(history, logits).cpu().expand(logits.shape)
        if is_fine:
            scores, parents, tokens = grbeam_ref.level_select_grouped(logits, scores, coarse[-1],
                                                                      w, m)
        else:
            scores, parents, tokens = grbeam_ref.level_select(logits, scores, w, m)
        history = torch.cat((history.gather(1, parents[..., None].expand(B, parents.shape[1], step)),
                             tokens[..., None]), -1)
    assert torch.equal(history, res.tokens.cpu())
    assert torch.allclose(scores, res.scores.cpu(), atol=1e-4)
