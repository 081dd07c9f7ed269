"""Direct parity at the headline model shape (Qwen3.5-0.8B-shaped: 24 layers,
GDN 16x128, attention 8/2 x 256, vocabulary 248,320, bf16).

The target asks for "logits and states within bf16 tolerance (rel 1e-2, fp32
accumulate)" and "top-k indices and beam SID sequences bit-exact wherever
logit gaps exceed tolerance".  Two yardsticks make that testable:

1. Layer by layer, with identical inputs.  bf16 rounding noise compounds
   over 24 layers -- the bf16 oracle's own logits are ~12% (relative L2) from
   the same arithmetic in fp32 at this depth -- so a whole-model comparison
   cannot test a 1e-2 bound.  Here each layer of the oracle is fed the GPU's
   own input to that layer, and its output is compared with the GPU's: the
   residual stream after every layer, the layer's own update of it, every
   prefix state the prefill leaves (conv state, S, K, V) and the logits of
   the GPU's final hidden state are all within rel 1e-2 of the bf16 oracle.
2. The selection, gap-aware.  The selection kernel is judged on the GPU's own
   logits against fp64 keys with delta = 2e-5 (the fp32 rounding of the
   log-softmax): every candidate more than delta above the W-th best key is
   picked, none more than delta below it is, scores are within delta.  Inside
   that band lie cross-row near-ties that fp32 rounding orders (a few per
   level among 63.6M candidates), where a CPU replay of the selection may
   legitimately differ.  The head and selection together are judged by the
   oracle's head plus an fp64 selection on the GPU's own final hidden state,
   with delta = that head's measured key error: most picks must be decided
   outside the band, and all of those equal.  The model's ranking is judged against the fp32
   oracle the same way, with delta = 4x the bf16 oracle's own largest key
   error on the fp32 top-2W; with random-init weights the logits are nearly
   flat and that band is ~1 nat wide (it holds nearly every pick), so this
   part only rules out gross errors -- the layer-by-layer bound above is
   where the rel 1e-2 tolerance is tested.
"""

import pytest
import torch
from torch.nn import functional as F

from conftest import assert_selection_gap_aware
from kadllm_amd import conditional_search, grbeam_search
from kadllm_amd.adapters import Qwen35GRBeamAdapter, native_model
from kadllm_amd.config import qwen35_08b_config
from kadllm_amd.weights import random_state_dict
from oracle import grbeam_ref
from oracle.qwen35_ref import OraclePrefix, Qwen35Oracle

pytestmark = pytest.mark.gpu

LAYER_REL = 1e-2       # rel L2 of a layer's output given the same input
UPDATE_REL = 1e-2      # rel L2 of a layer's update (output - input)


def rel_l2(a, e):
    a, e = a.detach().float().cpu(), e.detach().float().cpu()
    return ((a - e).norm() / e.norm()).item()


@pytest.fixture(scope="module")
def m08(device):
    cfg = qwen35_08b_config()
    sd = random_state_dict(cfg, seed=0, dtype=torch.bfloat16, device=device)
    adapter = Qwen35GRBeamAdapter(*native_model(cfg, sd))
    cpu = {k: v.cpu() for k, v in sd.items()}
    oracle = Qwen35Oracle(cfg, cpu)
    truth = Qwen35Oracle(cfg, {k: v.float() for k, v in cpu.items()})
    return cfg, adapter, oracle, truth


def _traced(adapter, fn, *args):
    seen = []
    adapter._runner.trace = lambda phase, li, x: seen.append(x.cpu())
    try:
        out = fn(*args)
        torch.cuda.synchronize()
    finally:
        adapter._runner.trace = None
    return out, seen


def _check_layer(name, got, ref, x_in):
    r_out = rel_l2(got, ref)
    r_upd = rel_l2(got.float() - x_in.float(), ref.float() - x_in.float())
    assert r_out <= LAYER_REL, f"{name}: output rel L2 {r_out:.2e}"
    assert r_upd <= UPDATE_REL, f"{name}: update rel L2 {r_upd:.2e}"
    return r_out, r_upd


@pytest.mark.timeout(600)
@pytest.mark.parametrize("B,L", [(2, 96), (1, 1024)])
def test_prefill_layerwise_rel_1e2(device, m08, B, L):
    """Two short prompts (2 chunks of the state recurrence) and the headline
    prompt length (1 x 1024 tokens: 16 chunks, 1,024-key causal attention)."""
    cfg, adapter, oracle, _ = m08
    ids = torch.randint(0, cfg.vocab_size, (B, L), generator=torch.Generator().manual_seed(1))
    res, seen = _traced(adapter, adapter.prefill, ids.to(device))
    nl = cfg.num_hidden_layers
    assert len(seen) == nl
    x_in = F.embedding(ids, oracle.w["embed_tokens.weight"])
    cos, sin = oracle.prompt_rope(B, L, x_in.dtype)
    worst = 0.0
    for li in range(nl):
        ref, snap = oracle.forward_layer(li, x_in, cos, sin)
        got = seen[li]
        if li == nl - 1:   # the pruned last layer: its last position only
            _check_layer(f"prefill layer {li}", got.view(B, -1), ref[:, -1], x_in[:, -1])
        else:
            got = got.view(B, L, -1)
            worst = max(worst, _check_layer(f"prefill layer {li}", got, ref, x_in)[1])
        for name, a, e in zip(("state a", "state b"), res.state.layers[li], snap):
            assert a.shape == e.shape, (li, name, a.shape, e.shape)
            r = rel_l2(a, e)
            assert r <= LAYER_REL, f"prefill layer {li} {name}: rel L2 {r:.2e}"
        x_in = got
    r = rel_l2(res.logits, oracle.head(seen[-1].view(B, -1)))
    assert r <= LAYER_REL, f"prefill logits: rel L2 {r:.2e}"
    print(f"prefill B{B} L{L}: worst layer update rel L2 {worst:.2e}, logits {r:.2e}", flush=True)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("B,L,W", [(2, 80, 16), (1, 1024, 256)])
@pytest.mark.parametrize("T", [1, 3])
def test_decode_layerwise_rel_1e2(device, m08, T, B, L, W):
    """Short prefixes with 16 beams, and the headline per-request shape
    (prefix 1024, 256 beams) with 1- and 3-token suffixes."""
    cfg, adapter, oracle, _ = m08
    g = torch.Generator().manual_seed(10 + T)
    ids = torch.randint(0, cfg.vocab_size, (B, L), generator=g)
    hist = torch.randint(0, cfg.vocab_size, (B, W, T), generator=g)
    pre = adapter.prefill(ids.to(device))
    # the oracle replays against the GPU's own prefix, so only decode is judged
    prefix = OraclePrefix(L, B, tuple((a.cpu(), b.cpu()) for a, b in pre.state.layers))
    logits, seen = _traced(adapter, adapter.decode, hist.to(device), pre.state)
    nl, rows = cfg.num_hidden_layers, B * W
    x_in = F.embedding(hist.reshape(rows, T), oracle.w["embed_tokens.weight"])
    cos, sin = oracle.suffix_rope(rows, L, T, x_in.dtype)
    worst = 0.0
    for li in range(nl):
        ref = oracle.decode_layer(li, x_in, prefix.layers[li], W, cos, sin)
        got = seen[li]
        if li == nl - 1 and T > 1:   # pruned last layer: the last token only
            worst = max(worst, _check_layer(f"decode T={T} layer {li}", got.view(rows, -1),
                                            ref[:, -1], x_in[:, -1])[1])
        else:
            got = got.view(rows, T, -1)
            worst = max(worst, _check_layer(f"decode T={T} layer {li}", got, ref, x_in)[1])
        x_in = got
    last = seen[-1].view(rows, -1) if T > 1 else seen[-1].view(rows, T, -1)[:, -1]
    r = rel_l2(logits.reshape(rows, -1), oracle.head(last))
    assert r <= LAYER_REL, f"decode logits: rel L2 {r:.2e}"
    print(f"decode B{B} L{L} W{W} T={T}: worst layer update rel L2 {worst:.2e}, "
          f"logits {r:.2e}", flush=True)


def _keys(logits, scores):
    """Cumulative candidate scores [B, Wp, V] in float64."""
    return logits.double().log_softmax(-1) + scores.double()[..., None]


@pytest.mark.timeout(600)
def test_headline_selection_gap_aware(device, m08):
    """B1, prefix 512, widths [256, 256, 256] (the headline per-request shape),
    followed level by level along the GPU's own path:
    - the selection kernel against fp64 keys of the GPU's own logits, with
      delta = 2e-5 (fp32 rounding of the log-softmax): bit-exact top-256 outside
      that band (cross-row near-ties inside it are ordered by rounding);
    - the SID clause: the oracle's final norm and LM head applied to the
      GPU's own final hidden state, with an fp64 log-softmax and selection,
      pick exactly what the GPU picks outside delta = that head's measured
      largest key error on its top 4W candidates, and more than half of the
      picks lie outside that band (printed per level);
    - the logits against the fp32 oracle within 1.5x the bf16 oracle's own
      distance (+0.2%), and the selection gap-aware against the fp32 oracle's
      keys with delta = 4x the bf16 oracle's largest key error there;
    - grbeam_search (incremental decode) returns exactly this path."""
    from kadllm_amd.grbeam import extend_history, select_level
    cfg, adapter, oracle, truth = m08
    widths = [256, 256, 256]
    ids = torch.randint(0, cfg.vocab_size, (1, 512), generator=torch.Generator().manual_seed(7))
    result = grbeam_search(adapter, ids.to(device), widths)
    torch.cuda.synchronize()
    b_logits, b_state = oracle.prefill(ids)
    t_logits, t_state = truth.prefill(ids)
    hist_d = torch.empty(1, 1, 0, dtype=torch.int64, device=device)
    s_d = torch.zeros(1, 1, device=device)
    s_bf = torch.zeros(1, 1, dtype=torch.float64)
    s_fp = torch.zeros(1, 1, dtype=torch.float64)
    pre, hidden = _traced(adapter, adapter.prefill, ids.to(device))
    last = hidden[-1].view(1, -1)
    gpu_d, bf_l, fp_l = pre.logits[:, None], b_logits[:, None], t_logits[:, None]
    decided_total = 0
    for step, w in enumerate(widths):
        history = hist_d.cpu()
        if step:
            gpu_d, hidden = _traced(adapter, adapter.decode, hist_d, pre.state)
            Wp, T = history.shape[1], history.shape[2]
            last = hidden[-1].view(Wp, -1) if T > 1 else hidden[-1].view(Wp, T, -1)[:, -1]
            bf_l = oracle.decode(history, b_state)
            fp_l = truth.decode(history, t_state)
        gpu_l = gpu_d.cpu()
        # SID clause: the oracle's head and an fp64 selection applied to the
        # GPU's own final hidden state pick what the GPU picks wherever the
        # keys are apart by more than that head's measured key error
        h_l = oracle.head(last).view(gpu_l.shape)
        k_head = _keys(h_l, s_d.cpu())
        k_gpu = _keys(gpu_l, s_d.cpu())
        cand = torch.topk(k_head.reshape(1, -1), 4 * w).indices
        delta_h = (k_gpu.reshape(1, -1).gather(1, cand)
                   - k_head.reshape(1, -1).gather(1, cand)).abs().max().item()
        delta_h = max(delta_h, 2e-5)
        e_ref, e_gpu = rel_l2(bf_l, fp_l), rel_l2(gpu_l, fp_l)
        assert e_gpu <= 1.5 * e_ref + 2e-3, f"level {step}: GPU {e_gpu:.3e} vs bf16 {e_ref:.3e}"
        s_new, p, t, valid = select_level(gpu_d, s_d, w)
        torch.cuda.synchronize()
        k_own = _keys(gpu_l, s_d.cpu())
        tight = assert_selection_gap_aware(s_new, p, t, k_own, w, 2e-5, name=f"kernel {step}")
        in_band = assert_selection_gap_aware(s_new, p, t, k_head, w, delta_h,
                                             name=f"oracle head {step}")
        decided = w - in_band
        decided_total += decided
        print(f"level {step}: oracle head on the GPU's hidden state: key error {delta_h:.3e}, "
              f"{decided} of {w} picks decided outside the band", flush=True)
        assert decided > w // 2, f"level {step}: only {decided} of {w} picks outside the band"
        k_fp, k_bf = _keys(fp_l, s_fp), _keys(bf_l, s_bf)
        top = torch.topk(k_fp.reshape(1, -1), 2 * w).indices
        noise = (k_bf.reshape(1, -1).gather(1, top) - k_fp.reshape(1, -1).gather(1, top)).abs()
        delta = max(4 * noise.max().item(), 1e-3)
        band = assert_selection_gap_aware(s_new, p, t, k_fp, w, delta, name=f"fp32 {step}")
        print(f"level {step}: logits rel L2 to fp32 GPU {e_gpu:.3e} / bf16 oracle {e_ref:.3e}; "
              f"kernel near-ties {tight}; fp32 band delta {delta:.3e} holds {band} of {w} picks",
              flush=True)
        flat = (p * gpu_l.shape[-1] + t).cpu()
        s_fp = k_fp.reshape(1, -1).gather(1, flat)
        s_bf = k_bf.reshape(1, -1).gather(1, flat)
        s_d = s_new
        hist_d = extend_history(hist_d, p, t)
    torch.cuda.synchronize()
    assert torch.equal(hist_d, result.tokens), "search differs from the level-by-level path"
    assert torch.equal(s_d, result.scores)


@pytest.mark.timeout(600)
def test_conditional_sid_workload_shape(device, m08):
    """The two-level conditional SID workload at its shapes: prefix 4096,
    coarse [32, 32] over the full vocabulary, then 16 children per coarse beam
    for 2 tokens inside a seeded 8192-id subset (1 request of the batch of 8).
    Every level's logits against the oracle (bf16-noise criterion, all beams at
    the coarse levels, 32 sampled beams of 512 at the fine ones) and every
    level's selection equal to the oracle's (grouped) selection on the GPU's
    own logits."""
    cfg, adapter, oracle, truth = m08
    V = cfg.vocab_size
    coarse, fine, n_sub = [32, 32], [16, 16], 8192
    sub = torch.zeros(V, dtype=torch.bool)
    sub[torch.randperm(V, generator=torch.Generator().manual_seed(0))[:n_sub]] = True
    subd, everything = sub.to(device), torch.ones(V, dtype=torch.bool, device=device)

    def allowed(history, logits):
        return subd if history.shape[2] >= len(coarse) else everything

    ids = torch.randint(0, V, (1, 4096), generator=torch.Generator().manual_seed(0))
    res = conditional_search(adapter, ids.to(device), coarse, fine, allowed=allowed)
    torch.cuda.synchronize()
    width = coarse[-1] * fine[-1]
    assert res.tokens.shape == (1, width, 4) and bool(res.valid.all())
    assert bool(sub[res.tokens[:, :, 2:].cpu()].all())
    pre = adapter.prefill(ids.to(device))
    b_logits, b_state = oracle.prefill(ids)
    t_logits, t_state = truth.prefill(ids)
    e_gpu, e_ref = rel_l2(pre.logits, t_logits), rel_l2(b_logits, t_logits)
    assert e_gpu <= 1.5 * e_ref + 2e-3, f"prefill: GPU {e_gpu:.3e} vs bf16 {e_ref:.3e}"
    history = torch.empty(1, 1, 0, dtype=torch.int64)
    scores = torch.zeros(1, 1)
    logits = pre.logits.cpu()[:, None]
    levels = [(w, False) for w in coarse] + [(w, True) for w in fine]
    g = torch.Generator().manual_seed(1)
    for step, (w, is_fine) in enumerate(levels):
        if step:
            logits = adapter.decode(history.to(device), pre.state).cpu()
            Wp = history.shape[1]
            pick = torch.randperm(Wp, generator=g)[:32].sort().values if Wp > 32 else \
                torch.arange(Wp)
            h = history[:, pick]
            e_gpu = rel_l2(logits[:, pick], truth.decode(h, t_state))
            e_ref = rel_l2(oracle.decode(h, b_state), truth.decode(h, t_state))
            assert e_gpu <= 1.5 * e_ref + 2e-3, f"level {step}: GPU {e_gpu:.3e} vs {e_ref:.3e}"
            print(f"conditional level {step}: logits rel L2 to fp32 GPU {e_gpu:.3e} / "
                  f"bf16 oracle {e_ref:.3e} ({len(pick)} beams)", flush=True)
        m = allowed(history, logits).cpu().expand(logits.shape)
        if is_fine:
            scores, parents, tokens = grbeam_ref.level_select_grouped(logits, scores, coarse[-1],
                                                                      w, m)
        else:
            scores, parents, tokens = grbeam_ref.level_select(logits, scores, w, m)
        history = torch.cat((history.gather(1, parents[..., None].expand(1, parents.shape[1], step)),
                             tokens[..., None]), -1)
    assert torch.equal(history, res.tokens.cpu()), "GPU search differs from its teacher-forced path"
    assert torch.allclose(scores, res.scores.cpu(), atol=1e-4)
