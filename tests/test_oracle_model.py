"""CPU pins of the model and search oracle (no GPU).

The oracle's Qwen3.5 layer math is pinned against the transformers modules
the reference adapter runs (src/kadllm/adapters/qwen3_5.py:50-53,111), the
suffix replay against a full forward (the stateless-decode invariant,
README.md:250-252), the search against exhaustive enumeration and against
golden vectors written by the reference ``grbeam_search`` +
``Qwen35GRBeamAdapter`` (tests/golden/make_fixtures.py).
"""

import numpy as np
import pytest
import torch

from _fixtures import load_npz
from kadllm_amd.config import tiny_hybrid_config
from kadllm_amd.weights import build_hf_text_model, random_state_dict
from oracle import grbeam_ref
from oracle.qwen35_ref import Qwen35Oracle


@pytest.fixture(scope="module")
def tiny_fp32():
    cfg = tiny_hybrid_config()
    sd = random_state_dict(cfg, seed=0, dtype=torch.float32)
    return cfg, sd, Qwen35Oracle(cfg, sd)


class _OracleAdapter:
    def __init__(self, oracle):
        self.oracle = oracle

    def prefill(self, ids):
        return self.oracle.prefill(ids)

    def decode(self, history, state):
        return self.oracle.decode(history, state)


def test_oracle_forward_matches_transformers(tiny_fp32):
    """Logits and every per-layer prefix tensor against Qwen3_5TextModel (fp32)."""
    cfg, sd, orc = tiny_fp32
    model, head = build_hf_text_model(cfg, sd)
    ids = torch.randint(0, cfg.vocab_size, (2, 70), generator=torch.Generator().manual_seed(0))
    with torch.no_grad():
        out = model(input_ids=ids, use_cache=True, return_dict=True)
        expected = head(out.last_hidden_state)
        logits = orc.full_logits(ids)
        _, snap = orc.forward(ids)
    scale = expected.abs().max().item()
    assert (logits - expected).abs().max().item() <= 1e-5 * scale
    for i, (kind, layer) in enumerate(zip(cfg.layer_types, out.past_key_values.layers)):
        if kind == "linear_attention":
            conv = layer.conv_states[0] if isinstance(layer.conv_states, dict) else layer.conv_states
            rec = (layer.recurrent_states[0] if isinstance(layer.recurrent_states, dict)
                   else layer.recurrent_states)
            assert torch.allclose(snap[i][0], conv, rtol=0, atol=1e-5), f"layer {i} conv state"
            assert rec.dtype == torch.float32
            assert torch.allclose(snap[i][1], rec, rtol=1e-4, atol=1e-5), f"layer {i} S"
        else:
            assert torch.allclose(snap[i][0], layer.keys.transpose(1, 2), atol=1e-5), f"layer {i} K"
            assert torch.allclose(snap[i][1], layer.values.transpose(1, 2), atol=1e-5), f"layer {i} V"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_oracle_decode_equals_full_forward(dtype):
    """decode(history)[b, w] is the last-token logits of a forward over prefix + suffix."""
    cfg = tiny_hybrid_config()
    sd = random_state_dict(cfg, seed=1, dtype=dtype)
    orc = Qwen35Oracle(cfg, sd)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, cfg.vocab_size, (2, 40), generator=g)
    hist = torch.randint(0, cfg.vocab_size, (2, 3, 3), generator=g)
    with torch.no_grad():
        _, state = orc.prefill(ids)
        dec = orc.decode(hist, state).float()
        for b in range(2):
            for w in range(3):
                full = orc.full_logits(torch.cat([ids[b], hist[b, w]])[None])[0, -1].float()
                tol = 1e-4 if dtype == torch.float32 else 0.1
                err = (full - dec[b, w]).abs().max().item()
                assert err <= tol * full.abs().max().item(), (b, w, err)


def test_oracle_bf16_is_bit_exact_to_reference_bf16_run():
    """The reference's grbeam_search + Qwen35GRBeamAdapter on the tiny model in
    bf16 (tests/golden/grbeam_tiny_bf16.npz: the transformers bf16 prefill
    loaded as from_pretrained(dtype=bf16) leaves it, and the reference's own
    bf16 decode): prefill logits, every prefix tensor, both decode levels'
    logits, tokens and scores, bit for bit.  This pins the oracle's bf16
    rounding points (RMSNorm cast, RMSNormGated order, RoPE cos/sin cast,
    the conv's rounding before SiLU, the fp32 state, SDPA) at model level."""
    from _fixtures import bf16_from_bits
    f = load_npz("grbeam_tiny_bf16.npz")
    cfg = tiny_hybrid_config()
    orc = Qwen35Oracle(cfg, random_state_dict(cfg, seed=0, dtype=torch.bfloat16))

    def t(name):
        a = f[name]
        return bf16_from_bits(a) if a.dtype == np.uint16 else torch.from_numpy(a)

    ids = t("input_ids")
    with torch.no_grad():
        logits, state = orc.prefill(ids)
        assert torch.equal(logits, t("prefill_logits"))
        for i, (a, b) in enumerate(state.layers):
            assert torch.equal(a, t(f"prefix{i}_a")), f"prefix {i} a"
            assert torch.equal(b, t(f"prefix{i}_b")), f"prefix {i} b"
        for step in (1, 2):
            assert torch.equal(orc.decode(t(f"decode{step}_history"), state),
                               t(f"decode{step}_logits")), f"decode {step}"
        tokens, scores, valid, _ = grbeam_ref.grbeam_search(_OracleAdapter(orc), ids,
                                                            [int(w) for w in f["widths"]])
    assert torch.equal(tokens, t("tokens"))
    assert torch.equal(scores, t("scores"))
    assert torch.equal(valid, t("valid"))


def test_oracle_reproduces_reference_search():
    """Tokens, scores, prefill/decode logits and prefix tensors of the reference
    search on the tiny fp32 model (config 1 of the workload family)."""
    f = load_npz("grbeam_tiny_fp32.npz")
    cfg = tiny_hybrid_config()
    sd = random_state_dict(cfg, seed=0, dtype=torch.float32)
    orc = Qwen35Oracle(cfg, sd)
    ids = torch.from_numpy(f["input_ids"])
    with torch.no_grad():
        _, state = orc.prefill(ids)
        tokens, scores, valid, seen = grbeam_ref.grbeam_search(
            _OracleAdapter(orc), ids, [int(w) for w in f["widths"]])
    assert np.array_equal(tokens.numpy(), f["tokens"])
    assert np.array_equal(valid.numpy(), f["valid"])
    assert np.abs(scores.numpy() - f["scores"]).max() <= 1e-5
    assert np.abs(seen[0][:, 0].numpy() - f["prefill_logits"]).max() <= 1e-4
    assert np.abs(seen[1].numpy() - f["decode1_logits"]).max() <= 1e-4
    assert np.abs(seen[2].numpy() - f["decode2_logits"]).max() <= 1e-4
    for i, (a, b) in enumerate(state.layers):
        assert np.abs(a.numpy() - f[f"prefix{i}_a"]).max() <= 1e-5, f"prefix {i} a"
        assert np.abs(b.numpy() - f[f"prefix{i}_b"]).max() <= 1e-5, f"prefix {i} b"


class _TableModel:
    """A deterministic toy language model: next-token logits depend on the request,
    the depth and the previous token, with no ties between candidates."""

    def __init__(self, B, V, depth, seed):
        g = torch.Generator().manual_seed(seed)
        self.V = V
        self.first = torch.randn(B, V, generator=g, dtype=torch.float64)
        self.table = torch.randn(depth, B, V, V, generator=g, dtype=torch.float64)

    def logits(self, r, seq):
        if not seq:
            return self.first[r]
        return self.table[len(seq) - 1, r, seq[-1]] + 0.01 * len(seq) * self.first[r]

    def logprob(self, r, seq):
        return self.logits(r, seq).log_softmax(-1)

    # adapter protocol
    def prefill(self, ids):
        B = ids.shape[0]
        return torch.stack([self.first[r] for r in range(B)]).float(), None

    def decode(self, history, state):
        B, W, _ = history.shape
        return torch.stack([torch.stack([self.logits(r, tuple(history[r, w].tolist()))
                                         for w in range(W)]) for r in range(B)]).float()


@pytest.mark.parametrize("widths", [[2, 3, 4], [5, 7, 3, 6]])
def test_search_equals_exhaustive_beam_search(widths):
    """The README shape (V=32, widths [2, 3, 4]) and a deeper schedule: tokens and
    cumulative full-vocabulary log-probabilities of the definition of beam search."""
    B, V = 2, 32
    lm = _TableModel(B, V, len(widths), seed=len(widths))
    ids = torch.zeros(B, 5, dtype=torch.int64)
    tokens, scores, valid, _ = grbeam_ref.grbeam_search(lm, ids, widths)
    assert tokens.shape == (B, widths[-1], len(widths)) and valid.all()
    brute = grbeam_ref.brute_force_beam(lm.logprob, B, V, widths)
    for r in range(B):
        assert [tuple(s) for s in tokens[r].tolist()] == [s for s, _ in brute[r]]
        assert np.allclose(scores[r].double().numpy(), [sc for _, sc in brute[r]], atol=1e-5)
        # scores are the cumulative log-probs of the emitted sequences
        for w, seq in enumerate(tokens[r].tolist()):
            cum = sum(float(lm.logprob(r, tuple(seq[:d]))[seq[d]]) for d in range(len(seq)))
            assert abs(cum - float(scores[r, w])) <= 1e-5


def test_search_with_constraint_mask():
    """A Constraint masks candidates without renormalising (src/kadllm/grbeam.py:41-42,80-84):
    masked slots never appear, and scores stay full-vocabulary log-probs."""
    B, V, widths = 1, 16, [3, 4]
    lm = _TableModel(B, V, 2, seed=7)
    allowed_tokens = torch.zeros(V, dtype=torch.bool)
    allowed_tokens[::3] = True

    def allowed(history, logits):
        return allowed_tokens.expand_as(logits)

    tokens, scores, valid, _ = grbeam_ref.grbeam_search(lm, torch.zeros(B, 2, dtype=torch.int64),
                                                         widths, allowed=allowed)
    assert valid.all() and bool((tokens % 3 == 0).all())
    for w, seq in enumerate(tokens[0].tolist()):
        cum = sum(float(lm.logprob(0, tuple(seq[:d]))[seq[d]]) for d in range(len(seq)))
        assert abs(cum - float(scores[0, w])) <= 1e-5


def test_search_rejects_width_beyond_candidates():
    lm = _TableModel(1, 4, 2, seed=0)
    with pytest.raises(ValueError):
        grbeam_ref.grbeam_search(lm, torch.zeros(1, 2, dtype=torch.int64), [4, 17])


def test_select_topk_ties_to_lower_index():
    x = torch.tensor([0.0, 1.0, 1.0, -1.0, 1.0, 0.5])
    s, i = grbeam_ref.select_topk(x, 4)
    assert i.tolist() == [1, 2, 4, 5] and s.tolist() == [1.0, 1.0, 1.0, 0.5]
    big = torch.zeros(5000)
    big[4999] = big[17] = 2.0
    s, i = grbeam_ref.select_topk(big, 3)
    assert i.tolist() == [17, 4999, 0]


@pytest.mark.parametrize("masked", [False, True])
def test_conditional_search_equals_exhaustive(masked):
    """Coarse levels, then per-coarse-beam quotas, against enumeration; with a
    fixed allowed-token subset on the fine levels (a broadcast [V] row)."""
    B, V, coarse, fine = 2, 12, [3, 4], [2, 3]
    lm = _TableModel(B, V, len(coarse) + len(fine), seed=11 + masked)
    sub = torch.zeros(V, dtype=torch.bool)
    sub[torch.randperm(V, generator=torch.Generator().manual_seed(3))[:5]] = True

    def allowed(history, logits):
        if not masked or history.shape[2] < len(coarse):
            return torch.ones(V, dtype=torch.bool)
        return sub

    def allowed_fn(r, seq):
        return sub if masked and len(seq) >= len(coarse) else None

    tokens, scores, valid, _ = grbeam_ref.conditional_search(
        lm, torch.zeros(B, 3, dtype=torch.int64), coarse, fine, allowed=allowed)
    assert tokens.shape == (B, coarse[-1] * fine[-1], len(coarse) + len(fine))
    brute = grbeam_ref.brute_force_conditional(lm.logprob, B, V, coarse, fine, allowed_fn)
    for r in range(B):
        assert [tuple(s) for s in tokens[r].tolist()] == [s for s, _ in brute[r]]
        assert np.allclose(scores[r].double().numpy(), [sc for _, sc in brute[r]], atol=1e-5)
        # every coarse beam keeps exactly fine[-1] descendants, grouped in order
        prefixes = [tuple(s[:len(coarse)]) for s in tokens[r].tolist()]
        groups = [prefixes[i:i + fine[-1]] for i in range(0, len(prefixes), fine[-1])]
        assert all(len(set(g)) == 1 for g in groups) and len({g[0] for g in groups}) == coarse[-1]
    if masked:
        assert bool(torch.isin(tokens[:, :, len(coarse):], torch.nonzero(sub)[:, 0]).all())
