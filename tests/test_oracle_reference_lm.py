"""The toy-model oracle against the reference's own outputs (CPU).

tests/golden/reference_lm_fp32.npz holds what the reference
``ReferenceHybridLM`` + ``grbeam_search`` (src/kadllm/adapters/reference.py,
src/kadllm/grbeam.py) produced for two seeded models, written by
tests/golden/make_fixtures.py.
"""

import numpy as np
import pytest
import torch

from oracle import grbeam_ref
from oracle.reference_lm_ref import ReferenceLMOracle
from tests._fixtures import load_npz


def reference_lm_case(ci):
    d = load_npz("reference_lm_fp32.npz")
    p = f"c{ci}_"
    vocab, hidden, heads = (int(x) for x in d[p + "config"])
    sd = {k[len(p) + 2:]: torch.from_numpy(np.array(d[k])) for k in d.files
          if k.startswith(p + "w:")}
    calls = []
    step = 1
    while p + f"decode{step}_history" in d.files:
        calls.append((torch.from_numpy(d[p + f"decode{step}_history"]),
                      torch.from_numpy(d[p + f"decode{step}_logits"])))
        step += 1
    return dict(vocab=vocab, hidden=hidden, heads=heads, sd=sd,
                widths=[int(w) for w in d[p + "widths"]],
                ids=torch.from_numpy(d[p + "input_ids"]),
                prefill_logits=torch.from_numpy(d[p + "prefill_logits"]),
                tokens=torch.from_numpy(d[p + "tokens"]),
                scores=torch.from_numpy(d[p + "scores"]),
                valid=torch.from_numpy(d[p + "valid"]), calls=calls)


@pytest.mark.parametrize("ci", [0, 1])
def test_reference_lm_oracle_matches_reference_outputs(ci):
    c = reference_lm_case(ci)
    oracle = ReferenceLMOracle(c["sd"], c["heads"])
    logits, prefix = oracle.prefill(c["ids"])
    torch.testing.assert_close(logits, c["prefill_logits"], atol=1e-5, rtol=1e-5)
    for history, expected in c["calls"]:
        torch.testing.assert_close(oracle.decode(history, prefix), expected, atol=1e-5,
                                   rtol=1e-5)
    tokens, scores, valid, _ = grbeam_ref.grbeam_search(oracle, c["ids"], c["widths"])
    assert torch.equal(tokens, c["tokens"])
    torch.testing.assert_close(scores, c["scores"], atol=1e-5, rtol=1e-5)
    assert torch.equal(valid, c["valid"])


def test_reference_lm_case0_is_the_readme_example():
    c = reference_lm_case(0)
    assert c["widths"] == [2, 3, 4] and tuple(c["ids"].shape) == (2, 5)
    assert tuple(c["tokens"].shape) == (2, 4, 3)  # README.md:265
