"""Write golden vectors from the reference GRBeam implementation.

Run in the development container only (it reads the reference sources at
/root/reference/src, which do not exist where the tests run):

    PYTHONPATH=/root/repo python tests/golden/make_fixtures.py

It writes, next to this script:

grbeam_tiny_fp32.npz
    The reference ``grbeam_search`` + ``Qwen35GRBeamAdapter`` (torch
    backends) on the tiny 4-layer hybrid model [GDN x3, attention], hidden
    256, vocabulary 4096, fp32, weights from
    ``kadllm_amd.weights.random_state_dict(cfg, seed=0, dtype=float32)``,
    batch 1, prompt of 128 ids drawn with torch.Generator seed 0, widths
    [8, 8, 8].  Stores the prompt, prefill logits, every decode call's
    history and logits, the prefix tensors, final tokens and scores.

grbeam_tiny_bf16.npz
    The same run with the model in bf16 (bf16 arrays as uint16 bits): the
    reference's bf16 rounding, in its transformers prefill and its own decode.

reference_lm_fp32.npz
    The reference's own toy adapter ``ReferenceHybridLM`` (torch backends,
    fp32): for each case, the state dict after ``torch.manual_seed(seed)``
    construction, the prompt, prefill logits, every decode call's history
    and logits, and the final tokens, scores and valid flags.  Case 0 is the
    README example (vocabulary 32, prompts [2, 5], widths [2, 3, 4]); case 1
    a wider model (vocabulary 64, hidden 32, 4 heads) over 6 levels.

ops_bf16.npz
    Bit-level outputs of the reference torch operators in bf16 on small
    seeded inputs (gated_delta, causal_conv1d, prefix_attention), pinning
    where the reference rounds.  bf16 arrays are stored as their uint16 bit
    patterns.

The reference code itself is not copied; only its outputs are stored.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE_SRC = "/root/reference/src"


def _bits(t):
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return t.detach().contiguous().numpy()


def make_grbeam_tiny_bf16():
    make_grbeam_tiny(torch.bfloat16, "grbeam_tiny_bf16.npz")


def make_grbeam_tiny(dtype=torch.float32, name="grbeam_tiny_fp32.npz"):
    from kadllm import grbeam_search
    from kadllm.adapters import Qwen35GRBeamAdapter

    from kadllm_amd.config import tiny_hybrid_config
    from kadllm_amd.weights import build_hf_text_model, random_state_dict

    cfg = tiny_hybrid_config()
    sd = random_state_dict(cfg, seed=0, dtype=dtype)
    model, head = build_hf_text_model(cfg, sd)
    adapter = Qwen35GRBeamAdapter(model, head)
    gen = torch.Generator().manual_seed(0)
    ids = torch.randint(0, cfg.vocab_size, (1, 128), generator=gen)

    calls = []
    decode = adapter.decode

    def recording_decode(history, state):
        logits = decode(history, state)
        calls.append((history.clone(), logits.clone()))
        return logits

    adapter.decode = recording_decode
    prefill = adapter.prefill
    captured = {}

    def recording_prefill(input_ids):
        out = prefill(input_ids)
        captured["logits"] = out.logits.clone()
        captured["state"] = out.state
        return out

    adapter.prefill = recording_prefill
    result = grbeam_search(adapter, ids, [8, 8, 8])
    arrays = {
        "input_ids": ids.numpy(),
        "widths": np.array([8, 8, 8]),
        "prefill_logits": _bits(captured["logits"]),
        "tokens": result.tokens.numpy(),
        "scores": _bits(result.scores),
        "valid": result.valid.numpy(),
    }
    for step, (hist, logits) in enumerate(calls, start=1):
        arrays[f"decode{step}_history"] = hist.numpy()
        arrays[f"decode{step}_logits"] = _bits(logits)
    for i, (a, b) in enumerate(captured["state"].layers):
        arrays[f"prefix{i}_a"] = _bits(a)
        arrays[f"prefix{i}_b"] = _bits(b)
    np.savez_compressed(os.path.join(HERE, name), **arrays)
    print(name, "tokens", result.tokens.tolist())


def make_reference_lm():
    from kadllm import grbeam_search
    from kadllm.adapters import ReferenceHybridLM

    cases = [dict(seed=0, vocab=32, hidden=16, heads=2, batch=2, prompt=5, widths=[2, 3, 4]),
             dict(seed=1, vocab=64, hidden=32, heads=4, batch=3, prompt=9,
                  widths=[4, 6, 5, 8, 3, 7])]
    arrays = {}
    for ci, c in enumerate(cases):
        torch.manual_seed(c["seed"])
        model = ReferenceHybridLM(vocab_size=c["vocab"], hidden_size=c["hidden"],
                                  num_heads=c["heads"]).eval()
        gen = torch.Generator().manual_seed(c["seed"])
        ids = torch.randint(0, c["vocab"], (c["batch"], c["prompt"]), generator=gen)
        calls = []
        decode, prefill = model.decode, model.prefill
        captured = {}

        def recording_decode(history, state, decode=decode, calls=calls):
            logits = decode(history, state)
            calls.append((history.clone(), logits.clone()))
            return logits

        def recording_prefill(input_ids, prefill=prefill, captured=captured):
            out = prefill(input_ids)
            captured["logits"] = out.logits.clone()
            return out

        model.decode, model.prefill = recording_decode, recording_prefill
        result = grbeam_search(model, ids, c["widths"])
        p = f"c{ci}_"
        arrays[p + "config"] = np.array([c["vocab"], c["hidden"], c["heads"]])
        arrays[p + "widths"] = np.array(c["widths"])
        arrays[p + "input_ids"] = ids.numpy()
        arrays[p + "prefill_logits"] = _bits(captured["logits"])
        arrays[p + "tokens"] = result.tokens.numpy()
        arrays[p + "scores"] = _bits(result.scores)
        arrays[p + "valid"] = result.valid.numpy()
        for step, (hist, logits) in enumerate(calls, start=1):
            arrays[p + f"decode{step}_history"] = hist.numpy()
            arrays[p + f"decode{step}_logits"] = _bits(logits)
        for name, t in model.state_dict().items():
            arrays[p + "w:" + name] = _bits(t)
        print(f"reference_lm case {ci}: tokens shape", tuple(result.tokens.shape))
    np.savez_compressed(os.path.join(HERE, "reference_lm_fp32.npz"), **arrays)


def make_ops_bf16():
    from kadllm.ops import causal_conv1d, gated_delta, prefix_attention

    gen = torch.Generator().manual_seed(1234)
    bf = torch.bfloat16

    def rn(*shape, std=1.0, dtype=bf):
        return (torch.randn(shape, generator=gen) * std).to(dtype)

    arrays = {}
    # gated delta: B=2 requests, W=3 beams, T=3, H=2 qk heads, HV=4 value heads, K=V=64
    B, W, T, H, HV, K, V = 2, 3, 3, 2, 4, 64, 64
    q, k, v = rn(B * W, T, H, K), rn(B * W, T, H, K), rn(B * W, T, HV, V)
    g = -torch.nn.functional.softplus(torch.randn(B * W, T, HV, generator=gen))
    beta = torch.sigmoid(torch.randn(B * W, T, HV, generator=gen)).to(bf)
    S = rn(B, HV, K, V, std=0.1, dtype=torch.float32)
    o = gated_delta(q, k, v, g, beta, S, beam_width=W, backend="torch")
    for name, t in dict(gdn_q=q, gdn_k=k, gdn_v=v, gdn_g=g, gdn_beta=beta, gdn_state=S,
                        gdn_out=o).items():
        arrays[name] = _bits(t)
    # causal conv: B=2, W=3, C=24, T=3, history 4
    C = 24
    x = rn(B * W, C, T)
    st = rn(B, C, 4)
    w = rn(C, 4, std=0.5)
    y = causal_conv1d(x, st, w, beam_width=W, backend="torch")
    for name, t in dict(conv_x=x, conv_state=st, conv_w=w, conv_out=y).items():
        arrays[name] = _bits(t)
    # prefix attention: B=2, W=3, T=3, H=4, HK=2, L=5, D=64
    H, HK, L, D = 4, 2, 5, 64
    qa = rn(B * W, T, H, D)
    pk, pv = rn(B, L, HK, D), rn(B, L, HK, D)
    sk, sv = rn(B * W, T, HK, D), rn(B * W, T, HK, D)
    mask = torch.ones(B, L, dtype=torch.bool)
    mask[1, 1] = False
    oa = prefix_attention(qa, pk, pv, sk, sv, beam_width=W, backend="torch")
    om = prefix_attention(qa, pk, pv, sk, sv, beam_width=W, prefix_mask=mask, backend="torch")
    for name, t in dict(att_q=qa, att_pk=pk, att_pv=pv, att_sk=sk, att_sv=sv,
                        att_out=oa, att_mask=mask, att_out_masked=om).items():
        arrays[name] = _bits(t) if t.dtype != torch.bool else t.numpy()
    np.savez_compressed(os.path.join(HERE, "ops_bf16.npz"), **arrays)
    print("ops_bf16 written")


if __name__ == "__main__":
    sys.path.insert(0, REFERENCE_SRC)
    torch.set_num_threads(4)
    which = sys.argv[1:] or ["grbeam_tiny", "grbeam_tiny_bf16", "ops_bf16", "reference_lm"]
    with torch.no_grad():
        for name in which:
            globals()["make_" + name]()
