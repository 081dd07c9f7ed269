"""fp32 models on the HIP path (kadllm_amd.qwen35_f32): the fp32 MFMA lane
layout, the fp32 GEMM and row-wise kernels against torch / the oracle, and the
reference's own end-to-end output on the CPU-plumbing configuration (tiny
hybrid model, fp32, batch 1, prefix 128, widths [8, 8, 8], seed 0) replayed
through the GPU: tokens exactly, scores, every level's logits and the prefix
within 1e-4 (the reference states < 1.6e-5 for its fp32 fixed-history
comparisons, README.md:152)."""

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from _fixtures import load_npz
from kadllm_amd import _lib, grbeam_search
from kadllm_amd.adapters import Qwen35GRBeamAdapter, native_model
from kadllm_amd.config import tiny_hybrid_config
from kadllm_amd.qwen35_f32 import EPI_RESIDUAL, EPI_SWIGLU, gemm, rmsnorm
from kadllm_amd.weights import random_state_dict
from oracle.qwen35_ref import Qwen35Oracle, rms_norm

pytestmark = pytest.mark.gpu


def test_mfma_f32_lane_layout(device):
    g = torch.Generator().manual_seed(0)
    a = torch.randn(16, 4, generator=g)
    b = torch.randn(4, 16, generator=g)
    c = torch.empty(16, 16, device=device)
    ad, bd = a.to(device), b.to(device)   # held until the kernel has read them
    _lib.call("kad_selftest_mfma_f32", _lib.ptr(ad), _lib.ptr(bd), _lib.ptr(c), _lib.stream_of(c))
    torch.cuda.synchronize()
    torch.testing.assert_close(c.cpu(), (a.double() @ b.double()).float(), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("M,N,K", [(1, 4096, 256), (70, 200, 37), (128, 768, 256), (3, 64, 1000)])
def test_gemm_f32_matches_torch(device, M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.05
    r = torch.randn(M, N, generator=g)
    ad, wd, rd = a.to(device), w.to(device), r.to(device)
    ref = a.double() @ w.double().T
    torch.testing.assert_close(gemm(ad, wd).cpu().double(), ref, atol=1e-4, rtol=1e-5)
    out = rd.clone()
    gemm(ad, wd, out=out, epilogue=EPI_RESIDUAL, residual=out)
    torch.testing.assert_close(out.cpu().double(), ref + r.double(), atol=1e-4, rtol=1e-5)
    if N % 64 == 0:
        blocks = ref.view(M, N // 64, 2, 32)
        expected = F.silu(blocks[:, :, 0]) * blocks[:, :, 1]
        got = gemm(ad, wd, epilogue=EPI_SWIGLU).cpu().double()
        torch.testing.assert_close(got, expected.reshape(M, N // 2), atol=1e-4, rtol=1e-5)


def test_rmsnorm_f32_matches_oracle(device):
    g = torch.Generator().manual_seed(2)
    x = torch.randn(33, 256, generator=g)
    w = torch.randn(256, generator=g) * 0.1
    got = rmsnorm(x.to(device), w.to(device), 1e-6)
    torch.testing.assert_close(got.cpu(), rms_norm(x, w, 1e-6), atol=1e-5, rtol=1e-5)


def _fixture_adapter(device):
    cfg = tiny_hybrid_config()
    sd = random_state_dict(cfg, seed=0, dtype=torch.float32)   # the fixture's weights (CPU draws)
    adapter = Qwen35GRBeamAdapter(*native_model(cfg, {k: v.to(device) for k, v in sd.items()}))
    return cfg, sd, adapter


def test_config1_reference_search_through_hip(device):
    """The reference's grbeam_search + Qwen35GRBeamAdapter output on the fp32
    tiny model (tests/golden/grbeam_tiny_fp32.npz) reproduced on the GPU."""
    d = load_npz("grbeam_tiny_fp32.npz")
    cfg, _, adapter = _fixture_adapter(device)
    assert adapter.decode_incremental is None   # fp32: stateless replay, as the reference
    ids = torch.from_numpy(d["input_ids"]).to(device)
    widths = [int(w) for w in d["widths"]]
    seen = {}
    decode, prefill = adapter.decode, adapter.prefill

    def rec_prefill(x):
        out = prefill(x)
        seen["prefill"] = out
        return out

    calls = []

    def rec_decode(history, state):
        out = decode(history, state)
        calls.append((history.cpu(), out.cpu()))
        return out

    adapter.prefill, adapter.decode = rec_prefill, rec_decode
    result = grbeam_search(adapter, ids, widths)
    torch.cuda.synchronize()
    worst = {}

    def close(name, got, expected, tol=1e-4):
        got, expected = got.detach().float().cpu(), torch.as_tensor(expected).float()
        assert got.shape == expected.shape, (name, got.shape, expected.shape)
        err = (got - expected).abs().max().item()
        worst[name] = err
        assert err <= tol, f"{name}: max abs error {err:.3e}"

    assert torch.equal(result.tokens.cpu(), torch.from_numpy(d["tokens"])), "tokens differ"
    assert torch.equal(result.valid.cpu(), torch.from_numpy(d["valid"]))
    close("scores", result.scores, d["scores"])
    close("prefill logits", seen["prefill"].logits, d["prefill_logits"])
    assert len(calls) == 2
    for step, (history, logits) in enumerate(calls, start=1):
        assert torch.equal(history, torch.from_numpy(d[f"decode{step}_history"]))
        close(f"decode{step} logits", logits, d[f"decode{step}_logits"])
    for i, (a, b) in enumerate(seen["prefill"].state.layers):
        close(f"prefix{i}_a", a, d[f"prefix{i}_a"])
        close(f"prefix{i}_b", b, d[f"prefix{i}_b"])
    print("config 1 max abs errors:", {k: f"{v:.2e}" for k, v in worst.items()}, flush=True)


def test_fp32_decode_matches_oracle_deeper(device):
    """fp32 decode of 5-token suffixes against the fp32 oracle (1e-4)."""
    cfg, sd, adapter = _fixture_adapter(device)
    oracle = Qwen35Oracle(cfg, sd)
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, cfg.vocab_size, (2, 50), generator=g)
    hist = torch.randint(0, cfg.vocab_size, (2, 3, 5), generator=g)
    pre = adapter.prefill(ids.to(device))
    logits = adapter.decode(hist.to(device), pre.state)
    ref_logits, state = oracle.prefill(ids)
    torch.testing.assert_close(pre.logits.cpu(), ref_logits, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(logits.cpu(), oracle.decode(hist, state), atol=1e-4, rtol=1e-4)
    assert np.isfinite(logits.cpu().numpy()).all()


def test_fp16_model_on_the_fp32_kernels(device):
    """An fp16 model (the reference adapter wraps any float dtype,
    src/kadllm/adapters/qwen3_5.py:40-104) runs on the fp32 kernels with its
    weights widened once: prefill and a 3-token decode no farther from the
    fp32 evaluation of the same fp16 weights than the oracle's own fp16
    arithmetic is, and the search equal to the oracle's selection on the GPU's
    own logits, level by level."""
    from oracle import grbeam_ref
    cfg = tiny_hybrid_config()
    sd = random_state_dict(cfg, seed=5, dtype=torch.float16)
    adapter = Qwen35GRBeamAdapter(*native_model(cfg, {k: v.to(device) for k, v in sd.items()}))
    assert adapter.decode_incremental is None
    half = Qwen35Oracle(cfg, sd)
    truth = Qwen35Oracle(cfg, {k: v.float() for k, v in sd.items()})
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, cfg.vocab_size, (2, 70), generator=g)
    hist = torch.randint(0, cfg.vocab_size, (2, 5, 3), generator=g)
    res = adapter.prefill(ids.to(device))
    logits = adapter.decode(hist.to(device), res.state)
    torch.cuda.synchronize()
    h_logits, h_state = half.prefill(ids)
    t_logits, t_state = truth.prefill(ids)

    def rel(a, e):
        return ((a.float().cpu() - e.float()).norm() / e.float().norm()).item()

    for name, got, ref, exact in (("prefill", res.logits, h_logits, t_logits),
                                  ("decode", logits, half.decode(hist, h_state),
                                   truth.decode(hist, t_state))):
        e_gpu, e_ref = rel(got, exact), rel(ref, exact)
        print(f"fp16 model {name}: rel L2 to fp32 evaluation {e_gpu:.2e} (fp16 oracle {e_ref:.2e})",
              flush=True)
        assert e_gpu <= e_ref, f"fp16 {name}: GPU {e_gpu:.2e} vs fp16 oracle {e_ref:.2e}"
    widths = [6, 5, 4]
    result = grbeam_search(adapter, ids.to(device), widths)
    torch.cuda.synchronize()
    scores = torch.zeros(2, 1)
    history = torch.empty(2, 1, 0, dtype=torch.int64)
    lg = res.logits.cpu()[:, None]
    for step, w in enumerate(widths):
        if step:
            lg = adapter.decode(history.to(device), res.state).cpu()
        scores, parents, tokens = grbeam_ref.level_select(lg, scores, w)
        history = torch.cat((history.gather(1, parents[..., None].expand(2, w, step)),
                             tokens[..., None]), -1)
    assert torch.equal(history, result.tokens.cpu())
    assert torch.allclose(result.scores.cpu(), scores, atol=1e-4)
