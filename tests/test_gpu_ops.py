"""HIP operator parity against the CPU oracle and the reference golden vectors."""

import pytest
import torch

from _fixtures import bf16_from_bits, conv_inputs, gdn_inputs, load_npz
from conftest import assert_close_rel
from kadllm_amd import _lib, layers, ops
from oracle import ops_ref

pytestmark = pytest.mark.gpu


def _to(device, *ts):
    return [t.to(device) for t in ts]


# --------------------------------------------------------------------------
# MFMA operand layouts assumed by every kernel


@pytest.mark.parametrize("shape,name", [((16, 32, 16), "kad_selftest_mfma16"),
                                        ((32, 16, 32), "kad_selftest_mfma32")])
def test_mfma_lane_layout(device, shape, name):
    m, kdim, n = shape
    g = torch.Generator().manual_seed(7)
    a = torch.randn(m, kdim, generator=g).bfloat16()
    b = torch.randn(kdim, n, generator=g).bfloat16()
    ad, bd = a.to(device), b.to(device)
    c = torch.full((m, n), float("nan"), device=device)
    _lib.call(name, _lib.ptr(ad), _lib.ptr(bd), _lib.ptr(c), _lib.stream_of(ad))
    torch.cuda.synchronize()
    expected = a.double() @ b.double()
    assert torch.allclose(c.cpu().double(), expected, rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------
# Gated DeltaNet suffix replay

GDN_CASES = [
    # B, W, T, H, HV, K, V
    (2, 256, 3, 16, 16, 128, 128),   # config-2 head shape, 2 of the 32 requests
    (3, 5, 2, 2, 4, 64, 64),         # GQA 2:1, ragged beam group
    (2, 20, 1, 4, 4, 128, 64),
    (2, 33, 4, 2, 2, 64, 128),
    (1, 1, 1, 1, 1, 64, 64),
    (2, 40, 5, 16, 16, 128, 128),    # suffixes past 4 tokens: 5..8
    (1, 17, 6, 2, 4, 64, 64),
    (2, 24, 7, 4, 4, 128, 128),
    (1, 130, 8, 2, 2, 128, 64),
]


@pytest.mark.parametrize("case", GDN_CASES)
def test_gdn_replay_bf16_matches_oracle(device, case):
    B, W, T, H, HV, K, V = case
    q, k, v, g, beta, S = gdn_inputs(B, W, T, H, HV, K, V, seed=sum(case))
    expected = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=W)
    qd, kd, vd, gd, bd, Sd = _to(device, q, k, v, g, beta, S)
    S_before = Sd.clone()
    out = ops.gated_delta(qd, kd, vd, gd, bd, Sd, beam_width=W)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == v.shape
    assert torch.equal(Sd, S_before), "shared prefix state was modified"
    # bf16 output: one rounding of a value computed from fp32 state
    assert_close_rel(out.cpu(), expected, rtol=1e-2, atol_frac=2e-3, name=f"gdn {case}")


@pytest.mark.parametrize("T", [1, 2, 3, 4])
@pytest.mark.parametrize("W", [16, 48, 256, 512])
def test_gdn_replay_lds_staged_equals_register_kernel(device, T, W):
    """The decode shapes (bf16, K = V = 128, fp32 decay, bf16 beta, beams in
    whole groups of 16) run the LDS-staged replay; the same values with an
    fp32 beta take the register-load kernel, whose arithmetic the staged one
    repeats, so the two agree bit for bit (W = 512: four workgroups of 128
    beams per request; 48: three groups, so the 3-stage ring wraps)."""
    B, H, HV, K, V = 2, 4, 8, 128, 128
    q, k, v, g, beta, S = gdn_inputs(B, W, T, H, HV, K, V, seed=T * 1000 + W)
    qd, kd, vd, gd, bd, Sd = _to(device, q, k, v, g, beta, S)
    staged = ops.gated_delta(qd, kd, vd, gd, bd, Sd, beam_width=W)
    plain = ops.gated_delta(qd, kd, vd, gd, bd.float(), Sd, beam_width=W)
    torch.cuda.synchronize()
    assert torch.equal(staged, plain)
    expected = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=W)
    assert_close_rel(staged.cpu(), expected, rtol=1e-2, atol_frac=2e-3, name=f"staged T={T} W={W}")


@pytest.mark.parametrize("case", [(2, 7, 3, 2, 4, 64, 64), (1, 16, 4, 4, 4, 128, 128),
                                  (1, 9, 8, 2, 2, 128, 128)])
def test_gdn_replay_fp32_matches_oracle(device, case):
    B, W, T, H, HV, K, V = case
    q, k, v, g, beta, S = gdn_inputs(B, W, T, H, HV, K, V, dtype=torch.float32, seed=3)
    expected = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=W, compute=torch.float64)
    out = ops.gated_delta(*_to(device, q, k, v, g, beta, S), beam_width=W)
    torch.cuda.synchronize()
    # hi/lo bf16 split MFMA: ~2^-16 relative products, fp32 accumulation
    assert_close_rel(out.cpu(), expected.float(), rtol=1e-4, atol_frac=1e-4, name="gdn fp32")


def test_gdn_replay_bf16_state_and_gates(device):
    # bf16 state and bf16 decay (the reference kernel benchmark's dtypes)
    B, W, T, H, HV, K, V = 2, 9, 3, 2, 2, 128, 128
    q, k, v, g, beta, S = gdn_inputs(B, W, T, H, HV, K, V, seed=11, state_std=0.1,
                                     state_dtype=torch.bfloat16)
    g = g.bfloat16()
    expected = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=W)
    out = ops.gated_delta(*_to(device, q, k, v, g, beta, S), beam_width=W)
    torch.cuda.synchronize()
    assert_close_rel(out.cpu(), expected, rtol=1e-2, atol_frac=2e-3, name="gdn bf16 state")


def test_gdn_replay_golden_fixture(device):
    f = load_npz("ops_bf16.npz")
    q, k, v = (bf16_from_bits(f[n]) for n in ("gdn_q", "gdn_k", "gdn_v"))
    g = torch.from_numpy(f["gdn_g"])
    beta = bf16_from_bits(f["gdn_beta"])
    S = torch.from_numpy(f["gdn_state"])
    expected = bf16_from_bits(f["gdn_out"])
    out = ops.gated_delta(*_to(device, q, k, v, g, beta, S), beam_width=3)
    torch.cuda.synchronize()
    assert_close_rel(out.cpu(), expected, rtol=1e-2, atol_frac=2e-3, name="gdn golden")


def test_gdn_replay_full_config2_sampled(device):
    """All 32 requests x 256 beams x 16 heads; requests 0, 17 and 31 checked
    against the oracle (requests are independent), prefix immutability checked."""
    B, W, T, H, HV, K, V = 32, 256, 3, 16, 16, 128, 128
    gen = torch.Generator(device=device).manual_seed(5)
    BW = B * W
    q = torch.randn(BW, T, H, K, generator=gen, device=device).bfloat16()
    k = torch.randn(BW, T, H, K, generator=gen, device=device).bfloat16()
    v = torch.randn(BW, T, HV, V, generator=gen, device=device).bfloat16()
    g = -torch.nn.functional.softplus(torch.randn(BW, T, HV, generator=gen, device=device))
    beta = torch.sigmoid(torch.randn(BW, T, HV, generator=gen, device=device)).bfloat16()
    S = torch.randn(B, HV, K, V, generator=gen, device=device) * 0.02
    S_before = S.clone()
    out = ops.gated_delta(q, k, v, g, beta, S, beam_width=W)
    torch.cuda.synchronize()
    assert torch.equal(S, S_before)
    for r in (0, 17, 31):
        rows = slice(r * W, (r + 1) * W)
        args = [t[rows].cpu() for t in (q, k, v, g, beta)] + [S[r:r + 1].cpu()]
        expected = ops_ref.gated_delta(*args, beam_width=W)
        assert_close_rel(out[rows].cpu(), expected, rtol=1e-2, atol_frac=2e-3,
                         name=f"config2 request {r}")


def test_gdn_replay_closed_form_beta_zero(device):
    """beta = 0: o_t = gamma_t S0^T q^_t (no delta update), in float64."""
    B, W, T, H, HV, K, V = 2, 16, 3, 2, 2, 128, 128
    q, k, v, g, beta, S = gdn_inputs(B, W, T, H, HV, K, V, dtype=torch.float32, seed=21)
    beta = torch.zeros_like(beta)
    out = ops.gated_delta(*_to(device, q, k, v, g, beta, S), beam_width=W)
    torch.cuda.synchronize()
    qn = q.double() / (q.double().square().sum(-1, keepdim=True) + 1e-6).sqrt() * K ** -0.5
    gam = g.double().cumsum(1).exp()                                  # [BW,T,HV]
    S0 = S.double().repeat_interleave(W, 0)                           # [BW,HV,K,V]
    expected = torch.einsum("nhkv,nthk->nthv", S0, qn) * gam[..., None]
    assert_close_rel(out.cpu(), expected.float(), rtol=1e-4, atol_frac=1e-4, name="beta=0")


def test_gdn_head_dims_outside_the_replay_and_the_limit(device):
    """Head dims the replay does not take run the per-token recurrence kernel;
    key dims past its 256 raise (KadLibraryError, a RuntimeError)."""
    q, k, v, g, beta, S = gdn_inputs(1, 2, 2, 1, 1, 96, 96)
    out = ops.gated_delta(*_to(device, q, k, v, g, beta, S), beam_width=2)
    expected = ops_ref.gated_delta(q, k, v, g, beta, S, beam_width=2)
    assert_close_rel(out, expected, rtol=1e-2, atol_frac=4e-3, name="K=V=96")
    q, k, v, g, beta, S = gdn_inputs(1, 2, 2, 1, 1, 320, 64)
    with pytest.raises(RuntimeError, match="key dims <= 256"):
        ops.gated_delta(*_to(device, q, k, v, g, beta, S), beam_width=2)


# --------------------------------------------------------------------------
# causal conv1d


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("layout", ["reference", "token_major"])
@pytest.mark.parametrize("case", [(2, 5, 24, 3), (3, 4, 6144, 2), (1, 1, 8, 1)])
def test_conv_matches_oracle(device, dtype, layout, case):
    B, W, C, T = case
    x, st, w = conv_inputs(B, W, C, T, dtype=dtype, seed=C + T)
    if layout == "token_major":
        # the adapter's transposed view of a [BW, T, C] projection (strides (T*C, 1, C))
        x = x.transpose(1, 2).contiguous().transpose(1, 2)
    expected = ops_ref.causal_conv1d(x, st, w, beam_width=W)
    xd, sd, wd = x.to(device), st.to(device), w.to(device)
    if layout == "token_major":
        xd = xd.transpose(1, 2).contiguous().transpose(1, 2)
    sd_before = sd.clone()
    out = ops.causal_conv1d(xd, sd, wd, beam_width=W)
    torch.cuda.synchronize()
    assert torch.equal(sd, sd_before)
    if dtype == torch.bfloat16:
        a, e = out.cpu().float(), expected.float()
        ulp = (e.abs() * 2 ** -7).clamp_min(1e-30)
        assert ((a - e).abs() <= ulp).all(), "bf16 conv differs by more than 1 ulp"
        exact = (a == e).float().mean().item()
        assert exact > 0.99, f"only {exact:.4f} bit-exact"
    else:
        assert_close_rel(out.cpu(), expected, rtol=1e-5, atol_frac=1e-6, name="conv fp32")


@pytest.mark.parametrize("T", [1, 2, 5])
@pytest.mark.parametrize("history", [3, 4, 6])
def test_conv_beam_groups_and_state_history(device, T, history):
    """Beam counts that straddle the kernel's beam groups, and prefix states holding
    3, 4 (the model's conv cache) or more taps."""
    B, W, C = 3, 13, 64
    x, st, w = conv_inputs(B, W, C, T, seed=history * 10 + T, history=history)
    x = x.transpose(1, 2).contiguous().transpose(1, 2)
    expected = ops_ref.causal_conv1d(x, st, w, beam_width=W)
    xd = x.to(device).transpose(1, 2).contiguous().transpose(1, 2)
    out = ops.causal_conv1d(xd, st.to(device), w.to(device), beam_width=W)
    torch.cuda.synchronize()
    a, e = out.cpu().float(), expected.float()
    assert ((a - e).abs() <= (e.abs() * 2 ** -7).clamp_min(1e-30)).all()
    assert (a == e).float().mean().item() > 0.99


@pytest.mark.parametrize("T", [1, 2, 3, 4])
@pytest.mark.parametrize("history", [3, 4, 6])
def test_conv_reference_layout_equals_token_major(device, T, history):
    """The contiguous [BW, C, T] layout (the reference's, with its own vector
    kernel) gives the token-major kernel's bits, beam counts straddling the
    beam groups and prefix states of 3, 4 and 6 taps."""
    B, W, C = 3, 13, 6144 // 8
    x, st, w = conv_inputs(B, W, C, T, seed=history * 7 + T, history=history)
    xd, sd, wd = x.to(device), st.to(device), w.to(device)
    ref_layout = ops.causal_conv1d(xd, sd, wd, beam_width=W)
    tm = ops.causal_conv1d(xd.transpose(1, 2).contiguous().transpose(1, 2), sd, wd, beam_width=W)
    torch.cuda.synchronize()
    assert ref_layout.is_contiguous() and torch.equal(ref_layout, tm)
    e = ops_ref.causal_conv1d(x, st, w, beam_width=W).float()
    a = ref_layout.cpu().float()
    assert ((a - e).abs() <= (e.abs() * 2 ** -7).clamp_min(1e-30)).all()


def test_conv_golden_fixture(device):
    f = load_npz("ops_bf16.npz")
    x, st, w = (bf16_from_bits(f[n]) for n in ("conv_x", "conv_state", "conv_w"))
    expected = bf16_from_bits(f["conv_out"])
    out = ops.causal_conv1d(*_to(device, x, st, w), beam_width=3)
    torch.cuda.synchronize()
    a, e = out.cpu().float(), expected.float()
    assert ((a - e).abs() <= e.abs() * 2 ** -7 + 1e-30).all()
    assert (a == e).float().mean().item() > 0.97


def test_conv_width_and_bias_variants(device):
    B, W, C, T = 2, 3, 16, 3
    g = torch.Generator().manual_seed(9)
    x = torch.randn(B * W, C, T, generator=g)
    st = torch.randn(B, C, 5, generator=g)
    for width in (1, 2, 3, 4):
        w = torch.randn(C, width, generator=g)
        bias = torch.randn(C, generator=g)
        for act in (None, "silu"):
            expected = ops_ref.causal_conv1d(x, st, w, beam_width=W, bias=bias, activation=act)
            out = ops.causal_conv1d(*_to(device, x, st, w), beam_width=W, bias=bias.to(device),
                                    activation=act)
            torch.cuda.synchronize()
            assert_close_rel(out.cpu(), expected, rtol=1e-5, atol_frac=1e-6,
                             name=f"conv width {width} act {act}")


def _conv_replay_inputs(B, W, T, H, HV, hist, seed):
    K = V = 128
    C = 2 * H * K + HV * V
    ld = C + 40                     # the projection row carries more columns (z, gates, pad)
    g = torch.Generator().manual_seed(seed)
    R = B * W * T
    proj = (torch.randn(R, ld, generator=g) * 0.7).bfloat16()
    cs = (torch.randn(B, hist + 2, C, generator=g) * 0.7).bfloat16().transpose(1, 2)  # strided
    cw = (torch.rand(C, 4, generator=g) - 0.5).bfloat16()
    logd = -torch.rand(R, HV, generator=g) * 0.3
    beta = torch.rand(R, HV, generator=g).bfloat16()
    S = torch.randn(B, HV, K, V, generator=g) * 0.05
    return proj, cs, cw, logd, beta, S, C, ld


@pytest.mark.parametrize("T", [1, 2])
@pytest.mark.parametrize("W,H,HV,hist", [(16, 2, 2, 4), (48, 4, 8, 4), (256, 2, 4, 6),
                                         (512, 1, 2, 4)])
def test_gdn_replay_conv_fused_equals_conv_then_replay(device, T, W, H, HV, hist):
    """kad_gdn_suffix_replay_conv against kad_causal_conv_suffix followed by
    kad_gdn_suffix_replay, bit for bit: projection rows wider than q | k | v,
    a strided prefix conv state with more than 3 slots, GQA heads, beams in
    one and in several workgroups per request (W = 512)."""
    B, K = 2, 128
    proj, cs, cw, logd, beta, S, C, ld = _conv_replay_inputs(B, W, T, H, HV, hist,
                                                             seed=T * 100 + W + hist)
    pd, csd, cwd, gd, bd, Sd = _to(device, proj, cs, cw, logd, beta, S)
    csd = csd[:, :, 1:1 + hist]     # [B, C, hist] view with strides (C*(hist+2), 1, C)
    R = B * W * T
    stream = _lib.stream_of(pd)
    conv = torch.empty(R, C, dtype=torch.bfloat16, device=device)
    _lib.call("kad_causal_conv_suffix", _lib.ptr(pd), T * ld, 1, ld, _lib.ptr(csd), *csd.stride(),
              hist, _lib.ptr(cwd), 4, None, _lib.ptr(conv), T * C, 1, C, B, W, C, T, 0, 1, stream)
    o1 = torch.empty(R, HV * K, dtype=torch.bfloat16, device=device)
    base, es = conv.data_ptr(), conv.element_size()
    _lib.call("kad_gdn_suffix_replay", _lib.ptr(conv), _lib.ptr_at(base + H * K * es),
              _lib.ptr_at(base + 2 * H * K * es), C, C, 0, _lib.ptr(gd), 2, _lib.ptr(bd), 0, HV,
              _lib.ptr(Sd), 2, _lib.ptr(o1), HV * K, B, W, T, H, HV, K, K, K ** -0.5, stream)
    o2 = torch.full((R, HV * K), 3.0, dtype=torch.bfloat16, device=device)
    _lib.call("kad_gdn_suffix_replay_conv", _lib.ptr(pd), ld, _lib.ptr(csd), *csd.stride(), hist,
              _lib.ptr(cwd), _lib.ptr(gd), 2, _lib.ptr(bd), 0, HV, _lib.ptr(Sd), 2, _lib.ptr(o2),
              HV * K, B, W, T, H, HV, K, K, K ** -0.5, stream)
    # the gated form against kad_rmsnorm_gated of the same outputs (gate rows:
    # any row-strided bf16 columns, here the projection's from column 8), all
    # tokens and the last token only
    zc = pd[:, 8:8 + HV * K]
    gen = torch.Generator().manual_seed(5 + T)
    nw = (1.0 + 0.1 * torch.randn(K, generator=gen)).bfloat16().to(device)
    eps = 1e-6
    y_all = layers.rmsnorm_gated(o1, zc, nw, eps, HV)
    y_last = layers.rmsnorm_gated(o1.view(B * W, T, -1)[:, -1], zc.view(B * W, T, -1)[:, -1],
                                  nw, eps, HV)
    for last, ref in ((0, y_all), (1, y_last)):
        yg = torch.full_like(ref, 5.0)
        _lib.call("kad_gdn_suffix_replay_conv_gated", _lib.ptr(pd), ld, _lib.ptr(csd),
                  *csd.stride(), hist, _lib.ptr(cwd), _lib.ptr(gd), 2, _lib.ptr(bd), 0, HV,
                  _lib.ptr(Sd), 2, _lib.ptr(zc), zc.stride(0), _lib.ptr(nw), eps, last,
                  _lib.ptr(yg), HV * K, B, W, T, H, HV, K, K, K ** -0.5, stream)
        torch.cuda.synchronize()
        assert torch.equal(yg, ref), f"gated fused replay differs (last_token_only={last})"
    torch.cuda.synchronize()
    assert torch.equal(o2, o1), "fused conv replay differs from conv then replay"
    # and the oracle on the conv output the HIP conv produced
    q = conv[:, :H * K].cpu().reshape(B * W, T, H, K)
    k = conv[:, H * K:2 * H * K].cpu().reshape(B * W, T, H, K)
    v = conv[:, 2 * H * K:].cpu().reshape(B * W, T, HV, K)
    expected = ops_ref.gated_delta(q, k, v, logd.reshape(B * W, T, HV),
                                   beta.reshape(B * W, T, HV), S, beam_width=W)
    assert_close_rel(o2.cpu().reshape(B * W, T, HV, K), expected, rtol=1e-2, atol_frac=2e-3,
                     name=f"fused T={T} W={W}")


def test_gdn_replay_conv_rejects_what_it_does_not_fuse(device):
    """Shapes outside the fused form are refused (the model then makes the two
    calls): three-token suffixes, beam counts off the 16-beam groups, K = 64."""
    for T, W, K in [(3, 16, 128), (1, 24, 128), (1, 16, 64)]:
        B, H, HV = 1, 2, 2
        C = 2 * H * K + HV * K
        proj = torch.zeros(B * W * T, C, dtype=torch.bfloat16, device=device)
        cs = torch.zeros(B, C, 4, dtype=torch.bfloat16, device=device)
        cw = torch.zeros(C, 4, dtype=torch.bfloat16, device=device)
        gd = torch.zeros(B * W * T, HV, device=device)
        bd = torch.zeros(B * W * T, HV, dtype=torch.bfloat16, device=device)
        Sd = torch.zeros(B, HV, K, K, device=device)
        o = torch.empty(B * W * T, HV * K, dtype=torch.bfloat16, device=device)
        with pytest.raises(_lib.KadLibraryError, match="unsupported"):
            _lib.call("kad_gdn_suffix_replay_conv", _lib.ptr(proj), C, _lib.ptr(cs), *cs.stride(),
                      4, _lib.ptr(cw), _lib.ptr(gd), 2, _lib.ptr(bd), 0, HV, _lib.ptr(Sd), 2,
                      _lib.ptr(o), HV * K, B, W, T, H, HV, K, K, K ** -0.5, _lib.stream_of(proj))


@pytest.mark.parametrize("W,Wp,H,HV", [(16, 16, 2, 2), (48, 32, 4, 8), (256, 256, 2, 4)])
def test_gdn_replay_conv_gated_parents_equals_gather(device, W, Wp, H, HV):
    """kad_gdn_suffix_replay_conv_gated_parents (the earlier token read through
    each beam's parent from the parent level's rows) against
    kad_gather_beam_rows of those rows followed by
    kad_gdn_suffix_replay_conv_gated on the gathered buffer, bit for bit,
    including a parent index past Wp (both clamp it)."""
    B, T, K, hist = 2, 2, 128, 4
    C = 2 * H * K + HV * K
    ld = C + HV * K + 40                 # q | k | v | z | more columns
    g = torch.Generator().manual_seed(W + Wp + H + HV)
    prev = (torch.randn(B * Wp * (T - 1), ld, generator=g) * 0.7).bfloat16().to(device)
    cur = (torch.randn(B * W, ld, generator=g) * 0.7).bfloat16().to(device)
    parents = torch.randint(0, Wp, (B, W), generator=g)
    parents[0, 3] = Wp + 5
    parents = parents.to(device)
    cs = (torch.randn(B, C, hist, generator=g) * 0.7).bfloat16().to(device)
    cw = (torch.rand(C, 4, generator=g) - 0.5).bfloat16().to(device)
    logd = (-torch.rand(B * W * T, HV, generator=g) * 0.3).to(device)
    beta = torch.rand(B * W * T, HV, generator=g).bfloat16().to(device)
    S = (torch.randn(B, HV, K, K, generator=g) * 0.05).to(device)
    nw = (1.0 + 0.1 * torch.randn(K, generator=g)).bfloat16().to(device)
    stream = _lib.stream_of(cur)
    # reference: the rows gathered into one [B*W*T] buffer
    full = torch.empty(B * W * T, ld, dtype=torch.bfloat16, device=device)
    _lib.call("kad_gather_beam_rows", _lib.ptr(prev), ld * 2, T - 1, _lib.ptr(full), ld * 2, T,
              T - 1, ld * 2, _lib.ptr(parents), B, W, Wp, stream)
    full.view(B * W, T, ld)[:, T - 1].copy_(cur)
    y1 = torch.empty(B * W, HV * K, dtype=torch.bfloat16, device=device)
    _lib.call("kad_gdn_suffix_replay_conv_gated", _lib.ptr(full), ld, _lib.ptr(cs), *cs.stride(),
              hist, _lib.ptr(cw), _lib.ptr(logd), 2, _lib.ptr(beta), 0, HV, _lib.ptr(S), 2,
              _lib.ptr(full[:, C:]), ld, _lib.ptr(nw), 1e-6, 1, _lib.ptr(y1), HV * K, B, W, T, H,
              HV, K, K, K ** -0.5, stream)
    y2 = torch.full_like(y1, 2.0)
    _lib.call("kad_gdn_suffix_replay_conv_gated_parents", _lib.ptr(prev), ld, _lib.ptr(parents), Wp,
              _lib.ptr(cur), ld, _lib.ptr(cs), *cs.stride(), hist, _lib.ptr(cw), _lib.ptr(logd), 2,
              _lib.ptr(beta), 0, HV, _lib.ptr(S), 2, _lib.ptr(cur[:, C:]), ld, _lib.ptr(nw), 1e-6,
              _lib.ptr(y2), HV * K, B, W, T, H, HV, K, K, K ** -0.5, stream)
    torch.cuda.synchronize()
    assert torch.equal(y2, y1), "parent-row fused replay differs from gather + fused replay"
