"""HIP GEMM, row-wise and attention kernels against fp32 references and the oracle."""

import pytest
import torch
from torch.nn import functional as F

from conftest import assert_close_rel
from kadllm_amd import layers, ops
from kadllm_amd.attention import attention_prefill
from oracle import ops_ref, qwen35_ref

pytestmark = pytest.mark.gpu


def _bf16_ulp_close(actual, expected, name, min_exact=0.95):
    """bf16 results within one ulp of the bf16-rounded fp32 reference.

    An absolute term of 2e-5 * max|e| covers outputs that cancel to near zero,
    where fp32 accumulation order alone moves the value by many bf16 ulps.
    """
    a = actual.float().cpu()
    e = expected.float().cpu()
    ulp = e.abs() * 2 ** -7 + 2e-5 * e.abs().max() + 1e-30
    bad = (a - e).abs() > ulp
    assert not bad.any(), f"{name}: {int(bad.sum())} elements differ by more than 1 ulp; " \
        f"max {(a - e).abs().max().item():.3e}"
    exact = (a == e).float().mean().item()
    assert exact >= min_exact, f"{name}: only {exact:.4f} bit-exact"


def test_cache_prefetch_reads_and_writes_nothing(device):
    """kad_cache_prefetch leaves its ranges as they were (odd tails included)
    and checks its arguments."""
    from kadllm_amd import _lib
    a = torch.randn(1 << 20, device=device).bfloat16()
    b = torch.randint(0, 255, (12345,), dtype=torch.uint8, device=device)
    a0, b0 = a.clone(), b.clone()
    layers.cache_prefetch(a, b)
    layers.cache_prefetch(a)
    torch.cuda.synchronize()
    assert torch.equal(a, a0) and torch.equal(b, b0)
    with pytest.raises(_lib.KadLibraryError, match="16-byte aligned"):
        layers.cache_prefetch(b[1:])
    with pytest.raises(_lib.KadLibraryError, match="null pointer"):
        _lib.call("kad_cache_prefetch", None, 64, None, 0, _lib.stream_of(a))


# --------------------------------------------------------------------------
# GEMM


@pytest.mark.parametrize("M,N,K", [(37, 200, 64), (130, 384, 128), (32, 4096, 256),
                                   (1024, 1536, 1024), (300, 8320, 1024)])
def test_gemm_store(device, M, N, K):
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16()
    out = layers.gemm(a.to(device), w.to(device))
    torch.cuda.synchronize()
    ref = (a.float() @ w.float().T).bfloat16()
    _bf16_ulp_close(out, ref, f"gemm {M}x{N}x{K}")


def test_gemm_full_decode_shape_sampled_rows(device):
    M, N, K = 8192, 8320, 1024
    gen = torch.Generator(device=device).manual_seed(1)
    a = torch.randn(M, K, generator=gen, device=device).bfloat16()
    w = (torch.randn(N, K, generator=gen, device=device) * 0.02).bfloat16()
    out = layers.gemm(a, w)
    torch.cuda.synchronize()
    rows = torch.tensor([0, 1, 127, 128, 4095, 8000, 8191])
    ref = (a[rows].float().cpu() @ w.float().cpu().T).bfloat16()
    _bf16_ulp_close(out[rows], ref, "gemm 8192x8320x1024")


def test_gemm_strided_operands_and_residual(device):
    M, N, K = 200, 256, 192
    g = torch.Generator().manual_seed(3)
    big_a = torch.randn(M, K + 64, generator=g).bfloat16()
    a = big_a[:, 32:32 + K]                       # row stride K+64, 64-byte offset
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16()
    x = torch.randn(M, N, generator=g).bfloat16()
    xd = x.to(device)
    layers.gemm(big_a.to(device)[:, 32:32 + K], w.to(device), out=xd,
                epilogue=layers.EPI_RESIDUAL, residual=xd)
    torch.cuda.synchronize()
    mixed = (a.float() @ w.float().T).bfloat16()
    ref = (x.float() + mixed.float()).bfloat16()
    _bf16_ulp_close(xd, ref, "gemm residual")


def test_gemm_swiglu(device):
    M, F_, K = 150, 192, 256
    g = torch.Generator().manual_seed(4)
    a = torch.randn(M, K, generator=g).bfloat16()
    wg = (torch.randn(F_, K, generator=g) * 0.05).bfloat16()
    wu = (torch.randn(F_, K, generator=g) * 0.05).bfloat16()
    packed = torch.stack((wg.reshape(F_ // 32, 32, K), wu.reshape(F_ // 32, 32, K)), 1).reshape(2 * F_, K)
    out = layers.gemm(a.to(device), packed.to(device), epilogue=layers.EPI_SWIGLU)
    torch.cuda.synchronize()
    gate = (a.float() @ wg.float().T).bfloat16()
    up = (a.float() @ wu.float().T).bfloat16()
    ref = F.silu(gate) * up                        # bf16 ops, as the MLP module
    _bf16_ulp_close(out, ref, "gemm swiglu", min_exact=0.9)


@pytest.mark.parametrize("epi", [layers.EPI_STORE, layers.EPI_RESIDUAL, layers.EPI_SWIGLU])
def test_gemm_tile_configurations_agree(device, epi):
    """Every tile configuration (including the 256x256 16x16x32 ones) on ragged
    M and N, a strided output and an in-place residual: bit-identical results
    (same K order) within 1 ulp of the fp32 reference."""
    from kadllm_amd import _lib
    M, N, K = 600, 832, 448  # 7 K tiles: the unpaired last tile
    g = torch.Generator().manual_seed(40 + epi)
    a = torch.randn(M, K, generator=g).bfloat16()
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16()
    n_out = N // 2 if epi == layers.EPI_SWIGLU else N
    x = torch.randn(M, n_out, generator=g).bfloat16()
    ad, wd = a.to(device), w.to(device)
    outs = {}
    cfgs = [c for c in (1, 2, 5, 11, 12, 16, 18, 19, 20)
            if not (c in (11, 12) and epi == layers.EPI_SWIGLU)]
    for cfg in cfgs:
        c = torch.zeros(M, n_out + 16, dtype=torch.bfloat16, device=device)  # ldc > width
        cv = c[:, :n_out]
        if epi == layers.EPI_RESIDUAL:
            cv.copy_(x.to(device))
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(ad), K, _lib.ptr(wd), K, _lib.ptr(cv), c.stride(0),
                  _lib.ptr(cv) if epi == layers.EPI_RESIDUAL else None,
                  c.stride(0) if epi == layers.EPI_RESIDUAL else 0, M, N, K, epi, cfg,
                  _lib.stream_of(ad))
        torch.cuda.synchronize()
        assert (c[:, n_out:] == 0).all(), f"config {cfg} wrote past the output width"
        outs[cfg] = cv.cpu()
    for cfg in cfgs[1:]:
        assert torch.equal(outs[cfg], outs[1]), f"config {cfg} differs from config 1"
    prod = (a.float() @ w.float().T).bfloat16()
    if epi == layers.EPI_STORE:
        _bf16_ulp_close(outs[16], prod, "gemm tiles store")
    elif epi == layers.EPI_RESIDUAL:
        # bf16(x + bf16(acc)): the inner rounding may differ by one ulp of the
        # product (fp32 summation order), which survives the add
        ref = (x.float() + prod.float()).bfloat16().float()
        tol = (ref.abs() + prod.float().abs()) * 2 ** -7 + 1e-30
        assert ((outs[16].float() - ref).abs() <= tol).all(), "gemm tiles residual"
        assert (outs[16].float() == ref).float().mean().item() > 0.9
    else:
        gu = prod.reshape(M, N // 64, 2, 32)
        ref = (F.silu(gu[:, :, 0]) * gu[:, :, 1]).reshape(M, n_out)
        _bf16_ulp_close(outs[16], ref, "gemm tiles swiglu", min_exact=0.9)


@pytest.mark.parametrize("N,epi", [(7168, layers.EPI_SWIGLU), (5120, layers.EPI_STORE),
                                   (5120, layers.EPI_RESIDUAL)])
def test_gemm_last_round_column_split_is_bitwise(device, N, epi):
    """At M = 8,192 the 256 x 256 tiles of the SwiGLU projection (N = 7,168)
    fill 3.5 rounds of the chip's CUs: the automatic choice runs the columns
    past the last whole round as 128 x 128 tiles in a second launch.  The
    result equals the unsplit 256 x 256 kernel's bit for bit (and so does the
    automatic choice for N = 5,120, left whole)."""
    from kadllm_amd import _lib
    M, K = 8192, 1024
    gen = torch.Generator(device=device).manual_seed(N + epi)
    a = torch.randn(M, K, generator=gen, device=device).bfloat16()
    w = (torch.randn(N, K, generator=gen, device=device) * 0.05).bfloat16()
    n_out = N // 2 if epi == layers.EPI_SWIGLU else N
    x = torch.randn(M, n_out, generator=gen, device=device).bfloat16()
    outs = []
    for cfg in (0, 16):
        c = x.clone() if epi == layers.EPI_RESIDUAL else torch.zeros(M, n_out, dtype=torch.bfloat16,
                                                                      device=device)
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(a), K, _lib.ptr(w), K, _lib.ptr(c), n_out,
                  _lib.ptr(c) if epi == layers.EPI_RESIDUAL else None,
                  n_out if epi == layers.EPI_RESIDUAL else 0, M, N, K, epi, cfg,
                  _lib.stream_of(a))
        outs.append(c)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    rows = torch.tensor([0, 4097, 8191], device=device)
    prod = (a[rows].float() @ w.float().T).bfloat16()
    if epi == layers.EPI_STORE:
        _bf16_ulp_close(outs[0][rows], prod, "split gemm store")


@pytest.mark.parametrize("M,N,K,epi", [(8192, 32, 1024, layers.EPI_STORE),
                                       (600, 20, 256, layers.EPI_STORE),
                                       (1000, 32, 768, layers.EPI_RESIDUAL),
                                       (333, 7, 2048, layers.EPI_STORE),
                                       (20000, 32, 512, layers.EPI_RESIDUAL)])
def test_gemm_narrow_output_whole_k_waves_agree(device, M, N, K, epi):
    """Outputs of at most 32 columns (the GDN gate projection): the whole-K
    32-row waves (configuration 13, which the automatic choice takes for
    them) against 64x32 and 32x256 tiles, on ragged M, strided A and C and
    K from one to eight 256-deep slices, with one wave per workgroup and
    (M = 20,000) four: the same bits, within 1 ulp of the fp32 product."""
    from kadllm_amd import _lib
    g = torch.Generator().manual_seed(M + N + K + epi)
    a_full = torch.randn(M, K + 64, generator=g).bfloat16().to(device)
    a = a_full[:, 32:32 + K]                       # lda = K + 64, 64-byte offset
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16().to(device)
    x = torch.randn(M, N, generator=g).bfloat16().to(device)
    outs = {}
    for cfg in (0, 1, 11, 13):
        c = torch.zeros(M, N + 8, dtype=torch.bfloat16, device=device)
        cv = c[:, :N]
        if epi == layers.EPI_RESIDUAL:
            cv.copy_(x)
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(a), a.stride(0), _lib.ptr(w), K, _lib.ptr(cv),
                  c.stride(0), _lib.ptr(cv) if epi == layers.EPI_RESIDUAL else None,
                  c.stride(0) if epi == layers.EPI_RESIDUAL else 0, M, N, K, epi, cfg,
                  _lib.stream_of(a))
        torch.cuda.synchronize()
        assert (c[:, N:] == 0).all(), f"config {cfg} wrote past the output width"
        outs[cfg] = cv.cpu()
    for cfg in (0, 1, 11):
        assert torch.equal(outs[cfg], outs[13]), f"config {cfg} differs from configuration 13"
    prod = (a.float().cpu() @ w.float().cpu().T).bfloat16()
    if epi == layers.EPI_STORE:
        _bf16_ulp_close(outs[13], prod, "narrow gemm store")
    else:
        ref = (x.float().cpu() + prod.float()).bfloat16().float()
        tol = (ref.abs() + prod.float().abs()) * 2 ** -7 + 1e-30
        assert ((outs[13].float() - ref).abs() <= tol).all(), "narrow gemm residual"


@pytest.mark.parametrize("N,K", [(33, 1024), (32, 448), (32, 2304)])
def test_gemm_narrow_output_configuration_rejects(device, N, K):
    """Configuration 13 takes N <= 32 and K a multiple of 256 up to 2,048 only."""
    from kadllm_amd import _lib
    a = torch.zeros(64, K, dtype=torch.bfloat16, device=device)
    w = torch.zeros(N, K, dtype=torch.bfloat16, device=device)
    c = torch.zeros(64, N, dtype=torch.bfloat16, device=device)
    with pytest.raises(_lib.KadLibraryError, match="tile configuration 13 needs"):
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(a), K, _lib.ptr(w), K, _lib.ptr(c), N, None, 0,
                  64, N, K, layers.EPI_STORE, 13, _lib.stream_of(a))


@pytest.mark.parametrize("K", [64, 128, 192])
def test_gemm_short_k_pipelines_agree(device, K):
    """The 16x16x32 configurations at K of one to three 64-deep tiles, where
    the loads of the tile after next run past the end of K."""
    from kadllm_amd import _lib
    M, N = 520, 768
    g = torch.Generator().manual_seed(70 + K)
    a = torch.randn(M, K, generator=g).bfloat16().to(device)
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16().to(device)
    outs = {}
    for cfg in (1, 2, 5, 16, 18, 19, 20):
        c = torch.zeros(M, N, dtype=torch.bfloat16, device=device)
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(a), K, _lib.ptr(w), K, _lib.ptr(c), N, None, 0,
                  M, N, K, layers.EPI_STORE, cfg, _lib.stream_of(a))
        outs[cfg] = c.cpu()
    for cfg in outs:
        assert torch.equal(outs[cfg], outs[1]), f"config {cfg} differs from config 1 at K={K}"
    ref = (a.float() @ w.float().T).cpu()
    assert ((outs[1].float() - ref).abs() <= 1e-2 * ref.abs() + 1e-2).all()


@pytest.mark.parametrize("K", [64, 192])
@pytest.mark.parametrize("epi", [layers.EPI_STORE, layers.EPI_RESIDUAL, layers.EPI_SWIGLU])
def test_gemm_persistent_tiles_agree(device, K, epi):
    """The persistent kernel (config 18) against the one-tile-per-workgroup
    forms (16, 19, 20) with more tiles than CUs, ragged last tiles in
    both dimensions, and tiles of one or three K slices, so that the load
    stream crosses tile boundaries at both stage parities; config 20 with the
    activations as its three-slot operand (M > N; the other order is covered
    by the tests above)."""
    from kadllm_amd import _lib
    M, N = 256 * 17 + 40, 256 * 16 + 64
    g = torch.Generator().manual_seed(90 + K + epi)
    a = torch.randn(M, K, generator=g).bfloat16().to(device)
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16().to(device)
    n_out = N // 2 if epi == layers.EPI_SWIGLU else N
    x = torch.randn(M, n_out, generator=g).bfloat16().to(device)
    outs = {}
    for cfg in (16, 18, 19, 20):
        c = x.clone() if epi == layers.EPI_RESIDUAL else torch.zeros(M, n_out, dtype=torch.bfloat16,
                                                                     device=device)
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(a), K, _lib.ptr(w), K, _lib.ptr(c), n_out,
                  _lib.ptr(c) if epi == layers.EPI_RESIDUAL else None,
                  n_out if epi == layers.EPI_RESIDUAL else 0, M, N, K, epi, cfg,
                  _lib.stream_of(a))
        torch.cuda.synchronize()
        outs[cfg] = c.cpu()
    assert torch.equal(outs[18], outs[16]), f"persistent 256x256 differs at K={K}"
    assert torch.equal(outs[16], outs[19]), f"128x128 tiles differ at K={K}"
    assert torch.equal(outs[16], outs[20]), f"three-slot 256x256 differs at K={K}"


@pytest.mark.parametrize("K", [64, 192, 1024])
@pytest.mark.parametrize("epi", [layers.EPI_STORE, layers.EPI_RESIDUAL, layers.EPI_SWIGLU])
def test_gemm_ping_pong_tiles_agree(device, K, epi):
    """The persistent ping-pong kernel (config 22) and the persistent 4-wave
    kernel (config 24) against config 16, bit for bit: 40 x 16 whole tiles
    (two or three per CU, so that epilogues run inside the next tile's first
    read phase, and a plain store's inside its first MFMA step) and tiles of
    one, three and 16 K slices, so that the load stream crosses tile
    boundaries at both stage parities."""
    from kadllm_amd import _lib
    M, N = 256 * 40, 256 * 16
    g = torch.Generator().manual_seed(190 + K + epi)
    a = torch.randn(M, K, generator=g).bfloat16().to(device)
    w = (torch.randn(N, K, generator=g) * 0.05).bfloat16().to(device)
    n_out = N // 2 if epi == layers.EPI_SWIGLU else N
    x = torch.randn(M, n_out, generator=g).bfloat16().to(device)
    outs = {}
    for cfg in (16, 22, 24):
        c = x.clone() if epi == layers.EPI_RESIDUAL else torch.zeros(M, n_out, dtype=torch.bfloat16,
                                                                     device=device)
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(a), K, _lib.ptr(w), K, _lib.ptr(c), n_out,
                  _lib.ptr(c) if epi == layers.EPI_RESIDUAL else None,
                  n_out if epi == layers.EPI_RESIDUAL else 0, M, N, K, epi, cfg,
                  _lib.stream_of(a))
        torch.cuda.synchronize()
        outs[cfg] = c.cpu()
    assert torch.equal(outs[22], outs[16]), f"ping-pong 256x256 differs at K={K}"
    assert torch.equal(outs[24], outs[16]), f"4-wave 256x256 differs at K={K}"


@pytest.mark.parametrize("epi", [layers.EPI_STORE, layers.EPI_RESIDUAL, layers.EPI_SWIGLU])
def test_gemm_four_wave_tiles_padded_rows(device, epi):
    """Config 24 with row strides above the widths (lda, ldw, ldc and ldr
    padded), one tile per CU or fewer (the first tile's fused store goes to a
    resource of no records), against config 16."""
    from kadllm_amd import _lib
    M, N, K = 256 * 8, 256 * 12, 320
    lda, ldw = K + 64, K + 32
    g = torch.Generator().manual_seed(290 + epi)
    a = torch.randn(M, lda, generator=g).bfloat16().to(device)
    w = (torch.randn(N, ldw, generator=g) * 0.05).bfloat16().to(device)
    n_out = N // 2 if epi == layers.EPI_SWIGLU else N
    ldc = n_out + 24
    x = torch.randn(M, ldc, generator=g).bfloat16().to(device)
    outs = {}
    for cfg in (16, 24):
        c = x.clone()
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(a), lda, _lib.ptr(w), ldw, _lib.ptr(c), ldc,
                  _lib.ptr(c) if epi == layers.EPI_RESIDUAL else None,
                  ldc if epi == layers.EPI_RESIDUAL else 0, M, N, K, epi, cfg, _lib.stream_of(a))
        torch.cuda.synchronize()
        outs[cfg] = c.cpu()
    assert torch.equal(outs[24], outs[16]), "4-wave 256x256 differs with padded rows"
    assert torch.equal(outs[24][:, n_out:], x[:, n_out:].cpu()), "wrote past the output width"


@pytest.mark.parametrize("cfg", [22, 24])
def test_gemm_whole_tile_kernels_reject_partial_tiles(device, cfg):
    from kadllm_amd import _lib
    a = torch.zeros(300, 64, dtype=torch.bfloat16, device=device)
    w = torch.zeros(256, 64, dtype=torch.bfloat16, device=device)
    c = torch.zeros(300, 256, dtype=torch.bfloat16, device=device)
    with pytest.raises(_lib.KadLibraryError, match="multiples of 256"):
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(a), 64, _lib.ptr(w), 64, _lib.ptr(c), 256, None,
                  0, 300, 256, 64, layers.EPI_STORE, cfg, _lib.stream_of(a))


def test_gemm_pipelined_tile_rejects_unaligned_output(device):
    from kadllm_amd import _lib
    a = torch.zeros(256, 64, dtype=torch.bfloat16, device=device)
    w = torch.zeros(256, 64, dtype=torch.bfloat16, device=device)
    c = torch.zeros(256, 263, dtype=torch.bfloat16, device=device)  # ldc not a multiple of 8
    with pytest.raises(_lib.KadLibraryError):
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(a), 64, _lib.ptr(w), 64, _lib.ptr(c), 263, None,
                  0, 256, 256, 64, layers.EPI_STORE, 16, _lib.stream_of(a))


@pytest.mark.parametrize("cfg", [11, 12, 13])
def test_gemm_skinny_tiles_reject_swiglu(device, cfg):
    """The 64x32 and 32x64 register-staged tiles carry no SwiGLU epilogue (a
    wave's 32 columns cannot hold a [gate 32 | up 32] block) and say so."""
    from kadllm_amd import _lib
    a = torch.zeros(64, 64, dtype=torch.bfloat16, device=device)
    w = torch.zeros(128, 64, dtype=torch.bfloat16, device=device)
    c = torch.zeros(64, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(_lib.KadLibraryError, match="has no SwiGLU epilogue"):
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(a), 64, _lib.ptr(w), 64, _lib.ptr(c), 64, None,
                  0, 64, 128, 64, layers.EPI_SWIGLU, cfg, _lib.stream_of(a))


@pytest.mark.parametrize("cfg", [3, 7, 17, 21, 23, -1])
def test_gemm_rejects_unknown_tile_configuration(device, cfg):
    from kadllm_amd import _lib
    a = torch.zeros(256, 64, dtype=torch.bfloat16, device=device)
    w = torch.zeros(256, 64, dtype=torch.bfloat16, device=device)
    c = torch.zeros(256, 256, dtype=torch.bfloat16, device=device)
    with pytest.raises(_lib.KadLibraryError, match="unknown gemm tile configuration"):
        _lib.call("kad_gemm_bf16_tiled", _lib.ptr(a), 64, _lib.ptr(w), 64, _lib.ptr(c), 256, None,
                  0, 256, 256, 64, layers.EPI_STORE, cfg, _lib.stream_of(a))


# --------------------------------------------------------------------------
# row-wise kernels


def test_rmsnorm_matches_oracle(device):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(333, 1024, generator=g).bfloat16()
    w = (torch.randn(1024, generator=g) * 0.1).bfloat16()
    out = layers.rmsnorm(x.to(device), w.to(device), 1e-6)
    torch.cuda.synchronize()
    _bf16_ulp_close(out, qwen35_ref.rms_norm(x, w, 1e-6), "rmsnorm", min_exact=0.99)


def test_rmsnorm_gated_matches_oracle(device):
    g = torch.Generator().manual_seed(6)
    rows, heads, D = 97, 16, 128
    big = torch.randn(rows, 3 * heads * D, generator=g).bfloat16()   # x and z live in a wider row
    x, z = big[:, :heads * D], big[:, 2 * heads * D:]
    w = (1 + torch.randn(D, generator=g) * 0.1).bfloat16()
    bd = big.to(device)
    out = layers.rmsnorm_gated(bd[:, :heads * D], bd[:, 2 * heads * D:], w.to(device), 1e-6, heads)
    torch.cuda.synchronize()
    ref = qwen35_ref.rms_norm_gated(x.reshape(-1, D), z.reshape(-1, D), w, 1e-6).reshape(rows, -1)
    _bf16_ulp_close(out, ref, "rmsnorm_gated", min_exact=0.99)


def test_gdn_gates_match_reference_formula(device):
    g = torch.Generator().manual_seed(7)
    rows, HV = 500, 16
    ab = torch.randn(rows, 40, generator=g).bfloat16()
    a, b = ab[:, 3:3 + HV], ab[:, 20:20 + HV]
    A_log = torch.log(torch.rand(HV, generator=g) * 16 + 1e-3).bfloat16()
    dt_bias = torch.ones(HV).bfloat16()
    abd = ab.to(device)
    gd, bd = layers.gdn_gates(abd[:, 3:3 + HV], abd[:, 20:20 + HV], A_log.to(device),
                              dt_bias.to(device))
    torch.cuda.synchronize()
    g_ref = -A_log.float().exp() * F.softplus(a.float() + dt_bias)   # qwen3_5.py:161-163
    b_ref = b.sigmoid()                                               # qwen3_5.py:169
    assert_close_rel(gd.cpu(), g_ref, rtol=1e-6, atol_frac=1e-7, name="g")
    _bf16_ulp_close(bd, b_ref, "beta", min_exact=0.99)


def test_qk_norm_rope_matches_oracle(device):
    from kadllm_amd.config import qwen35_08b_config
    cfg = qwen35_08b_config()
    g = torch.Generator().manual_seed(8)
    rows, T, H, D = 24, 3, 8, 256
    proj = torch.randn(rows * T, H * 2 * D, generator=g).bfloat16()
    wq = (torch.randn(D, generator=g) * 0.1).bfloat16()
    L0 = 1024
    inv = qwen35_ref.rope_inv_freq(cfg)
    out = torch.empty(rows * T, H, D, dtype=torch.bfloat16, device=device)
    layers.qk_norm_rope(proj.to(device), H * 2 * D, 2 * D, H, wq.to(device), out,
                        (0, H * D, D), rows * T, rows * T, D, 64, inv.to(device), L0, T, 1e-6)
    torch.cuda.synchronize()
    q = proj.reshape(rows, T, H, 2 * D)[..., :D]
    qn = qwen35_ref.rms_norm(q, wq, 1e-6).transpose(1, 2)              # [rows,H,T,D]
    pos = torch.arange(L0, L0 + T)[None].expand(rows, T)
    cos, sin = qwen35_ref.rope_cos_sin(cfg, pos, torch.bfloat16)
    ref = qwen35_ref.apply_rope(qn, cos[:, None], sin[:, None]).transpose(1, 2)
    _bf16_ulp_close(out.reshape(rows, T, H, D), ref, "qk_norm_rope", min_exact=0.99)


def test_embedding(device):
    g = torch.Generator().manual_seed(9)
    table = torch.randn(1000, 256, generator=g).bfloat16()
    ids = torch.randint(0, 1000, (7, 5), generator=g)
    out = layers.embedding(ids.to(device), table.to(device))
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), table[ids.reshape(-1)])


# --------------------------------------------------------------------------
# attention


def _attn_inputs(B, W, T, H, HK, L, D, seed):
    g = torch.Generator().manual_seed(seed)
    bf = torch.bfloat16
    q = torch.randn(B * W, T, H, D, generator=g).to(bf)
    pk = torch.randn(B, HK, L, D, generator=g).to(bf).transpose(1, 2)    # HF cache view
    pv = torch.randn(B, HK, L, D, generator=g).to(bf).transpose(1, 2)
    sk = torch.randn(B * W, T, HK, D, generator=g).to(bf)
    sv = torch.randn(B * W, T, HK, D, generator=g).to(bf)
    return q, pk, pv, sk, sv


@pytest.mark.parametrize("B,W,T,H,HK,L,D", [
    (2, 256, 1, 8, 2, 1024, 256), (2, 256, 3, 8, 2, 1024, 256),   # config-3 shape, 2 requests
    (2, 5, 2, 4, 1, 70, 64), (3, 3, 4, 4, 2, 5, 128), (1, 2, 3, 2, 2, 0, 64),
    (2, 3, 7, 4, 1, 45, 64),    # head dim 64 with 5-8 suffix keys (the 8-key fold)
    (1, 4, 6, 4, 2, 33, 128),   # head dim 128 with the 8-key fold
])
def test_prefix_attention_matches_oracle(device, B, W, T, H, HK, L, D):
    q, pk, pv, sk, sv = _attn_inputs(B, W, T, H, HK, L, D, seed=L + T)
    exp = ops_ref.prefix_attention(q, pk, pv, sk, sv, beam_width=W, compute=torch.float64)
    dev = [t.to(device) for t in (q, pk, pv, sk, sv)]
    pk_before = dev[1].clone()
    out = ops.prefix_attention(*dev, beam_width=W, backend="flash_attn")
    torch.cuda.synchronize()
    assert torch.equal(dev[1], pk_before)
    assert_close_rel(out.cpu(), exp, rtol=1e-2, atol_frac=4e-3, name="prefix attention")


def test_prefix_attention_mask_and_gate(device):
    B, W, T, H, HK, L, D = 2, 6, 3, 8, 2, 130, 256
    q, pk, pv, sk, sv = _attn_inputs(B, W, T, H, HK, L, D, seed=31)
    mask = torch.rand(B, L, generator=torch.Generator().manual_seed(2)) > 0.3
    mask[1] = False                                                      # fully masked prefix
    gate = torch.randn(B * W, T, H * D, generator=torch.Generator().manual_seed(3)).bfloat16()
    exp = ops_ref.prefix_attention(q, pk, pv, sk, sv, beam_width=W, prefix_mask=mask)
    exp = exp.reshape(B * W, T, -1) * gate.sigmoid()                     # bf16, qwen3_5.py:199-201
    dev = [t.to(device) for t in (q, pk, pv, sk, sv)]
    out = ops.prefix_attention(*dev, beam_width=W, prefix_mask=mask.to(device),
                               gate=gate.to(device))
    torch.cuda.synchronize()
    assert_close_rel(out.reshape(B * W, T, -1).cpu(), exp, rtol=1e-2, atol_frac=4e-3,
                     name="masked gated attention")


@pytest.mark.parametrize("D", [64, 256])
def test_prefix_attention_wide_score_range(device, D):
    """Scores that grow by far more than 2^64 (log2 units) after the first
    ones a row sees: the kernel's fixed softmax reference must be raised (its
    second pass), for the suffix-first decode order and across key tiles."""
    B, W, T, H, HK, L = 1, 4, 2, 4, 1, 200
    q, pk, pv, sk, sv = _attn_inputs(B, W, T, H, HK, L, D, seed=77)
    u = torch.randn(D, generator=torch.Generator().manual_seed(5))
    u = u / u.norm()
    q = (u * 12.0).expand_as(q).bfloat16().contiguous()     # every query along u
    sk = (-u * 12.0).expand_as(sk).bfloat16().contiguous()  # suffix scores -144, prefix ~N(0, 144)
    pk = pk.clone()
    pk[:, 150:] = (u * 14.0).bfloat16()                     # late prefix keys score far higher
    dev = [t.to(device) for t in (q, pk, pv, sk, sv)]
    out = ops.prefix_attention(*dev, beam_width=W, scale=1.0, backend="flash_attn")
    exp = ops_ref.prefix_attention(q, pk, pv, sk, sv, beam_width=W, scale=1.0,
                                   compute=torch.float64)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert_close_rel(out.cpu(), exp, rtol=1e-2, atol_frac=4e-3, name="wide-range attention")


@pytest.mark.parametrize("B,W,T,L", [(2, 5, 6, 77), (1, 3, 8, 0), (2, 4, 5, 19), (1, 2, 2, 33)])
def test_prefix_attention_d256_suffix_fold_and_ragged_prefix(device, B, W, T, L):
    """Head dim 256 with the 8-key suffix fold (T > 4), no prefix, a prefix
    shorter than one 32-key tile and ragged last tiles, against fp64."""
    H, HK, D = 8, 2, 256
    q, pk, pv, sk, sv = _attn_inputs(B, W, T, H, HK, L, D, seed=300 + L + T)
    exp = ops_ref.prefix_attention(q, pk, pv, sk, sv, beam_width=W, compute=torch.float64)
    dev = [t.to(device) for t in (q, pk, pv, sk, sv)]
    out = ops.prefix_attention(*dev, beam_width=W)
    torch.cuda.synchronize()
    assert_close_rel(out.cpu(), exp, rtol=1e-2, atol_frac=4e-3, name="d256 attention")


@pytest.mark.parametrize("Tk,Tq", [(5, 1), (7, 3), (3, 2)])
def test_prefix_attention_d256_query_offset_is_bitwise(device, Tk, Tq):
    """Queries that are the last Tq of Tk suffix tokens give, bit for bit, the
    last Tq rows of the full Tk-token call: a row's arithmetic does not depend
    on how many rows the launch holds (what the cached-suffix decode needs)."""
    from kadllm_amd.attention import prefix_attention_decode
    B, W, H, HK, L, D = 2, 6, 8, 2, 70, 256
    q, pk, pv, sk, sv = _attn_inputs(B, W, Tk, H, HK, L, D, seed=400 + Tk)
    gate = torch.randn(B * W, Tk, H * D, generator=torch.Generator().manual_seed(Tk)).bfloat16()
    qd, pkd, pvd, skd, svd, gd = (t.to(device) for t in (q, pk, pv, sk, sv, gate))
    full = prefix_attention_decode(qd, pkd, pvd, skd, svd, W, None, D ** -0.5, gate=gd)
    tail = prefix_attention_decode(qd[:, Tk - Tq:].contiguous(), pkd, pvd, skd, svd, W, None,
                                   D ** -0.5, gate=gd[:, Tk - Tq:].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(tail.cpu(), full[:, Tk - Tq:].cpu())


@pytest.mark.parametrize("B,L,H,HK,D", [(2, 100, 8, 2, 256), (1, 1024, 8, 2, 256), (2, 37, 4, 1, 64)])
def test_attention_prefill_causal(device, B, L, H, HK, D):
    g = torch.Generator().manual_seed(L)
    bf = torch.bfloat16
    q = torch.randn(B, L, H, D, generator=g).to(bf)
    kc = torch.randn(B, HK, L, D, generator=g).to(bf)        # cache layout [B,HK,L,D]
    vc = torch.randn(B, HK, L, D, generator=g).to(bf)
    gate = torch.randn(B, L, H * D, generator=g).to(bf)
    rep = H // HK
    s = q.double().transpose(1, 2) @ kc.double().repeat_interleave(rep, 1).transpose(-1, -2)
    s = s * D ** -0.5
    s = s.masked_fill(~torch.ones(L, L, dtype=torch.bool).tril(), -torch.inf)
    o = (s.softmax(-1) @ vc.double().repeat_interleave(rep, 1)).transpose(1, 2)   # [B,L,H,D]
    exp = o.to(bf).reshape(B, L, -1) * gate.sigmoid()
    qd, kd, vd, gd = q.to(device), kc.to(device), vc.to(device), gate.to(device)
    out = attention_prefill(qd, kd.transpose(1, 2), vd.transpose(1, 2), D ** -0.5, gate=gd,
                            gate_strides=(gd.stride(0), gd.stride(1), D))
    torch.cuda.synchronize()
    assert_close_rel(out.reshape(B, L, -1).cpu(), exp, rtol=1e-2, atol_frac=4e-3,
                     name="prefill attention")
