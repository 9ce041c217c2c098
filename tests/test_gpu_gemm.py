"""GPU parity: FP8 GEMM and the FP8 weight cache (C ABI via flower_amd) vs the CPU oracle.

Gate: against the float64 closed form on the same e4m3 codes and scales, every output within
one bf16 rounding step plus fp32-accumulation slack: |d| <= 2^-7 * |ref| + 1e-3 * rms(ref).
"""

import numpy as np
import pytest
import torch
import torch.nn as nn

from gpu_util import seeded, to_np
from oracle.gemm import fp8_linear_a8w8, scaled_mm
from oracle.quant import rowwise_fp8

pytestmark = pytest.mark.gpu


def assert_gemm_close(got, ref):
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    tol = 2.0 ** -7 * np.abs(ref) + 1e-3 * np.sqrt(np.mean(ref ** 2))
    bad = np.abs(got - ref) > tol
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside tolerance; max |d| {np.abs(got - ref).max()}"


def codes(shape, seed):
    """Random finite e4m3 codes (no NaN)."""
    c = np.random.default_rng(seed).integers(0, 256, size=shape, dtype=np.uint8)
    c[(c & 0x7F) == 0x7F] = 0x38
    return c


@pytest.mark.parametrize("M,N,K", [(128, 256, 512), (100, 36, 80), (257, 132, 1040), (1, 16, 16),
                                   (300, 132, 256), (1, 20, 128), (513, 260, 1024), (256, 512, 384),
                                   (5120, 3328, 128), (4900, 1280, 320)])
@pytest.mark.parametrize("sx_per_row,sw_per_col", [(True, True), (False, False), (True, False)])
def test_scaled_mm_matches_closed_form(M, N, K, sx_per_row, sw_per_col):
    """The 256-tile kernel against the closed form: small and ragged shapes, and outputs with more
    256 x 256 tiles than compute units whose last round the 256 x 128 tiles fill better (260 tiles;
    a ragged 100 with K % 128 == 64)."""
    from flower_amd import _lib as L
    lb = L.load()
    x8, w8 = codes((M, K), 1), codes((N, K), 2)
    rng = np.random.default_rng(3)
    sx = rng.uniform(0.001, 0.01, M if sx_per_row else 1).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N if sw_per_col else 1).astype(np.float32)
    tx8, tw8 = torch.from_numpy(x8).cuda(), torch.from_numpy(w8).cuda()
    tsx, tsw = torch.from_numpy(sx).cuda(), torch.from_numpy(sw).cuda()
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    L.check(lb.flw_fp8_scaled_mm(tx8.data_ptr(), M, K, tw8.data_ptr(), N, tsx.data_ptr(), sx.size,
                                 tsw.data_ptr(), sw.size, y.data_ptr(), N, L.stream_of(y)), "scaled_mm")
    ref = scaled_mm(x8, w8, np.broadcast_to(sx, (M,)), np.broadcast_to(sw, (N,)))
    assert_gemm_close(to_np(y), ref)


@pytest.mark.parametrize("M,N,K", [(256, 256, 4096), (512, 1024, 2048), (4096, 1024, 8192), (300, 260, 1024),
                                   (100, 36, 80), (256, 256, 4160), (4096, 1024, 3392), (1024, 512, 192),
                                   (300, 260, 320), (3840, 1280, 1536), (2560, 1280, 2560)])
def test_scaled_mm_split_k_matches_closed_form(M, N, K):
    """flw_fp8_scaled_mm_ws: outputs with few 256 x 256 tiles are split over K into the workspace
    (1 tile -> 8 ranges, 8 tiles -> 4, the C2 wgrad shape 64 tiles -> 4; an even split runs on
    256 x 128 tiles with half the ranges, an odd one -- 75 tiles -> 3, 50 -> 5 -- on 256 x 256
    tiles) and summed by the finish kernel; shapes without a split (K % 64 != 0) take the plain
    path through the same call.
    K % 128 == 64 (the SwiGLU width 3392 of the 450M block among them) ends the last K range on a
    64-deep stage, in the 256 x 256 and the 256 x 128 tiles, split or not. Against the closed
    form, and equal to the unsplit call within the GEMM tolerance."""
    from flower_amd import _lib as L
    lb = L.load()
    x8, w8 = codes((M, K), 4), codes((N, K), 5)
    rng = np.random.default_rng(6)
    sx = rng.uniform(0.001, 0.01, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32)
    tx8, tw8 = torch.from_numpy(x8).cuda(), torch.from_numpy(w8).cuda()
    tsx, tsw = torch.from_numpy(sx).cuda(), torch.from_numpy(sw).cuda()
    need = lb.flw_fp8_scaled_mm_workspace_bytes(M, N, K)
    if K % 64 == 0 and K >= 512 and M * N <= 8 * 256 * 256:
        assert need > 0
    ws = L.workspace(need, "cuda")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    L.check(lb.flw_fp8_scaled_mm_ws(tx8.data_ptr(), M, K, tw8.data_ptr(), N, tsx.data_ptr(), M, tsw.data_ptr(),
                                    N, y.data_ptr(), N, ws.data_ptr(), ws.numel(), L.stream_of(y)), "mm_ws")
    ref = scaled_mm(x8, w8, sx, sw)
    assert_gemm_close(to_np(y), ref)
    y1 = torch.empty_like(y)
    L.check(lb.flw_fp8_scaled_mm(tx8.data_ptr(), M, K, tw8.data_ptr(), N, tsx.data_ptr(), M, tsw.data_ptr(), N,
                                 y1.data_ptr(), N, L.stream_of(y)), "mm")
    assert_gemm_close(to_np(y), to_np(y1).astype(np.float64))


def test_config2_fp8_linear_full_size():
    """W [4096 x 1024] ~ N(0, 0.02) bf16 per-channel e4m3; X [8192 x 1024]
    ~ N(0, 1) bf16 with 0.1% outliers x20; A8W8 output checked on sampled rows against the
    closed form, activation codes bit-exact."""
    from flower_amd.precision import fp8_linear_forward, quantize_weight
    g = torch.Generator().manual_seed(7)
    W = (torch.randn(4096, 1024, generator=g) * 0.02).to(torch.bfloat16)
    X = torch.randn(8192, 1024, generator=g)
    idx = torch.randperm(X.numel(), generator=g)[: X.numel() // 1000]
    X.view(-1)[idx] *= 20
    X = X.to(torch.bfloat16)
    w8, ws = quantize_weight(W.cuda(), "rowwise")
    want_w8, want_ws = rowwise_fp8(W.float().numpy())
    np.testing.assert_array_equal(to_np(w8), want_w8)
    np.testing.assert_array_equal(to_np(ws), want_ws.reshape(-1))
    y = to_np(fp8_linear_forward(X.cuda(), w8, ws))
    rows = np.random.default_rng(0).choice(8192, 256, replace=False)
    ref, _, _ = fp8_linear_a8w8(X.float().numpy()[rows], want_w8, want_ws.reshape(-1))
    assert_gemm_close(y[rows], ref)
    # vs the unquantised bf16 product: the reference's FP8-head acceptance bounds
    # (tests/test_training_speedups.py:375-389)
    full = (X.float().numpy()[rows] @ W.float().numpy().T)
    rel = np.linalg.norm(y[rows] - full) / np.linalg.norm(full)
    assert rel < 0.05 and 0.9 < np.linalg.norm(y[rows]) / np.linalg.norm(full) < 1.1, rel


@pytest.mark.parametrize("M,N,K", [(128, 256, 512), (100, 36, 64), (257, 132, 1024), (1, 16, 64),
                                   (513, 260, 1088), (256, 512, 384)])
@pytest.mark.parametrize("per_channel", [True, False])
def test_w8a16_matches_closed_form(M, N, K, per_channel):
    """FLW_GEMM_W8A16: bf16 activations (with x20 outliers) times widened e4m3 weights, against
    the float64 closed form on the same values; a strided x (row stride K + 64) as well."""
    from flower_amd import _lib as L
    from oracle.gemm import fp8_linear_w8a16
    lb = L.load()
    w8 = codes((N, K), 4)
    g = torch.Generator().manual_seed(5)
    xs = K + 64
    xbuf = (torch.randn(M, xs, generator=g) * 2).to(torch.bfloat16)
    xbuf.view(-1)[::997] *= 20
    x = xbuf[:, :K]
    sw = np.random.default_rng(6).uniform(0.001, 0.01, N if per_channel else 1).astype(np.float32)
    tw8, tsw, tx = torch.from_numpy(w8).cuda(), torch.from_numpy(sw).cuda(), xbuf.cuda()
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    L.check(lb.flw_fp8_linear(tx.data_ptr(), M, K, xs, tw8.data_ptr(), N, tsw.data_ptr(), sw.size,
                              L.GEMM_W8A16, y.data_ptr(), N, None, 0, L.stream_of(y)), "w8a16")
    ref = fp8_linear_w8a16(x.float().numpy(), w8, np.broadcast_to(sw, (N,)))
    assert_gemm_close(to_np(y), ref)


def test_w8a16_rejects_unsupported_k():
    from flower_amd import _lib as L
    lb = L.load()
    t = torch.empty(4096, dtype=torch.uint8, device="cuda")
    rc = lb.flw_fp8_linear(t.data_ptr(), 16, 80, 80, t.data_ptr(), 16, t.data_ptr(), 1, L.GEMM_W8A16,
                           t.data_ptr(), 16, None, 0, None)
    assert rc == 2 and b"multiple of 64" in lb.flw_last_error()


def test_config2_weight_only_full_size():
    """BASELINE config 2 in weight-only mode: the cached per-channel e4m3 weight times the bf16
    activations with their outliers, sampled rows against the closed form and the unquantised
    product within the reference's FP8-head bounds."""
    from flower_amd.precision import fp8_linear_forward, quantize_weight
    from oracle.gemm import fp8_linear_w8a16
    g = torch.Generator().manual_seed(7)
    W = (torch.randn(4096, 1024, generator=g) * 0.02).to(torch.bfloat16)
    X = torch.randn(8192, 1024, generator=g)
    idx = torch.randperm(X.numel(), generator=g)[: X.numel() // 1000]
    X.view(-1)[idx] *= 20
    X = X.to(torch.bfloat16)
    w8, ws = quantize_weight(W.cuda(), "weight_only")
    y = to_np(fp8_linear_forward(X.cuda(), w8, ws, "weight_only"))
    rows = np.random.default_rng(1).choice(8192, 256, replace=False)
    ref = fp8_linear_w8a16(X.float().numpy()[rows], to_np(w8), to_np(ws))
    assert_gemm_close(y[rows], ref)
    full = X.float().numpy()[rows] @ W.float().numpy().T
    rel = np.linalg.norm(y[rows] - full) / np.linalg.norm(full)
    assert rel < 0.05 and 0.9 < np.linalg.norm(y[rows]) / np.linalg.norm(full) < 1.1, rel


def test_fp8_linear_module_matches_bf16_linear_and_backprops():
    from flower_amd.precision import Fp8Linear
    torch.manual_seed(0)
    lin = nn.Linear(256, 512, bias=True).cuda().to(torch.bfloat16)
    f8 = Fp8Linear.from_linear(lin)
    x = torch.randn(4, 32, 256, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    y = f8(x)
    ref = lin(x.detach())
    rel = ((y.float() - ref.float()).norm() / ref.float().norm()).item()
    assert y.shape == (4, 32, 512) and y.dtype == torch.bfloat16 and rel < 0.05, rel
    y.float().square().mean().backward()
    assert x.grad is not None and lin.weight.grad is not None and torch.isfinite(x.grad).all()


# ---------------------------------------------------------------- fp8_weight_cache (test_fp8_weight_cache.py)

def _fp8_model(d: int = 256, hid: int = 512) -> nn.Module:
    from flower_amd.precision import Fp8Linear
    torch.manual_seed(0)
    m = nn.Sequential(nn.Linear(d, hid, bias=False), nn.Linear(hid, d, bias=False))
    m = m.cuda().to(torch.bfloat16)
    return nn.Sequential(*(Fp8Linear.from_linear(l) for l in m))


@pytest.mark.parametrize("recipe", ["rowwise", "tensorwise", "weight_only"])
def test_cached_is_bit_identical_to_uncached(recipe):
    from flower_amd.precision import fp8_weight_cache
    accum = 3
    xs = [torch.randn(128, 256, device="cuda", dtype=torch.bfloat16) for _ in range(accum)]

    def run(use_cache: bool):
        m = _fp8_model()
        for mod in m:
            mod.recipe = recipe
        opt = torch.optim.SGD(m.parameters(), lr=0.01)
        for _ in range(2):
            opt.zero_grad(set_to_none=True)
            if use_cache:
                with fp8_weight_cache(m):
                    for x in xs:
                        m(x).float().square().mean().backward()
            else:
                for x in xs:
                    m(x).float().square().mean().backward()
            opt.step()
        return [p.detach().float().clone() for p in m.parameters()]

    for a, b in zip(run(False), run(True)):
        assert torch.equal(a, b), "cached path diverged from uncached"


def test_raises_when_a_weight_changes_while_cache_is_live():
    from flower_amd.precision import fp8_weight_cache
    m = _fp8_model()
    x = torch.randn(128, 256, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="stale"):
        with fp8_weight_cache(m):
            m(x).float().sum().backward()
            with torch.no_grad():
                m[0].weight.data -= 0.1
            m(x).float().sum().backward()


def test_forwards_are_restored_after_exit_and_after_exception():
    from flower_amd.precision import fp8_weight_cache
    m = _fp8_model()
    before = [mod.forward for mod in m]
    with fp8_weight_cache(m):
        pass
    assert all(mod.forward == orig for mod, orig in zip(m, before))
    with pytest.raises(ValueError):
        with fp8_weight_cache(m):
            raise ValueError("boom")
    assert all(mod.forward == orig for mod, orig in zip(m, before))


def test_cache_uses_one_quantisation_per_enter():
    """Inside the cache the layer must not re-quantise its weight on each microstep (counted: the
    plain weight cast, and the training forward's cast in both layouts when it quantises afresh)."""
    from flower_amd.precision import Fp8Linear, fp8_weight_cache
    m = _fp8_model()
    calls = {"n": 0}
    orig, orig_t = Fp8Linear.quantize_weight, Fp8Linear.tensorwise_codes

    def counting(self):
        calls["n"] += 1
        return orig(self)

    def counting_t(self):
        cached = getattr(self, "_fp8_cached", None) is not None
        out = orig_t(self)
        calls["n"] += 0 if cached else 1
        return out

    Fp8Linear.quantize_weight = counting
    Fp8Linear.tensorwise_codes = counting_t
    try:
        x = torch.randn(64, 256, device="cuda", dtype=torch.bfloat16)
        with fp8_weight_cache(m):
            for _ in range(4):
                m(x)
        assert calls["n"] == 2
        m(x)
        assert calls["n"] == 4
    finally:
        Fp8Linear.quantize_weight = orig
        Fp8Linear.tensorwise_codes = orig_t



# ---------------------------------------------------------------- FP8 LM head (base.py:865-924)

@pytest.mark.parametrize("shift", [0.0, -2.5])
def test_fp8_lm_head_matches_bf16_head(shift):
    """fp8_head vs the bf16 head on a tied-embedding-shaped weight (vocab 16384, d 1024): the
    reference's bounds (test_training_speedups.py:359-412: relative Frobenius < 0.05, norm ratio in
    (0.9, 1.1), next-token CE within 0.1; the -2.5 shift is its all-negative-rows regression),
    and sampled rows against the oracle's closed form on the same codes."""
    from flower_amd.precision import compute_logits, fp8_head
    from oracle.quant import rowwise_fp8
    torch.manual_seed(0)
    vocab, d, B, T = 16384, 1024, 2, 64
    head = nn.Linear(d, vocab, bias=False).cuda().to(torch.bfloat16)
    with torch.no_grad():
        head.weight.normal_(0.0, 0.02)
    x = (torch.randn(B, T, d, device="cuda") + shift).to(torch.bfloat16)
    with torch.no_grad():
        fp8 = fp8_head(x, head.weight).float()
        ref = head(x).float()
        routed = compute_logits(head, x, fp8_lm_head=True, training=False).float()
        train = compute_logits(head, x, fp8_lm_head=True, training=True).float()
    assert fp8.shape == (B, T, vocab) and torch.equal(routed, fp8) and torch.equal(train, ref)
    rel = ((fp8 - ref).norm() / ref.norm()).item()
    assert rel < 0.05 and 0.9 < (fp8.norm() / ref.norm()).item() < 1.1, rel
    labels = torch.randint(0, vocab, (B, T - 1), device="cuda")
    ce = lambda lg: torch.nn.functional.cross_entropy(lg[:, :-1].reshape(-1, vocab), labels.reshape(-1))
    assert abs(ce(fp8).item() - ce(ref).item()) < 0.1
    w8, sw = rowwise_fp8(head.weight.detach().float().cpu().numpy())
    xs = x.reshape(-1, d).float().cpu().numpy()[:16]
    want, _, _ = fp8_linear_a8w8(xs, w8, sw.reshape(-1))
    assert_gemm_close(to_np(fp8.reshape(-1, vocab)[:16]), want)


@pytest.mark.parametrize("M,N,K", [(512, 1024, 1024), (300, 260, 128), (100, 36, 80), (512, 1024, 320)])
def test_scaled_mm_residual_epilogue(M, N, K):
    """flw_fp8_scaled_mm_residual: y = bf16(residual + bf16(scaled product)), against the closed
    form with both roundings; the 256-tile kernel (K % 64 == 0; 320 ends on a 64-deep stage) and
    the general one."""
    from flower_amd import _lib as L
    from oracle.e4m3 import round_bf16
    lb = L.load()
    x8, w8 = codes((M, K), 11), codes((N, K), 12)
    rng = np.random.default_rng(13)
    sx = rng.uniform(0.001, 0.01, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32)
    res = torch.randn(M, N + 4, generator=torch.Generator().manual_seed(14)).to(torch.bfloat16)
    tx8, tw8, tsx, tsw = (torch.from_numpy(a).cuda() for a in (x8, w8, sx, sw))
    tres = res.cuda()
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    L.check(lb.flw_fp8_scaled_mm_residual(tx8.data_ptr(), M, K, tw8.data_ptr(), N, tsx.data_ptr(), M,
                                          tsw.data_ptr(), N, y.data_ptr(), N, tres.data_ptr(), N + 4,
                                          L.stream_of(y)), "residual")
    prod = round_bf16(scaled_mm(x8, w8, sx, sw))
    ref = round_bf16((prod + res[:, :N].float().numpy()).astype(np.float32))
    got = to_np(y).astype(np.float64)
    # the product may differ from the closed form by one bf16 step (accumulation order), which the
    # add carries into the sum, where it can flip the final rounding by one step
    tol = 2.0 ** -7 * np.abs(prod) + 2.0 ** -7 * np.abs(ref) + 1e-3 * np.sqrt(np.mean(prod.astype(np.float64) ** 2))
    bad = np.abs(got - ref) > tol
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside tolerance"
    assert (got == ref).mean() > 0.95


@pytest.mark.parametrize("M,N,K,gcols", [(300, 768, 256, 64), (1024, 3072, 1024, 64), (513, 512, 128, 8),
                                         (256, 1024, 384, 256), (64, 192, 128, 64), (300, 768, 320, 64)])
def test_group_amax_epilogue(M, N, K, gcols):
    """flw_fp8_scaled_mm_group_amax: y identical to flw_fp8_scaled_mm's, and amax_out[g] equal to
    max |y[:, g*gcols:(g+1)*gcols]| over all rows (fp32 bit pattern of the bf16 maximum), called
    twice on one buffer (the call clears it itself)."""
    from flower_amd import _lib as L
    lb = L.load()
    x8, w8 = codes((M, K), 11), codes((N, K), 12)
    rng = np.random.default_rng(13)
    sx = rng.uniform(0.001, 0.01, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32)
    tx8, tw8 = torch.from_numpy(x8).cuda(), torch.from_numpy(w8).cuda()
    tsx, tsw = torch.from_numpy(sx).cuda(), torch.from_numpy(sw).cuda()
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    y0 = torch.empty_like(y)
    amax = torch.full((N // gcols,), -1, dtype=torch.int32, device="cuda")
    for _ in range(2):
        L.check(lb.flw_fp8_scaled_mm_group_amax(tx8.data_ptr(), M, K, tw8.data_ptr(), N, tsx.data_ptr(), M,
                                                tsw.data_ptr(), N, y.data_ptr(), N, gcols, amax.data_ptr(),
                                                L.stream_of(y)), "group amax")
    L.check(lb.flw_fp8_scaled_mm(tx8.data_ptr(), M, K, tw8.data_ptr(), N, tsx.data_ptr(), M, tsw.data_ptr(), N,
                                 y0.data_ptr(), N, L.stream_of(y)), "mm")
    assert torch.equal(y, y0)
    want = y.float().abs().reshape(M, N // gcols, gcols).amax(dim=(0, 2)).view(torch.int32)
    assert torch.equal(amax, want)


def test_group_amax_rejects_bad_groups():
    from flower_amd import _lib as L
    lb = L.load()
    t = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    s = torch.ones(1024, device="cuda")
    p = t.data_ptr()
    rc = lb.flw_fp8_scaled_mm_group_amax(p, 128, 128, p, 96, s.data_ptr(), 128, s.data_ptr(), 96, p, 96, 48, p,
                                         L.stream_of(t))
    assert rc == 1 and b"power of two" in lb.flw_last_error()
    rc = lb.flw_fp8_scaled_mm_group_amax(p, 128, 80, p, 128, s.data_ptr(), 128, s.data_ptr(), 128, p, 128, 64, p,
                                         L.stream_of(t))
    assert rc == 2 and b"K %" in lb.flw_last_error()


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("qk_norm,use_rope", [(True, True), (False, True), (True, False)])
def test_qk_norm_rope_amax_epilogue(D, qk_norm, use_rope):
    """flw_fp8_scaled_mm_qk_norm_rope_amax: the QKV projection with qkv_heads' HeadRMSNorm and RoPE
    (flower/models/base.py:618-639) applied to the q / k columns in the epilogue. Against the plain
    GEMM y0 on the same codes: the v columns bit for bit; q', k' bit for bit against the Q / K / V
    quantiser's transform of y0's heads (flw_qk_norm_rope_quant_e4m3, the same arithmetic), and
    within the fused-quantiser tests' bounds of the oracle's HeadRMSNorm + RoPE of y0; the maxima
    those of q', k', v. B2 T300: M = 600 (a partial last row tile, positions wrapping at the batch
    boundary); called twice on one amax buffer."""
    from flower_amd import _lib as L
    from flower_amd.attention import RotaryEmbedding
    from flower_amd.kernels import qk_norm_rope_quant_e4m3
    from oracle.block import head_rmsnorm, rope
    lb = L.load()
    B, T, H, K = 2, 300, 4, 256
    M, d = B * T, H * D
    N = 3 * d
    x8, w8 = codes((M, K), 21), codes((N, K), 22)
    rng = np.random.default_rng(23)
    sx = rng.uniform(0.001, 0.01, M).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, N).astype(np.float32) * np.repeat(rng.lognormal(0, 1, 3 * H), D).astype(np.float32)
    tx8, tw8 = torch.from_numpy(x8).cuda(), torch.from_numpy(w8).cuda()
    tsx, tsw = torch.from_numpy(sx).cuda(), torch.from_numpy(sw).cuda()
    cos, sin = RotaryEmbedding(D, T).tables(T, torch.bfloat16, "cuda") if use_rope else (None, None)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    y0 = torch.empty_like(y)
    amax = torch.full((3 * H,), -1, dtype=torch.int32, device="cuda")
    for _ in range(2):
        L.check(lb.flw_fp8_scaled_mm_qk_norm_rope_amax(tx8.data_ptr(), M, K, tw8.data_ptr(), N, tsx.data_ptr(), M,
                                                       tsw.data_ptr(), N, y.data_ptr(), N, D, 2 * d, int(qk_norm),
                                                       1e-6, L.ptr(cos), L.ptr(sin), T, amax.data_ptr(),
                                                       L.stream_of(y)), "qkv epilogue")
    L.check(lb.flw_fp8_scaled_mm(tx8.data_ptr(), M, K, tw8.data_ptr(), N, tsx.data_ptr(), M, tsw.data_ptr(), N,
                                 y0.data_ptr(), N, L.stream_of(y)), "mm")
    torch.cuda.synchronize()
    assert torch.equal(y[:, 2 * d:], y0[:, 2 * d:])
    split = lambda t: t.view(B, T, H, D).transpose(1, 2)          # noqa: E731
    q0, k0, v0 = (split(t) for t in y0.chunk(3, dim=-1))
    _, _, _, _, qt, kt = qk_norm_rope_quant_e4m3(q0, k0, v0, qk_norm=qk_norm, eps=1e-6, rope_cos=cos, rope_sin=sin,
                                                 granularity="head", return_transformed=True)
    q1, k1, _ = (split(t) for t in y.chunk(3, dim=-1))
    assert torch.equal(q1.contiguous(), qt) and torch.equal(k1.contiguous(), kt)
    for raw, got in ((q0, q1), (k0, k1)):
        want = raw.float().cpu().numpy()
        if qk_norm:
            want = head_rmsnorm(want, 1e-6, "bf16")
        if use_rope:
            want = rope(want, cos.float().cpu().numpy(), sin.float().cpu().numpy(), "bf16")
        g = got.float().cpu().numpy()
        dd = np.abs(g.astype(np.float64) - want)
        if qk_norm:
            assert (dd > 0).mean() < 2e-3 and (dd <= 2.0 ** -7 * (np.abs(want) + 1.0)).all(), float(dd.max())
        else:
            assert np.array_equal(g.view(np.uint32), want.view(np.uint32))
    want_amax = y.float().abs().reshape(M, 3 * H, D).amax(dim=(0, 2)).view(torch.int32)
    assert torch.equal(amax, want_amax)
