"""GPU: the attention module's FP8 route (flower_amd.attention.CausalSelfAttention with
attn_precision "fp8", the reference's CausalSelfAttention, flower/models/base.py:553-665, routed by
config.py:373) and the fused QK-norm + RoPE + e4m3 quantiser behind it, through the C ABI.

Gates (written here):
  - the fused quantiser's q', k' (the transform it applies before quantising) against the oracle's
    HeadRMSNorm + RoPE (oracle/block.py) on the same inputs: RoPE alone bit for bit; with the norm
    (whose mean of squares may differ in the last place, summation order) < 0.2 % of values differ,
    each by <= 2^-7 (|v| + 1) in bf16 (1e-6 (|v| + 1) in fp32) -- absolute against the row's unit
    RMS, since RoPE's sum can cancel a one-ulp input difference into many ulps of a small result;
  - its codes and scales bit-exact against the oracle's per_tensor_fp8 applied to its own q', k'
    and to v (V in the kernel's tile layout);
  - the module's attention output against the oracle's FP8 simulator on those codes:
    max|d|/max|ref| <= 2e-2, mean <= 5e-3 (the attention tests' gate);
  - the module output against the same module composed from torch's qkv_heads and
    fp8_swa_attention_forward (the reference's route): relative Frobenius < 2e-2, and against fp32
    attention of the unquantised heads: < 0.1 (the reference's own FP8 error is ~0.05).
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from gpu_util import rel_errors, to_np, vtile_permute
from oracle.block import head_rmsnorm, rope
from oracle.quant import per_tensor_fp8
from oracle.swa import fp8_swa_simulate, swa_banded

pytestmark = pytest.mark.gpu


def _ulp_bf16(a, b):
    from oracle.e4m3 import f32_to_bf16_bits
    ia = f32_to_bf16_bits(np.asarray(a, np.float32)).astype(np.int32)
    ib = f32_to_bf16_bits(np.asarray(b, np.float32)).astype(np.int32)
    return np.abs(ia - ib)


def _tables(T, D, dtype):
    from flower_amd.attention import RotaryEmbedding
    return RotaryEmbedding(D, T).tables(T, dtype, "cuda")


def _check_transform(got, want, dtype, normed):
    """RoPE alone is exact (every product and sum rounded as the oracle rounds them). After the
    norm, whose mean of squares may differ in the last place, a value may be off by one ulp and
    RoPE's sum can cancel, so the bound is absolute against the row's unit RMS."""
    if not normed:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        return
    d = np.abs(got.astype(np.float64) - want)
    if dtype == torch.bfloat16:
        bad = d > 0
        assert bad.mean() < 2e-3, bad.mean()
        assert (d <= 2.0 ** -7 * (np.abs(want) + 1.0)).all(), float(d.max())
    else:
        assert (d <= 1e-6 * (np.abs(want) + 1.0)).all(), float(d.max())


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("gran", ["head", "tensor", "bh"])
@pytest.mark.parametrize("qk_norm,use_rope", [(True, True), (False, True), (True, False)])
def test_fused_quantiser_against_oracle(qk_norm, use_rope, gran, dtype, D):
    """Every head_dim the entry point accepts: the HeadRMSNorm row sum is reduced over D / N lanes
    (4 / 8 / 16 lanes for bf16 at D = 32 / 64 / 128, 8 / 16 / 32 for fp32) and the RoPE tables are
    indexed per D, so each width is its own case."""
    from flower_amd.kernels import qk_norm_rope_quant_e4m3
    B, T, H = 2, 300, 4
    name = "bf16" if dtype == torch.bfloat16 else "f32"
    g = torch.Generator().manual_seed(71)
    scale = torch.randn(1, 1, 3 * H, 1, generator=g).exp()
    y = (torch.randn(B, T, 3 * H, D, generator=g) * scale).reshape(B, T, 3 * H * D).to(dtype).cuda()
    q, k, v = (t.view(B, T, H, D).transpose(1, 2) for t in y.chunk(3, dim=-1))     # strided views
    cos, sin = _tables(T, D, dtype) if use_rope else (None, None)
    q8, k8, vt, sc, qt, kt = qk_norm_rope_quant_e4m3(q, k, v, qk_norm=qk_norm, eps=1e-6, rope_cos=cos,
                                                     rope_sin=sin, granularity=gran, return_transformed=True)
    torch.cuda.synchronize()
    # the transform against the oracle on the same inputs
    for src, got in ((q, qt), (k, kt)):
        want = to_np(src.contiguous())
        if qk_norm:
            want = head_rmsnorm(want, 1e-6, name)
        if use_rope:
            want = rope(want, to_np(cos), to_np(sin), name)
        _check_transform(to_np(got), want, dtype, qk_norm)
    # the codes and scales on its own transformed values, bit for bit
    G = {"tensor": 1, "head": H, "bh": B * H}[gran]
    for i, (vals, codes, layout) in enumerate(((qt, q8, "bhtd"), (kt, k8, "bhtd"), (v, vt, "vtile"))):
        want_c, want_s = per_tensor_fp8(to_np(vals.contiguous()), gran)
        if layout == "vtile":
            want_c = vtile_permute(want_c)
        assert np.array_equal(to_np(codes).reshape(-1), want_c.reshape(-1)), i
        assert np.array_equal(to_np(sc[i * G:(i + 1) * G]).view(np.uint32),
                              np.asarray(want_s, np.float32).reshape(-1).view(np.uint32)), i


def test_fused_quantiser_without_transforms_equals_the_plain_qkv_quantiser():
    from flower_amd import _lib as L
    from flower_amd.kernels import qk_norm_rope_quant_e4m3
    lib = L.load()
    B, H, T, D = 1, 3, 200, 64
    q, k, v = ((torch.randn(B, H, T, D, generator=torch.Generator().manual_seed(s)) * (s + 1))
               .to(torch.bfloat16).cuda() for s in (1, 2, 3))
    q8, k8, vt, sc = qk_norm_rope_quant_e4m3(q, k, v, qk_norm=False, granularity="head")
    r8, rk8 = torch.empty_like(q8), torch.empty_like(k8)
    rvt, rsc = torch.empty_like(vt), torch.empty_like(sc)
    ws = L.workspace(3 * lib.flw_quant_workspace_bytes(B, H, T, D), q.device)
    L.check(lib.flw_quant_qkv_e4m3(q.data_ptr(), k.data_ptr(), v.data_ptr(), L.BF16, B, H, T, D,
                                   L.i64s(*q.stride()[:3], *k.stride()[:3], *v.stride()[:3]), L.SCALE_HEAD,
                                   r8.data_ptr(), rk8.data_ptr(), rvt.data_ptr(), rsc.data_ptr(), ws.data_ptr(),
                                   ws.numel(), L.stream_of(q)), "plain")
    torch.cuda.synchronize()
    for a, b in ((q8, r8), (k8, rk8), (vt, rvt), (sc.view(torch.int32), rsc.view(torch.int32))):
        assert torch.equal(a, b)


def _module(d_model, H, T, W, qk_norm=True, precision="fp8", seed=0):
    from flower_amd.attention import CausalSelfAttention
    cfg = SimpleNamespace(d_model=d_model, num_heads=H, max_seq_len=T, rope_base=10000.0, use_bias=False,
                          qk_norm=qk_norm, attn_precision=precision)
    m = CausalSelfAttention(cfg, local_window=W)
    g = torch.Generator().manual_seed(seed)
    for lin in (m.qkv, m.out):
        lin.weight.data.copy_(torch.randn(lin.weight.shape, generator=g) * 0.02)
    return m.to("cuda", torch.bfloat16)


def test_module_fp8_route_at_the_reference_measurement_shape():
    """The FP8 route of the attention module with QK-norm on, at the reference's FP8 measurement
    shape (B1 H20 T4096 D64 W2048, the 450M model's heads): stage by stage as in the header."""
    B, T, H, D, W = 1, 4096, 20, 64, 2048
    d = H * D
    m = _module(d, H, T, W, seed=72)
    x = torch.randn(B, T, d, generator=torch.Generator().manual_seed(73)).to("cuda", torch.bfloat16)
    tr = {}
    with torch.no_grad():
        out = m(x, trace=tr)
        unfused = m.forward_unfused(x)
    torch.cuda.synchronize()
    # the transform on the module's own projection
    cos, sin = m.rope.tables(T, torch.bfloat16, "cuda")
    q, k, v = (m._split(t) for t in tr["qkv"].chunk(3, dim=-1))
    for src, got in ((q, tr["q"]), (k, tr["k"])):
        want = rope(head_rmsnorm(to_np(src.contiguous()), m.qk_norm.eps, "bf16"), to_np(cos), to_np(sin), "bf16")
        _check_transform(to_np(got), want, torch.bfloat16, True)
    # codes bit-exact on its own q', k', v
    codes = [per_tensor_fp8(to_np(t.contiguous()), "head") for t in (tr["q"], tr["k"], v)]
    assert np.array_equal(to_np(tr["q8"]), codes[0][0]) and np.array_equal(to_np(tr["k8"]), codes[1][0])
    assert np.array_equal(to_np(tr["v_tiles"]), vtile_permute(codes[2][0]))
    # attention against the simulator on those codes, two heads
    attn = to_np(tr["attn"].view(B, T, H, D).transpose(1, 2))
    for h in (0, 13):
        sl = slice(h, h + 1)
        ref = fp8_swa_simulate(codes[0][0][:, sl], codes[1][0][:, sl], codes[2][0][:, sl], codes[0][1][:, sl],
                               codes[1][1][:, sl], codes[2][1][:, sl], W, chunk=1024)
        mx, mean = rel_errors(attn[:, sl], ref)
        assert mx <= 2e-2 and mean <= 5e-3, (h, mx, mean)
    # the whole module against the reference's composition and against fp32 attention
    rel_u = float((out.float() - unfused.float()).norm() / unfused.float().norm())
    assert rel_u < 2e-2, rel_u
    with torch.no_grad():
        qh, kh, vh = (t.float() for t in m.qkv_heads(x))
        ref32 = torch.from_numpy(swa_banded(to_np(qh[:, :4]), to_np(kh[:, :4]), to_np(vh[:, :4]), W, chunk=512))
    got4 = tr["attn"].view(B, T, H, D)[:, :, :4].transpose(1, 2).float().cpu()
    rel32 = float((got4 - ref32).norm() / ref32.norm())
    print(f"[model] fused vs unfused {rel_u:.2e}; attention (4 heads) vs fp32 {rel32:.3f}")
    assert rel32 < 0.1
    assert torch.isfinite(out).all()


def test_module_fp8_route_trains_through_the_differentiable_fp8_attention():
    """With gradients needed the FP8 route is qkv_heads in torch + fp8_swa_attention: its output
    equals the inference route's (the fused HIP QK-norm + RoPE) to the transform's last-place
    differences, and gradients reach the projection weights through the FP8 attention's backward
    (against the same loss through the differentiable bf16 route on the same module, the
    reference's FP8 error band: relative Frobenius < 0.15)."""
    m = _module(256, 4, 128, 64, seed=74)
    x = torch.randn(1, 128, 256, generator=torch.Generator().manual_seed(75)).to("cuda", torch.bfloat16)
    y = m(x)
    assert y.requires_grad
    with torch.no_grad():
        y_inf = m(x)
    rel = float((y.detach().float() - y_inf.float()).norm() / y_inf.float().norm())
    assert rel < 1e-2, rel
    y.float().square().mean().backward()
    g_fp8 = m.qkv.weight.grad.detach().float().clone()
    assert torch.isfinite(g_fp8).all() and g_fp8.abs().sum() > 0
    m.zero_grad()
    m.attn_precision = "bf16"
    m(x).float().square().mean().backward()
    g_bf16 = m.qkv.weight.grad.detach().float()
    rel_g = float((g_fp8 - g_bf16).norm() / g_bf16.norm())
    print(f"[model] fp8 route qkv weight grad vs the bf16 route: {rel_g:.3f}")
    assert rel_g < 0.15, rel_g


def test_module_bf16_route_trains_through_the_hip_kernel():
    """attn_precision "bf16": qkv_heads in torch, then the HIP bf16 sliding-window kernel; the
    output against float64 attention of the same heads (the bf16 kernel's gates), and gradients
    reach the projection weights."""
    from oracle.swa import swa_dense
    B, T, H, D, W = 1, 256, 4, 64, 100
    m = _module(H * D, H, T, W, qk_norm=True, precision="bf16", seed=75)
    x = torch.randn(B, T, H * D, generator=torch.Generator().manual_seed(76)).to("cuda", torch.bfloat16)
    y = m(x)
    y.float().square().mean().backward()
    assert m.qkv.weight.grad is not None and torch.isfinite(m.qkv.weight.grad).all()
    with torch.no_grad():
        q, k, v = m.qkv_heads(x)
        from flower_amd.kernels.swa_attention import swa_attention
        a = swa_attention(q, k, v, W)
    ref = swa_dense(*(t.double().cpu().numpy() for t in (q, k, v)), W)
    mx, mean = rel_errors(to_np(a), ref)
    assert mean < 0.01 and mx < 2e-2, (mx, mean)


def test_fp8_attention_helper_on_normed_rotated_heads():
    """fp8_attention (the FP8 route on heads that are already normed and rotated) equals
    fp8_swa_attention_forward with the same window, and local_window=None means full causal."""
    from flower_amd.attention import fp8_attention
    from flower_amd.kernels import fp8_swa_attention_forward
    q, k, v = (torch.randn(1, 2, 192, 64, generator=torch.Generator().manual_seed(s)).to("cuda", torch.bfloat16)
               for s in (77, 78, 79))
    a = fp8_attention(q, k, v, 64)
    b = fp8_swa_attention_forward(q, k, v, 64, granularity="head")
    c = fp8_attention(q, k, v, None)
    d = fp8_swa_attention_forward(q, k, v, 192, granularity="head")
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(c, d)
