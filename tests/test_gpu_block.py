"""GPU: the FP8 decoder block of BASELINE config 5 (flower_amd/block.py), composed from the
C-ABI kernels, against the same block in plain fp32 torch (the reference's TransformerBlock maths,
base.py:698-722, with the attention's HeadRMSNorm and RoPE of qkv_heads, base.py:618-639) and, for
the attention stage, against the CPU oracle.

Gates (written here; FP8 e4m3 is far coarser than the fp32 reference):
  - block update delta = out - x vs fp32: Frobenius relative error < 0.1 (each FP8 linear adds
    ~2-3 %, FP8 attention ~5 %: the reference's own FP8 attention error, fp8_swa_attention.py:48-57);
  - the attention stage on the block's own strided Q/K/V views vs the oracle's FP8 simulator on
    the same e4m3 codes: max|d|/max|ref| <= 2e-2, mean <= 5e-3;
  - inside fp8_weight_cache the block output is bit-identical to the uncached one.
"""

import numpy as np
import pytest
import torch

from gpu_util import rel_errors, to_np, vtile_permute
from oracle.quant import per_tensor_fp8
from oracle.swa import fp8_swa_simulate

pytestmark = pytest.mark.gpu

CFG = dict(d_model=256, num_heads=4, ffn_dim=1024, local_window=64)


def make_block(seed=0):
    from flower_amd.block import Fp8DecoderBlock, init_block_
    blk = Fp8DecoderBlock(**CFG)
    init_block_(blk, std=0.02, seed=seed)
    return blk.to("cuda", torch.bfloat16)


def fp32_reference(blk, x):
    """The same block in fp32 torch: RMSNorm, qkv, HeadRMSNorm of q and k, RoPE (fp32 tables),
    masked softmax attention, out, GELU MLP."""
    def rms(mod, t):
        return t * t.pow(2).mean(-1, keepdim=True).add(mod.eps).rsqrt() * mod.weight.float()
    B, T, d = x.shape
    H, D, W = CFG["num_heads"], d // CFG["num_heads"], CFG["local_window"]
    x = x.float()
    h = rms(blk.ln1, x)
    q, k, v = (h @ blk.attn.qkv.weight.float().t()).chunk(3, dim=-1)
    q, k, v = (t.reshape(B, T, H, D).transpose(1, 2).contiguous() for t in (q, k, v))
    q, k = (t * t.pow(2).mean(-1, keepdim=True).add(blk.attn.qk_norm.eps).rsqrt() for t in (q, k))
    cos, sin = (t.to(x.device) for t in blk.attn.rope._tables(T))

    def rot(t):
        return torch.stack((-t[..., 1::2], t[..., ::2]), dim=-1).flatten(-2)
    q, k = q * cos + rot(q) * sin, k * cos + rot(k) * sin
    s = (q @ k.transpose(-1, -2).contiguous()) / D ** 0.5
    i = torch.arange(T, device=x.device)
    keep = (i[:, None] >= i[None, :]) & ((i[:, None] - i[None, :]) < W)
    a = torch.softmax(s.masked_fill(~keep, float("-inf")), -1) @ v
    x = x + a.transpose(1, 2).reshape(B, T, d) @ blk.attn.out.weight.float().t()
    h = rms(blk.ln2, x)
    f = torch.nn.functional.gelu(h @ blk.ff.net[0].weight.float().t())
    return x + f @ blk.ff.net[3].weight.float().t()


@pytest.mark.parametrize("B,T", [(2, 384), (1, 200)])
def test_block_matches_fp32_reference(B, T):
    blk = make_block()
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, T, CFG["d_model"], generator=g).to("cuda", torch.bfloat16)
    out = blk(x)
    torch.cuda.synchronize()
    assert out.shape == x.shape and out.dtype == torch.bfloat16
    ref = fp32_reference(blk, x)
    delta, ref_delta = (out.float() - x.float()), (ref - x.float())
    rel = float((delta - ref_delta).norm() / ref_delta.norm())
    print(f"block delta Frobenius rel error vs fp32: {rel:.4f}")
    assert rel < 0.1


def test_block_attention_stage_matches_oracle():
    blk = make_block(seed=3)
    g = torch.Generator().manual_seed(2)
    B, T = 1, 256
    x = torch.randn(B, T, CFG["d_model"], generator=g).to("cuda", torch.bfloat16)
    from flower_amd.kernels.fp8_swa_attention import fp8_swa_attention_forward
    with torch.no_grad():
        q, k, v = blk.attn.qkv_heads(blk.ln1(x))      # QK-norm and RoPE (base.py:618-639)
        vt = torch.empty(B, T, v.shape[1], v.shape[3], dtype=v.dtype, device=v.device).transpose(1, 2)
        v = vt.copy_(v)                                  # the head split's (B, T, H, D) layout:
        assert not v.is_contiguous()                     # read in place through its strides
        out = fp8_swa_attention_forward(q, k, v, CFG["local_window"], granularity="head")
    torch.cuda.synchronize()
    codes = [per_tensor_fp8(to_np(t.contiguous()), "head") for t in (q, k, v)]
    ref = fp8_swa_simulate(codes[0][0], codes[1][0], codes[2][0], codes[0][1], codes[1][1],
                           codes[2][1], CFG["local_window"])
    mx, mean = rel_errors(to_np(out), ref)
    assert mx <= 2e-2 and mean <= 5e-3, (mx, mean)


def test_block_weight_cache_is_bit_identical():
    from flower_amd.precision import fp8_weight_cache
    blk = make_block(seed=5)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 128, CFG["d_model"], generator=g).to("cuda", torch.bfloat16)
    plain = blk(x)
    with fp8_weight_cache(blk):
        cached = blk(x)
        cached2 = blk(x)
    torch.cuda.synchronize()
    assert torch.equal(plain, cached) and torch.equal(cached, cached2)


def test_qk_epilogue_and_quantiser_routes_are_bit_identical():
    """The fused block's two places for QK-norm + RoPE -- the QKV GEMM's epilogue (with the
    per-head maxima, Q quantised on load) and the Q / K / V quantiser's pass pair -- apply the same
    transform and derive the same scales and codes, so the block outputs are equal bit for bit
    (ragged T, so the GEMM's last row tile is partial and positions wrap at the batch boundary)."""
    blk = make_block(seed=9)
    x = torch.randn(2, 300, CFG["d_model"], generator=torch.Generator().manual_seed(10)).to("cuda", torch.bfloat16)
    assert blk._fusable(x)
    blk.fuse_qk_epilogue = True
    tr_e = {}
    a = blk._forward_fused(x, trace=tr_e)
    blk.fuse_qk_epilogue = False
    tr_q = {}
    b = blk._forward_fused(x, trace=tr_q)
    torch.cuda.synchronize()
    assert "amax" in tr_e and "q8" in tr_q
    assert torch.equal(tr_e["q"].contiguous(), tr_q["q"]) and torch.equal(tr_e["k"].contiguous(), tr_q["k"])
    assert torch.equal(a, b)


@pytest.mark.parametrize("fuse_qk_epilogue", [True, False])
def test_fused_forward_matches_the_unfused_composition(fuse_qk_epilogue):
    """The fused path (RMSNorm / GELU fused with the per-row quantisers, QK-norm + RoPE in the QKV
    epilogue or in the Q / K / V quantiser, residual adds in the GEMM epilogues, attention written
    in place) against the module-by-module composition (QK-norm and RoPE in torch ops): the two
    differ only where torch's RMSNorm / HeadRMSNorm / GELU round differently in the last place."""
    blk = make_block(seed=7)
    blk.fuse_qk_epilogue = fuse_qk_epilogue
    g = torch.Generator().manual_seed(8)
    x = torch.randn(2, 512, CFG["d_model"], generator=g).to("cuda", torch.bfloat16)
    assert blk._fusable(x)
    fused = blk(x).float()
    plain = blk.forward_unfused(x).float()
    torch.cuda.synchronize()
    d_f, d_p = fused - x.float(), plain - x.float()
    rel = float((d_f - d_p).norm() / d_p.norm())
    print(f"fused vs unfused delta rel: {rel:.2e}")
    assert rel < 1e-2


def _ulp_bf16(a, b):
    from oracle.e4m3 import f32_to_bf16_bits
    ia = f32_to_bf16_bits(np.asarray(a, np.float32)).astype(np.int32)
    ib = f32_to_bf16_bits(np.asarray(b, np.float32)).astype(np.int32)
    return np.abs(ia - ib)


def _gemm_close(got, ref, what):
    tol = 2.0 ** -7 * np.abs(ref) + 1e-3 * np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    bad = np.abs(got - ref) > tol
    assert not bad.any(), (what, int(bad.sum()), float(np.abs(got - ref).max()))


def test_config5_full_shape_stage_by_stage():
    """BASELINE config 5 at its full shape: B1 T32768 d1024 H16 (D64) ffn4096 W4096, every linear
    from the FP8 weight cache (base.py:698-722 block, base.py:514-525 GELU MLP), fused forward.
    Each stage is checked on the kernels' own inputs:
      (i)   attention, two heads, against the oracle's FP8 simulator on the oracle's per-head codes
            of the block's own q', k', v (QK-normed and rotated as in (iv));
      (ii)  256 sampled rows of every linear (QKV, O + residual, FF1, FF2 + residual) against the
            float64 closed form on the kernel's codes and scales (rounded to bf16, then the
            residual added in bf16);
      (iii) the RMSNorm, attention-output and GELU row quantisers: codes and scales bit-exact
            against the per-row recipe on their own h, and h within 1 bf16 ulp of the oracle's
            RMSNorm / GELU on the sampled rows;
      (iv)  the attention's quantisation point (qkv_heads, base.py:618-639) in the QKV epilogue:
            the stored q', k' against the oracle's HeadRMSNorm + RoPE of the raw projection (the
            plain GEMM on the same codes) on the sampled rows (the per-value bounds of the
            fused-quantiser tests) and bit for bit against the Q / K / V quantiser's transform on
            the whole tensors; v untouched; the epilogue's per-head maxima equal to max |q'|,
            |k'|, |v| (the attention stage (i) then checks the codes derived from them).
    The traced call returns the same bits as the untraced one."""
    from flower_amd.block import Fp8DecoderBlock, init_block_
    from flower_amd.precision import fp8_weight_cache
    from oracle.block import gelu, head_rmsnorm, rmsnorm, rope
    from oracle.e4m3 import round_bf16
    from oracle.gemm import scaled_mm
    from oracle.quant import rowwise_fp8

    B, T, d, H, ffn, W = 1, 32768, 1024, 16, 4096, 4096
    D, M = d // H, B * T
    blk = Fp8DecoderBlock(d, H, ffn, W)
    init_block_(blk, std=0.02, seed=55)
    blk = blk.to("cuda", torch.bfloat16)
    x = torch.randn(B, T, d, generator=torch.Generator().manual_seed(56)).to("cuda", torch.bfloat16)
    print("[c5] fused forward at B1 T32768 d1024 H16 ffn4096 W4096", flush=True)
    with fp8_weight_cache(blk):
        tr = {}
        out = blk._forward_fused(x, trace=tr)
        plain = blk(x)
        wq = [lin.weight_codes() for lin in blk._linears()]
        torch.cuda.synchronize()
    assert torch.equal(out, plain)

    rows = np.sort(np.random.default_rng(57).choice(M, 256, replace=False))
    ridx = torch.from_numpy(rows).cuda()
    cpu = lambda t: to_np(t.index_select(0, ridx))     # noqa: E731  sampled rows on the host
    x2 = x.view(M, d)
    w8 = [(to_np(w.view(torch.uint8)), to_np(s)) for w, s in wq]

    # (iv) the quantisation point in the QKV epilogue: the raw projection (the plain GEMM on the same
    # codes) against the fused output -- v bit for bit; q', k' on sampled rows against the oracle's
    # HeadRMSNorm + RoPE of the raw heads, and on the whole tensors bit for bit against the Q / K / V
    # quantiser's transform; the epilogue's maxima are those of q', k', v.
    from flower_amd import _lib as L
    from flower_amd.kernels import qk_norm_rope_quant_e4m3
    lib = L.load()
    qkv = tr["qkv"].view(M, 3 * d)
    raw = torch.empty_like(qkv)
    L.check(lib.flw_fp8_scaled_mm(tr["c1"].data_ptr(), M, d, wq[0][0].data_ptr(), 3 * d, tr["s1"].data_ptr(), M,
                                  wq[0][1].data_ptr(), 3 * d, raw.data_ptr(), 3 * d, L.stream_of(raw)), "raw qkv")
    assert torch.equal(qkv[:, 2 * d:], raw[:, 2 * d:])
    cos_t, sin_t = blk.attn.rope.tables(T, torch.bfloat16, "cuda")
    rq, rk, rv = (blk.attn._split(t) for t in raw.view(B, T, 3 * d).chunk(3, dim=-1))
    _, _, _, _, qt, kt = qk_norm_rope_quant_e4m3(rq, rk, rv, qk_norm=True, eps=blk.attn.qk_norm.eps, rope_cos=cos_t,
                                                 rope_sin=sin_t, granularity="head", return_transformed=True)
    assert torch.equal(tr["q"].contiguous(), qt) and torch.equal(tr["k"].contiguous(), kt)
    cos, sin = to_np(cos_t), to_np(sin_t)
    raw_rows = cpu(raw).reshape(len(rows), 3, H, D)
    pos = rows % T
    for i, name in enumerate(("q", "k")):
        want = rope(head_rmsnorm(raw_rows[:, i], blk.attn.qk_norm.eps, "bf16"), cos[pos][:, None], sin[pos][:, None],
                    "bf16")
        got = cpu(qkv).reshape(len(rows), 3, H, D)[:, i]
        d_ = np.abs(got.astype(np.float64) - want)
        assert (d_ > 0).mean() < 2e-3 and (d_ <= 2.0 ** -7 * (np.abs(want) + 1.0)).all(), (name, float(d_.max()))
    want_amax = qkv.view(M, 3 * H, D).float().abs().amax(dim=(0, 2))
    assert torch.equal(tr["amax"], want_amax.view(torch.int32))
    vv = blk.attn._split(tr["qkv"].chunk(3, dim=-1)[2])
    quant = [per_tensor_fp8(to_np(t.contiguous()), "head") for t in (tr["q"], tr["k"], vv)]

    # (iii) row quantisers: codes / scales on their own h; h against the oracle on sampled rows
    for c, s, h in (("c1", "s1", "h1"), ("c2", "s2", "h2"), ("cg", "sg", "hg")):
        want_c, want_s = rowwise_fp8(cpu(tr[h]))
        np.testing.assert_array_equal(cpu(tr[c]), want_c, err_msg=c)
        np.testing.assert_array_equal(to_np(tr[s])[rows], want_s.reshape(-1), err_msg=s)
    want_c, want_s = rowwise_fp8(cpu(tr["attn"].view(M, d)))
    np.testing.assert_array_equal(cpu(tr["ca"]), want_c)
    np.testing.assert_array_equal(to_np(tr["sa"])[rows], want_s.reshape(-1))
    for h, want in (("h1", rmsnorm(cpu(x2), to_np(blk.ln1.weight), blk.ln1.eps)),
                    ("h2", rmsnorm(cpu(tr["x1"]), to_np(blk.ln2.weight), blk.ln2.eps))):
        dd = _ulp_bf16(cpu(tr[h]), want)
        assert dd.max() <= 1 and (dd > 0).mean() < 1e-3, (h, dd.max(), (dd > 0).mean())
    got, want = cpu(tr["hg"]), gelu(cpu(tr["f"]))
    big = np.abs(want) > 1e-4
    dd = _ulp_bf16(got[big], want[big])
    assert dd.max() <= 1 and (dd > 0).mean() < 0.02, ("hg", dd.max(), (dd > 0).mean())
    assert np.abs(got[~big] - want[~big]).max() < 2e-6

    # (ii) the four linears on their own codes (QKV: the raw projection, before the q / k transform)
    def closed(cname, sname, wi):
        return round_bf16(scaled_mm(cpu(tr[cname]), w8[wi][0], to_np(tr[sname])[rows], w8[wi][1]))
    _gemm_close(cpu(raw), closed("c1", "s1", 0), "qkv")
    _gemm_close(cpu(tr["f"]), closed("c2", "s2", 2), "ff1")
    for yname, res, cn, sn, wi in (("x1", x2, "ca", "sa", 1), ("out", tr["x1"], "cg", "sg", 3)):
        y = cpu(out.view(M, d)) if yname == "out" else cpu(tr[yname])
        prod = closed(cn, sn, wi)
        ref = round_bf16(prod + cpu(res))
        tol = (2.0 ** -7 * (np.abs(prod) + np.abs(ref))
               + 1e-3 * np.sqrt(np.mean(prod.astype(np.float64) ** 2)))
        assert (np.abs(y - ref) <= tol).all(), (yname, float(np.abs(y - ref).max()))

    # (i) attention on the block's own q' / k' / v codes (checked above), two heads
    attn = to_np(tr["attn"].view(B, T, H, D).transpose(1, 2))
    for h in (2, 11):
        sl = slice(h, h + 1)
        ref = fp8_swa_simulate(quant[0][0][:, sl], quant[1][0][:, sl], quant[2][0][:, sl], quant[0][1][:, sl],
                               quant[1][1][:, sl], quant[2][1][:, sl], W, chunk=1024)
        mx, mean = rel_errors(attn[:, sl], ref)
        print(f"[c5] attention head {h}: max-rel {mx:.2e} mean-rel {mean:.2e}", flush=True)
        assert mx <= 2e-2 and mean <= 5e-3, (h, mx, mean)
    assert torch.isfinite(out).all()
