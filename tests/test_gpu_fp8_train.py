"""GPU: the FP8 backward of the FP8 linear (dgrad / wgrad, torchao Float8Linear's backward under
training.fp8_linear) through the C ABI, against the oracle (oracle/gemm.py: cols_fp8,
fp8_linear_backward).

- flw_quant_cols_e4m3: codes and scales bit-exact against the oracle (per column and per tensor,
  bf16 and fp32, ragged rows / columns, zero padding up to ld, a column with an inf);
- the gradient GEMMs against the oracle's closed form on the same codes: |d| <= 2^-7 |ref| +
  2^-7 |prod| + 1e-3 rms(ref) (the scaled-GEMM tolerance of the forward);
- Fp8Linear autograd: grads equal fp8_linear_backward's; inside fp8_weight_cache the weight's
  column codes are made once and the grads are bit-identical to the uncached ones;
- BASELINE C2 shape (x [8192, 1024], W [4096, 1024]): both gradients within the FP8-head bounds
  of the bf16 product.
"""

import numpy as np
import pytest
import torch

from oracle.gemm import cols_fp8, fp8_linear_backward as oracle_backward, rows_fp8, scaled_mm

pytestmark = pytest.mark.gpu


def _rnd(shape, seed, scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("gran", ["column", "tensor"])
@pytest.mark.parametrize("R,C,ld", [(300, 72, 320), (1024, 256, 1024), (16, 8, 16), (777, 136, 896)])
def test_quant_cols_bit_exact(dtype, gran, R, C, ld):
    from flower_amd.precision import quantize_cols
    x = _rnd((R, C), 1, dtype=dtype)
    codes, scale = quantize_cols(x.cuda(), gran, ld)
    want, ws = cols_fp8(x.float().numpy(), gran)
    got = codes.cpu().numpy()
    np.testing.assert_array_equal(got[:, :R], want)
    assert not got[:, R:].any()
    np.testing.assert_array_equal(scale.cpu().numpy(), ws)


def test_quant_cols_nonfinite_column():
    from flower_amd.precision import quantize_cols
    x = _rnd((256, 64), 2)
    x[5, 3] = float("inf")
    x[9, 40] = float("nan")
    for gran in ("column", "tensor"):
        codes, scale = quantize_cols(x.cuda(), gran)
        want, ws = cols_fp8(x.float().numpy(), gran)
        np.testing.assert_array_equal(codes.cpu().numpy(), want)
        np.testing.assert_array_equal(scale.cpu().numpy(), ws)


def test_quant_cols_strided_rows():
    from flower_amd.precision import quantize_cols
    big = _rnd((512, 200), 3)
    x = big[:, 16:144]                     # row stride 200, 128 columns
    codes, scale = quantize_cols(x.cuda(), "column")
    want, ws = cols_fp8(x.float().numpy(), "column")
    np.testing.assert_array_equal(codes.cpu().numpy(), want)
    np.testing.assert_array_equal(scale.cpu().numpy(), ws)


def _close(got, want, prod):
    tol = 2.0 ** -7 * np.abs(want) + 2.0 ** -7 * np.abs(prod) + 1e-3 * np.sqrt(np.mean(want ** 2))
    bad = np.abs(got - want) > tol
    assert not bad.any(), (int(bad.sum()), float(np.abs(got - want).max()))


@pytest.mark.parametrize("recipe", ["rowwise", "tensorwise"])
@pytest.mark.parametrize("M,N,K", [(256, 128, 64), (300, 96, 160), (1024, 512, 256)])
def test_backward_gemms_against_oracle(recipe, M, N, K):
    from flower_amd.precision import fp8_linear_backward, quantize_weight_cols
    g, x, w = _rnd((M, N), 4), _rnd((M, K), 5), _rnd((N, K), 6, 0.02)
    gx, gw = fp8_linear_backward(g.cuda(), x.cuda(), quantize_weight_cols(w.cuda(), recipe), recipe)
    want_gx, want_gw = oracle_backward(g.float().numpy(), x.float().numpy(), w.float().numpy(), recipe)
    prod_gx = g.double().numpy() @ w.double().numpy()
    prod_gw = g.double().numpy().T @ x.double().numpy()
    _close(gx.float().cpu().numpy(), want_gx, prod_gx)
    _close(gw.float().cpu().numpy(), want_gw, prod_gw)


@pytest.mark.parametrize("recipe", ["rowwise", "tensorwise"])
def test_fp8_linear_autograd_and_cache(recipe, monkeypatch):
    import flower_amd.precision as P
    torch.manual_seed(0)
    lin = torch.nn.Linear(256, 384, bias=False).cuda().to(torch.bfloat16)
    mod = P.Fp8Linear.from_linear(lin, recipe)
    x = _rnd((4, 96, 256), 7).cuda().requires_grad_(True)
    g = _rnd((4, 96, 384), 8).cuda()
    mod(x).backward(g)
    gx0, gw0 = x.grad.clone(), mod.weight.grad.clone()
    want_gx, want_gw = P.fp8_linear_backward(g.reshape(-1, 384), x.detach().reshape(-1, 256),
                                             P.quantize_weight_cols(mod.weight, recipe), recipe)
    assert torch.equal(gx0.reshape(-1, 256), want_gx)
    assert torch.equal(gw0, want_gw)
    x.grad = None
    mod.weight.grad = None
    calls = []
    orig = P.quantize_weight_cols

    def counting(*a, **k):
        calls.append(1)
        return orig(*a, **k)

    monkeypatch.setattr(P, "quantize_weight_cols", counting)
    with P.fp8_weight_cache(torch.nn.ModuleDict({"m": mod})):
        for _ in range(2):
            mod(x).backward(g)
    assert len(calls) == 1 and mod._fp8_cached_cols is None
    assert torch.equal(x.grad, 2 * gx0)
    assert torch.equal(mod.weight.grad, 2 * gw0)


def test_bf16_backward_switch():
    from flower_amd.precision import Fp8Linear
    lin = torch.nn.Linear(128, 64, bias=True).cuda().to(torch.bfloat16)
    mod = Fp8Linear.from_linear(lin, "rowwise")
    mod.backward_fp8 = False
    x = _rnd((32, 128), 9).cuda().requires_grad_(True)
    g = _rnd((32, 64), 10).cuda()
    mod(x).backward(g)
    assert torch.equal(x.grad, (g @ mod.weight).to(x.dtype))
    assert torch.equal(mod.bias.grad, g.sum(0))


@pytest.mark.parametrize("recipe", ["rowwise", "tensorwise"])
def test_c2_shape_gradients_within_fp8_bounds(recipe):
    from flower_amd.precision import fp8_linear_backward, quantize_weight_cols
    M, N, K = 8192, 4096, 1024
    g, x, w = _rnd((M, N), 11).cuda(), _rnd((M, K), 12).cuda(), _rnd((N, K), 13, 0.02).cuda()
    gx, gw = fp8_linear_backward(g, x, quantize_weight_cols(w, recipe), recipe)
    for got, want in ((gx, g.float() @ w.float()), (gw, g.float().t() @ x.float())):
        err = float((got.float() - want).norm() / want.norm())
        ratio = float(got.float().norm() / want.norm())
        assert err < 0.05 and 0.9 < ratio < 1.1, (err, ratio)


@pytest.mark.parametrize("R,C,ld", [(4096, 1024, 4096), (300, 48, 384), (1, 16, 16), (129, 3392, 256), (70, 208, 80)])
def test_transposed_tensorwise_codes_equal_the_column_quantiser(R, C, ld):
    """flw_transpose_e4m3 on the per-tensor row codes of x gives flw_quant_cols_e4m3's per-tensor
    column codes of x bit for bit (one scale for the whole matrix), with the columns past R zero."""
    from flower_amd.precision import _quantize_rows, quantize_cols, transpose_codes
    x = (_rnd((R, C), R + C) * 3).cuda()
    x8, sx = _quantize_rows(x, "tensorwise")
    want8, want_s = quantize_cols(x, "tensor", ld)
    got8 = transpose_codes(x8, ld)
    assert torch.equal(sx, want_s)
    assert torch.equal(got8, want8)
    assert not got8[:, R:].any()


@pytest.mark.parametrize("R,C,ld,pad,special", [(4096, 1024, 4096, 0, None), (300, 48, 384, 0, None),
                                                (1, 16, 16, 0, None), (129, 3392, 256, 0, None),
                                                (70, 208, 80, 16, None), (257, 1280, 384, 0, "inf"),
                                                (100, 64, 128, 0, "nan"), (64, 128, 64, 0, "zero")])
def test_one_pass_tensorwise_codes_in_both_layouts(R, C, ld, pad, special):
    """flw_quant_tensor_t_e4m3 (through _quantize_tensorwise_t): the row codes and scale of the
    tensorwise quantiser (_quantize_rows) and their transpose (flw_transpose_e4m3), bit for bit,
    with the columns past R zero -- contiguous matrices (the amax pass over 64-value rows) and
    strided rows (over the matrix's rows), an inf or a NaN in the matrix (the exact path) and an
    all-zero matrix (the scale floor)."""
    from flower_amd.precision import _quantize_rows, _quantize_tensorwise_t, transpose_codes
    base = (_rnd((R, C + pad), R + C) * 3).cuda()
    if special == "inf":
        base[R // 2, 7] = float("inf")
    elif special == "nan":
        base[3, 5] = float("nan")
    elif special == "zero":
        base.zero_()
    x = base[:, :C]
    x8, x8t, sx = _quantize_tensorwise_t(x, ld)
    want8, want_s = _quantize_rows(x.contiguous(), "tensorwise")
    assert torch.equal(sx, want_s) or (special == "nan" and torch.isnan(sx).all() and torch.isnan(want_s).all())
    assert torch.equal(x8, want8)
    assert torch.equal(x8t, transpose_codes(want8, ld))
    assert not x8t[:, R:].any()


@pytest.mark.parametrize("recipe", ["rowwise", "tensorwise"])
@pytest.mark.parametrize("bias", [False, True])
def test_fp8_linear_residual_argument(recipe, bias):
    """Fp8Linear(x, residual=r) equals r + Fp8Linear(x) bit for bit (in the tensorwise GEMM's
    epilogue without a bias, in torch otherwise), and its gradients -- r's is the output's -- equal
    those of the separate add; the forward's weight codes in both layouts (training) equal the
    plain weight cast's."""
    from flower_amd.precision import Fp8Linear
    torch.manual_seed(1)
    lin = torch.nn.Linear(256, 384, bias=bias).cuda().to(torch.bfloat16)
    mod = Fp8Linear.from_linear(lin, recipe)
    x = _rnd((3, 100, 256), 31).cuda()
    r = _rnd((3, 100, 384), 32).cuda()
    g = _rnd((3, 100, 384), 33).cuda()
    xa, ra = x.clone().requires_grad_(True), r.clone().requires_grad_(True)
    ya = mod(xa, residual=ra)
    ya.backward(g)
    ga = (xa.grad, ra.grad, mod.weight.grad.clone())
    mod.weight.grad = None
    if bias:
        gba = mod.bias.grad.clone()
        mod.bias.grad = None
    xb, rb = x.clone().requires_grad_(True), r.clone().requires_grad_(True)
    yb = rb + mod(xb)
    yb.backward(g)
    assert torch.equal(ya, yb)
    assert torch.equal(ga[0], xb.grad) and torch.equal(ga[1], rb.grad) and torch.equal(ga[2], mod.weight.grad)
    if bias:
        assert torch.equal(gba, mod.bias.grad)
    if recipe == "tensorwise":
        w8, sw, w8t = mod.tensorwise_codes()
        p8, ps = mod.quantize_weight()
        assert torch.equal(w8, p8) and torch.equal(sw, ps)
        assert torch.equal(w8t[:, :384], w8.t()) and w8t.shape == (256, 384)
