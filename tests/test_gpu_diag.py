"""GPU: the issue-cost probe behind `bench.py --issue-probe` runs every supported mask, and its
two basic orderings hold on the device: a v_exp_f32 costs more issue time than a v_fma_f32, and
an MFMA mixed with independent VALU work takes less than the two run apart (some overlap).
Also the attention kernel's e4m3 MFMA on given operands: exact where the dot product is small
integers, and within a stated bound of the exact dot product otherwise."""

import numpy as np
import pytest
import torch

from oracle.e4m3 import e4m3_to_f32

pytestmark = pytest.mark.gpu

MASKS = [1, 2, 4, 8, 16, 32, 64, 65, 66, 68, 72, 80, 3, 67]


def _time(lib, mask, out, blocks):
    from flower_amd import _lib
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.flw_diag_issue_probe(mask, out.data_ptr(), out.numel(), blocks, stream), "probe", lib)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    _lib.check(lib.flw_diag_issue_probe(mask, out.data_ptr(), out.numel(), blocks, stream), "probe", lib)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def test_issue_probe_masks_and_orderings():
    from flower_amd import _lib
    lib = _lib.load_diag()
    blocks = 4 * torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    ms = {m: _time(lib, m, out, blocks) for m in MASKS}
    assert ms[2] > 1.5 * ms[1], ms                   # exp is a multi-slot instruction
    assert ms[65] < ms[1] + ms[64], ms               # MFMA partly hidden under fma
    assert ms[66] < ms[2] + ms[64], ms


def _mfma_products(lib, A, B, A2=None, B2=None):
    """flw_diag_mfma_e4m3_dot on code arrays A [n, 32, 64], B [n, 64, 32] (and the chained pair)."""
    from flower_amd import _lib

    def frag(M, rows_major):
        out = np.empty((M.shape[0], 64, 32), np.uint8)
        for lane in range(64):
            k0 = 32 * (lane // 32)
            out[:, lane] = M[:, lane % 32, k0:k0 + 32] if rows_major else M[:, k0:k0 + 32, lane % 32]
        return torch.from_numpy(out.reshape(M.shape[0], 2048)).cuda()

    n = A.shape[0]
    ta, tb = frag(A, True), frag(B, False)
    chain = A2 is not None
    ta2, tb2 = (frag(A2, True), frag(B2, False)) if chain else (ta, tb)
    d = torch.empty((n, 1024), dtype=torch.float32, device="cuda")
    _lib.check(lib.flw_diag_mfma_e4m3_dot(ta.data_ptr(), tb.data_ptr(), ta2.data_ptr(), tb2.data_ptr(), d.data_ptr(),
                                          n, int(chain), torch.cuda.current_stream().cuda_stream), "mfma dot", lib)
    torch.cuda.synchronize()
    raw = d.cpu().numpy()
    D = np.empty((n, 32, 32), np.float32)
    for v in range(16):
        for lane in range(64):
            D[:, 8 * (v // 4) + 4 * (lane // 32) + v % 4, lane % 32] = raw[:, 64 * v + lane]
    return D.astype(np.float64)


def test_mfma_e4m3_dot_layout_is_exact_on_small_integers():
    """Operands whose products and sums are small integers (exact in any accumulator): the
    diagnostic's fragment layout and the MFMA give the exact products, single and chained."""
    from flower_amd import _lib
    from oracle.e4m3 import f32_to_e4m3
    lib = _lib.load_diag()
    rng = np.random.default_rng(11)
    mk = lambda shape: f32_to_e4m3(rng.integers(-2, 3, size=shape).astype(np.float32))  # noqa: E731
    dec = lambda c: e4m3_to_f32(c).astype(np.float64)  # noqa: E731
    A, B, A2, B2 = mk((16, 32, 64)), mk((16, 64, 32)), mk((16, 32, 64)), mk((16, 64, 32))
    assert np.array_equal(_mfma_products(lib, A, B), dec(A) @ dec(B))
    assert np.array_equal(_mfma_products(lib, A, B, A2, B2), dec(A) @ dec(B) + dec(A2) @ dec(B2))


@pytest.mark.parametrize("chain", [False, True])
def test_mfma_e4m3_accumulation_error_is_bounded(chain):
    """The FP8 MFMA's fp32 accumulation is not the correctly rounded dot product (measured on
    gfx950: up to ~3e-4 of the largest product for normal-like codes, ~5.5e-4 for codes drawn
    uniformly; about a third of the results or fewer equal the rounded exact sum), so attention
    scores differ from the simulator's exact dot products by that much; a P code whose 448 p lies
    that close to an e4m3 rounding boundary can round the other way. Bound: 2^-10 of the largest
    product of each 64-deep (or chained 128-deep) dot."""
    from flower_amd import _lib
    from oracle.e4m3 import f32_to_e4m3
    lib = _lib.load_diag()
    rng = np.random.default_rng(12)
    dec = lambda c: e4m3_to_f32(c).astype(np.float64)  # noqa: E731

    def normal(shape):
        return f32_to_e4m3(np.clip(rng.standard_normal(shape) * 110.0, -448, 448).astype(np.float32))

    def uniform(shape):
        c = rng.integers(0, 256, size=shape).astype(np.uint8)
        c[(c & 0x7F) == 0x7F] = 0                       # no NaN codes
        return c

    for mk in (normal, uniform):
        A, B = mk((128, 32, 64)), mk((128, 64, 32))
        prods = dec(A)[:, :, :, None] * dec(B)[:, None, :, :]
        exact, pmax = prods.sum(axis=2), np.abs(prods).max(axis=2)
        if chain:
            A2, B2 = mk((128, 32, 64)), mk((128, 64, 32))
            p2 = dec(A2)[:, :, :, None] * dec(B2)[:, None, :, :]
            exact, pmax = exact + p2.sum(axis=2), np.maximum(pmax, np.abs(p2).max(axis=2))
            hw = _mfma_products(lib, A, B, A2, B2)
        else:
            hw = _mfma_products(lib, A, B)
        err = np.abs(hw - exact) / np.maximum(pmax, 1e-30)
        assert err.max() <= 2.0 ** -10, (mk.__name__, chain, err.max())
