"""GPU: the stream contract of the C ABI (every entry point launches on the stream it is given --
torch's current stream -- and nowhere else) and NaN propagation through the FP8 attention.

Streams: one entry point of each family (QKV quantiser, FP8 attention, FP8 GEMM, bf16 SWA
backward) is run inside ``torch.cuda.stream(side)`` on a default-priority side stream, with the
inputs produced on the default stream beforehand, and compared bit for bit with the same call on
the default stream. A call that launched on the default stream, or read its inputs before the
side stream had waited for them, would differ or race.

NaN: with per-head scales a NaN in one head of Q, of K or of V makes that head's scale NaN, hence
its codes NaN, hence every output row of that head NaN (the reference's per-tensor case makes the
whole output NaN, fp8_swa_attention.py:195-205); heads without a NaN are bit-identical to the
NaN-free call.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _on_side_stream(fn):
    side = torch.cuda.Stream()                 # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out = fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    return out


def _seeded(shape, seed, dtype=torch.bfloat16):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).to("cuda", dtype)


def test_quantiser_and_attention_on_a_side_stream():
    from flower_amd.kernels import fp8_swa_attention_forward, qk_norm_rope_quant_e4m3
    q, k, v = (_seeded((2, 4, 1000, 64), s) * (s + 1) for s in (1, 2, 3))

    def run():
        codes = qk_norm_rope_quant_e4m3(q, k, v, qk_norm=True, granularity="head")
        return [c.clone() for c in codes] + [fp8_swa_attention_forward(q, k, v, 300, granularity="head")]
    base = run()
    torch.cuda.synchronize()
    side = _on_side_stream(run)
    for a, b in zip(base, side):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_fp8_gemm_on_a_side_stream():
    from flower_amd.precision import Fp8Linear
    lin = Fp8Linear(1024, 2048, bias=False).to("cuda", torch.bfloat16)
    x = _seeded((4096, 1024), 4)
    with torch.no_grad():
        base = lin(x)
        torch.cuda.synchronize()
        side = _on_side_stream(lambda: lin(x))
    assert torch.equal(base, side)


def test_bf16_swa_backward_on_a_side_stream():
    from flower_amd.kernels.swa_attention import swa_attention
    base_in = [_seeded((1, 2, 512, 64), s) for s in (5, 6, 7)]
    g = _seeded((1, 2, 512, 64), 8)

    def run():
        q, k, v = (t.clone().requires_grad_(True) for t in base_in)
        swa_attention(q, k, v, 128).backward(g)
        return [q.grad, k.grad, v.grad]
    base = run()
    torch.cuda.synchronize()
    side = _on_side_stream(run)
    for a, b in zip(base, side):
        assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_nan_in_one_head_poisons_that_head_only(dtype):
    from flower_amd.kernels import fp8_swa_attention_forward
    B, H, T, D, W = 2, 4, 384, 64, 128
    q, k, v = (_seeded((B, H, T, D), s, dtype) for s in (9, 10, 11))
    clean = fp8_swa_attention_forward(q, k, v, W, granularity="head")
    q[0, 1, 5, 3] = float("nan")
    k[1, 2, 300, 0] = float("nan")
    v[0, 3, 77, 63] = float("nan")
    out = fp8_swa_attention_forward(q, k, v, W, granularity="head")
    torch.cuda.synchronize()
    for h in (1, 2, 3):
        assert torch.isnan(out[:, h]).all(), h
    assert torch.equal(out[:, 0], clean[:, 0])
    # per-tensor scales: one NaN anywhere reaches the one scale and every output
    q2, k2, v2 = (_seeded((1, 2, 256, 64), s, dtype) for s in (12, 13, 14))
    v2[0, 1, 10, 10] = float("nan")
    assert torch.isnan(fp8_swa_attention_forward(q2, k2, v2, 64)).all()
