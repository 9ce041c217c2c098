"""GPU: the allocation-free QKV quantiser (flw_quant_qkv_e4m3_noalloc) through the C ABI against
the workspace entry point it mirrors (flw_quant_qkv_e4m3): codes, V tiles and scales bit for bit,
on two calls in a row (the second on a smaller input, so stale scratch contents from the first
call would show), for each scale granularity. The refusal of a shape whose amax partials do not fit
the library's scratch array is a host check, tested on the CPU with fake pointers
(tests/test_abi.py)."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(B, H, T, D, seed):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(B, H, T, D, generator=g) * torch.randn(1, H, 1, 1, generator=g).exp())
            .to(torch.bfloat16).cuda() for _ in range(3)]


def _outputs(lib, B, H, T, D, G):
    q8 = torch.full((B, H, T, D), 0xAB, dtype=torch.uint8, device="cuda")
    k8 = torch.full_like(q8, 0xCD)
    vt = torch.full((lib.flw_vtile_bytes(B, H, T, D),), 0xEF, dtype=torch.uint8, device="cuda")
    sc = torch.full((3 * G,), -1.0, dtype=torch.float32, device="cuda")
    return q8, k8, vt, sc


def _run(noalloc, q, k, v, gran):
    from flower_amd import _lib as L
    lib = L.load()
    B, H, T, D = q.shape
    G = {"tensor": 1, "head": H, "bh": B * H}[gran]
    q8, k8, vt, sc = _outputs(lib, B, H, T, D, G)
    strides = L.i64s(*q.stride()[:3], *k.stride()[:3], *v.stride()[:3])
    if noalloc:
        rc = lib.flw_quant_qkv_e4m3_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), L.BF16, B, H, T, D,
                                            strides, L.GRANULARITY[gran], q8.data_ptr(), k8.data_ptr(),
                                            vt.data_ptr(), sc.data_ptr(), L.stream_of(q))
    else:
        ws = L.workspace(3 * lib.flw_quant_workspace_bytes(B, H, T, D), q.device)
        rc = lib.flw_quant_qkv_e4m3(q.data_ptr(), k.data_ptr(), v.data_ptr(), L.BF16, B, H, T, D, strides,
                                    L.GRANULARITY[gran], q8.data_ptr(), k8.data_ptr(), vt.data_ptr(),
                                    sc.data_ptr(), ws.data_ptr(), ws.numel(), L.stream_of(q))
    L.check(rc, "noalloc" if noalloc else "workspace")
    return q8, k8, vt, sc


@pytest.mark.parametrize("gran", ["tensor", "head", "bh"])
def test_noalloc_quantiser_equals_the_workspace_entry_point(gran):
    # First a large call (B2 H8 T4096: 1,536 partials), then a smaller one (B1 H3 T300: 27 partials)
    # whose partials occupy the start of the same scratch array.
    for shape, seed in (((2, 8, 4096, 64), 1), ((1, 3, 300, 64), 2)):
        q, k, v = _inputs(*shape, seed)
        print(f"[noalloc] {gran} {shape}", flush=True)
        want = _run(False, q, k, v, gran)
        got = _run(True, q, k, v, gran)
        torch.cuda.synchronize()
        for name, a, b in zip(("q8", "k8", "v_tiles", "scales"), got, want):
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), (gran, shape, name)
        assert torch.isfinite(got[3]).all() and bool((got[3] > 0).all())
