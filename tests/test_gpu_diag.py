"""GPU: the issue-cost probe behind `bench.py --issue-probe` runs every supported mask, and its
two basic orderings hold on the device: a v_exp_f32 costs more issue time than a v_fma_f32, and
an MFMA mixed with independent VALU work takes less than the two run apart (some overlap)."""

import pytest
import torch

pytestmark = pytest.mark.gpu

MASKS = [1, 2, 4, 8, 16, 32, 64, 65, 66, 68, 72, 80, 3, 67]


def _time(lib, mask, out, blocks):
    from flower_amd import _lib
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.flw_diag_issue_probe(mask, out.data_ptr(), out.numel(), blocks, stream), "probe")
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    _lib.check(lib.flw_diag_issue_probe(mask, out.data_ptr(), out.numel(), blocks, stream), "probe")
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def test_issue_probe_masks_and_orderings():
    from flower_amd import _lib
    lib = _lib.load()
    blocks = 4 * torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    ms = {m: _time(lib, m, out, blocks) for m in MASKS}
    assert ms[2] > 1.5 * ms[1], ms                   # exp is a multi-slot instruction
    assert ms[65] < ms[1] + ms[64], ms               # MFMA partly hidden under fma
    assert ms[66] < ms[2] + ms[64], ms
