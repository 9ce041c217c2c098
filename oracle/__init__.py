"""CPU oracle for the FP8 sliding-window-attention path. TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference's FP8-simulated PyTorch path:

- ``e4m3``  : bit-exact fp32/bf16 <-> e4m3fn codecs (the ``Tensor.to(torch.float8_e4m3fn)``
              cast the reference relies on, restated from the OCP FP8 spec);
- ``quant`` : the three quantisation recipes on the path
              (``_per_tensor_fp8``  flower/kernels/fp8_swa_attention.py:195-205,
               ``_fake_quant_e4m3`` flower/models/base.py:167-203,
               ``_fp8_head`` row/channel scales flower/models/base.py:887-924)
              plus the per-head / per-(b,h) granularity this build defines;
- ``swa``   : the causal sliding-window mask (base.py:418-423), the dense fp32 reference
              (fp8_swa_attention.py:262-273), a banded form of it for long sequences, and a
              kernel-faithful simulator of the FP8 flash-attention loop
              (fp8_swa_attention.py:129-192);
- ``gemm``  : the closed form of the scaled FP8 GEMM (``torch._scaled_mm`` as called at
              base.py:919-923).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker (or, for the CPU baseline, as the thing timed on the host).
The product path in ``flower_amd`` never imports it and has no CPU fallback.

Parity status of each function (what pins it) is listed in each module's header.
"""
