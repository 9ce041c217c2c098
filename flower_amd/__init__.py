"""flower_amd -- MI355X-native (gfx950) FP8 sliding-window-attention path of sims1253/flower.

The operators keep the reference's Python API; their work runs in ``libflower_amd.so``
(hand-written HIP for CDNA4, C ABI in ``include/flower_amd.h``), loaded through ctypes.

    from flower_amd.kernels.fp8_swa_attention import fp8_swa_attention_forward
    from flower_amd.attention import _fake_quant_e4m3
    from flower_amd.precision import Fp8Linear, fp8_weight_cache, convert_model_to_fp8
"""

__version__ = "0.1.0"
