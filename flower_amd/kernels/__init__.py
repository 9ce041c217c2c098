"""HIP (gfx950) kernels behind the reference's ``flower.kernels`` operator API."""

from .fp8_swa_attention import (E4M3_MAX, _per_tensor_fp8, amax_e4m3, dequantize_e4m3, fp8_swa_attention,
                                fp8_swa_attention_forward, fp8_swa_attention_from_codes, qk_norm_rope_quant_e4m3,
                                quantize_e4m3_with_amax, reference_swa_attention)

__all__ = ["E4M3_MAX", "_per_tensor_fp8", "amax_e4m3", "dequantize_e4m3", "fp8_swa_attention",
           "fp8_swa_attention_forward", "fp8_swa_attention_from_codes", "qk_norm_rope_quant_e4m3",
           "quantize_e4m3_with_amax", "reference_swa_attention"]
