"""The two DeepSeek-V4 attention pre-processing ops (reference: src/flaggems_vllm/ops/__init__.py:61-64)."""
from .fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert import (
    fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert,
)
from .fused_inv_rope_fp8_quant import SUPPORTED_FP8_DTYPE, fused_inv_rope_fp8_quant

__all__ = [
    "fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert",
    "fused_inv_rope_fp8_quant",
    "SUPPORTED_FP8_DTYPE",
]
