"""DeepSeek-V4 attention pre-processing ops (reference: src/flaggems_vllm/ops/__init__.py:23-38, 55, 56, 57, 58-65, 78, 122, 142-143, 187, 229)."""
from .cp_gather_indexer_k_quant_cache import cp_gather_indexer_k_quant_cache
from .deepseek_v4_attention_combine_topk_swa_indices import combine_topk_swa_indices
from .deepseek_v4_attention_compute_global_topk_indices_and_lens import compute_global_topk_indices_and_lens
from .deepseek_v4_attention_dequantize_and_gather_k_cache import dequantize_and_gather_k_cache
from .deepseek_v4_attention_fused_q_kv_rmsnorm import fused_q_kv_rmsnorm
from .fp8_einsum import fp8_einsum
from .fp8_fp4_mqa_logits import fp8_fp4_mqa_logits
from .fp8_fp4_paged_mqa_logits import fp8_fp4_paged_mqa_logits
from .flash_mla_sparse import flash_mla_sparse_fwd
from .flash_mla_with_kvcache import FlashMLASchedMeta, flash_mla_with_kvcache, get_mla_metadata
from .fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert import (
    fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert,
)
from .fused_indexer_q_rope_quant import fused_indexer_q_rope_quant
from .fused_inv_rope_fp8_quant import SUPPORTED_FP8_DTYPE, fused_inv_rope_fp8_quant
from .indexer_k_quant_and_cache import indexer_k_quant_and_cache
from .persistent_topk import persistent_topk
from .slot_mapping import compute_slot_mapping_parallel
from .top_k_per_row import top_k_per_row_decode, top_k_per_row_prefill

__all__ = [
    "FlashMLASchedMeta",
    "combine_topk_swa_indices",
    "compute_global_topk_indices_and_lens",
    "compute_slot_mapping_parallel",
    "cp_gather_indexer_k_quant_cache",
    "flash_mla_sparse_fwd",
    "flash_mla_with_kvcache",
    "fp8_einsum",
    "fp8_fp4_mqa_logits",
    "fp8_fp4_paged_mqa_logits",
    "get_mla_metadata",
    "dequantize_and_gather_k_cache",
    "fused_q_kv_rmsnorm",
    "fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert",
    "fused_indexer_q_rope_quant",
    "fused_inv_rope_fp8_quant",
    "indexer_k_quant_and_cache",
    "SUPPORTED_FP8_DTYPE",
    "persistent_topk",
    "top_k_per_row_decode",
    "top_k_per_row_prefill",
]
