"""flaggems_vllm for MI355X (gfx950): the DeepSeek-V4 attention pre-processing path.

Public names follow the reference package (src/flaggems_vllm/__init__.py:21-46):
``fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert``, ``fused_inv_rope_fp8_quant``,
their compatibility aliases ``ops_deepseek_v4_qnorm_rope_kv_rope_quant_insert`` and
``ops_inv_rope_fp8_quant``, ``SUPPORTED_FP8_DTYPE``, ``device`` and ``vendor_name``;
and the ops either side of that path (src/flaggems_vllm/ops/__init__.py): the
K-cache gather, q/kv RMSNorm, the sparse indexer (q quant, key cache and
logits and their top-k per row), the index rows sparse attention reads (global
top-k indices, top-k plus sliding window), slot mapping, sparse MLA decode, sparse MLA prefill
(``flash_mla_sparse_fwd``) and the block-FP8 grouped output projection (``fp8_einsum``) after the sibling op.  Every op runs hand-written HIP kernels through the C ABI declared in
include/flaggems_vllm_amd.h; there is no Triton, no vendor dispatch and no
CPU fallback.
"""
from . import ops  # noqa: F401
from .ops import (  # noqa: F401
    SUPPORTED_FP8_DTYPE,
    FlashMLASchedMeta,
    combine_topk_swa_indices,
    compute_global_topk_indices_and_lens,
    compute_slot_mapping_parallel,
    cp_gather_indexer_k_quant_cache,
    dequantize_and_gather_k_cache,
    flash_mla_sparse_fwd,
    flash_mla_with_kvcache,
    fp8_einsum,
    fp8_fp4_mqa_logits,
    fp8_fp4_paged_mqa_logits,
    fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert,
    fused_indexer_q_rope_quant,
    fused_inv_rope_fp8_quant,
    fused_q_kv_rmsnorm,
    get_mla_metadata,
    indexer_k_quant_and_cache,
    persistent_topk,
    top_k_per_row_decode,
    top_k_per_row_prefill,
)

from . import library  # noqa: F401,E402  (torch.ops.flaggems_vllm.* registrations)

device = "cuda"
vendor_name = "amd"
__version__ = "0.1.0"

ops_deepseek_v4_qnorm_rope_kv_rope_quant_insert = fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert
ops_inv_rope_fp8_quant = fused_inv_rope_fp8_quant

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
    "ops_deepseek_v4_qnorm_rope_kv_rope_quant_insert",
    "ops_inv_rope_fp8_quant",
    "SUPPORTED_FP8_DTYPE",
    "persistent_topk",
    "top_k_per_row_decode",
    "top_k_per_row_prefill",
]
