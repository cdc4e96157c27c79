"""torch.library registrations of the path's ops (``torch.ops.flaggems_vllm.*``).

The public API stays the plain Python functions the reference package exports
(src/flaggems_vllm/__init__.py:21-46); vllm-plugin-fl calls those directly.
These registrations expose the same ops to torch.compile and graph capture as
opaque custom ops: the schemas declare what each op writes, namely ``q`` and
``k_cache`` for the main op (alias-annotated ``Tensor(a0!) q``, ``Tensor(a2!) k_cache``), ``out``
for the gather, ``slot_mapping`` for the slot mapping, ``kv_cache`` for the
indexer key insert and ``k_fp8`` / ``k_fp8_scale`` for its gather, ``indices`` for the top-k per row
(``output`` and, for rows long enough to split, ``workspace`` for ``persistent_topk``),
``out`` for ``fp8_einsum_out`` (the index-row ops, ``fp8_einsum`` and ``flash_mla_sparse_fwd`` write only what they return).  The fake (meta)
implementations give the output shapes and strides the real ops return.
The main op and the sibling are C++ ops (the torch extension's
``torch_ops.cpp``, loaded here): the same checks and launch the Python
functions call, raising RuntimeError on a failure as vLLM's compiled op does.
Every other registered op calls its Python wrapper, so argument checks and
errors are the wrapper's.

``fused_indexer_q_rope_quant`` returns ``(q, q_scale, weights)`` here, with an
empty ``q_scale`` for FP8, because an op schema cannot return the nested tuple
the Python function returns for MXFP4.  ``flash_mla_with_kvcache`` takes a
scheduler-metadata object and is not registered.
"""
from typing import List, Optional, Tuple

import torch

from . import _native
from .ops import (
    combine_topk_swa_indices,
    compute_global_topk_indices_and_lens,
    compute_slot_mapping_parallel,
    cp_gather_indexer_k_quant_cache,
    dequantize_and_gather_k_cache,
    flash_mla_sparse_fwd,
    fp8_einsum,
    fused_indexer_q_rope_quant,
    fused_q_kv_rmsnorm,
    indexer_k_quant_and_cache,
    persistent_topk,
    top_k_per_row_decode,
    top_k_per_row_prefill,
)

NAMESPACE = "flaggems_vllm"


def _op(name: str, mutates: Tuple[str, ...] = ()):
    return torch.library.custom_op(f"{NAMESPACE}::{name}", mutates_args=mutates, device_types="cuda")


# The main op and the sibling are C++ ops (torch_ops.cpp), registered in this
# namespace when the torch extension loads; their fakes are registered here.
_native.torch_ext()


@torch.library.register_fake(f"{NAMESPACE}::fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert")
def _(q, kv, k_cache, slot_mapping, position_ids, cos_sin_cache, eps, cache_block_size):
    return None


@torch.library.register_fake(f"{NAMESPACE}::fused_inv_rope_fp8_quant")
def _(o, positions, cos_sin_cache, n_groups, heads_per_group, nope_dim=448, rope_dim=64, quant_group_size=128,
      eps=1e-10, tma_aligned_scales=False):
    # the real op's layout: fp8 (G, T, d) and scales (G, K, Tpad), both
    # returned transposed to token-major views
    t = o.shape[0]
    d = heads_per_group * o.shape[-1]
    blocks = d // quant_group_size
    tpad = (t + 3) // 4 * 4
    inner = (blocks + 3) // 4 if tma_aligned_scales else blocks
    fp8 = o.new_empty((n_groups, t, d), dtype=torch.float8_e4m3fn).transpose(0, 1)
    scale = o.new_empty(n_groups * inner * tpad, dtype=torch.int32 if tma_aligned_scales else torch.float32)
    scale = scale.as_strided((n_groups, t, inner), (inner * tpad, 1, tpad)).transpose(0, 1)
    return fp8, scale


@_op("fused_q_kv_rmsnorm")
def _q_kv_rmsnorm(qr: torch.Tensor, kv: torch.Tensor, q_weight: torch.Tensor, kv_weight: torch.Tensor,
                  eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    return fused_q_kv_rmsnorm(qr, kv, q_weight, kv_weight, eps)


@_q_kv_rmsnorm.register_fake
def _(qr, kv, q_weight, kv_weight, eps):
    return torch.empty_like(qr), torch.empty_like(kv)


@_op("dequantize_and_gather_k_cache", ("out",))
def _dequantize_and_gather(out: torch.Tensor, k_cache: torch.Tensor, seq_lens: torch.Tensor,
                           gather_lens: Optional[torch.Tensor], block_table: torch.Tensor, block_size: int,
                           offset: int = 0, rope_dim: int = 64, nope_dim: Optional[int] = None,
                           scale_slots: Optional[int] = None) -> None:
    dequantize_and_gather_k_cache(out, k_cache, seq_lens, gather_lens, block_table, block_size, offset, rope_dim,
                                  nope_dim, scale_slots)


@_dequantize_and_gather.register_fake
def _(out, k_cache, seq_lens, gather_lens, block_table, block_size, offset=0, rope_dim=64, nope_dim=None,
      scale_slots=None):
    return None


@_op("fused_indexer_q_rope_quant")
def _indexer_q_rope_quant(positions: torch.Tensor, index_q: torch.Tensor, index_q_cos_sin_cache: torch.Tensor,
                          index_weights: torch.Tensor, index_weights_softmax_scale: float,
                          index_weights_head_scale: float,
                          use_fp4: bool = False) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    q, w = fused_indexer_q_rope_quant(positions, index_q, index_q_cos_sin_cache, index_weights,
                                      index_weights_softmax_scale, index_weights_head_scale, use_fp4=use_fp4)
    if use_fp4:
        return q[0], q[1], w
    return q, q.new_empty((0,), dtype=torch.uint8), w


@_indexer_q_rope_quant.register_fake
def _(positions, index_q, index_q_cos_sin_cache, index_weights, index_weights_softmax_scale,
      index_weights_head_scale, use_fp4=False):
    # the real op's outputs: weights like index_weights in float32; FP8 codes
    # like index_q; MXFP4 nibbles [T, H, D/2] and the UE8M0 bytes [T, H, D/32]
    # viewed as int32 [T, H, D/128], squeezed to [T, H] when D == 128
    t, h, d = positions.shape[0], index_q.shape[1], index_q.shape[2]
    w = torch.empty_like(index_weights, dtype=torch.float32)
    if use_fp4:
        scale = index_q.new_empty((t, h, d // 128), dtype=torch.int32)
        return index_q.new_empty((t, h, d // 2), dtype=torch.uint8), scale.squeeze(-1), w
    return torch.empty_like(index_q, dtype=torch.float8_e4m3fn), index_q.new_empty((0,), dtype=torch.uint8), w


@_op("compute_slot_mapping_parallel", ("slot_mapping",))
def _slot_mapping(num_tokens: int, max_num_tokens: int, query_start_loc: torch.Tensor, num_reqs: int,
                  positions: torch.Tensor, block_table: torch.Tensor, slot_mapping: torch.Tensor, block_size: int,
                  cp_world_size: int = 1, cp_rank: int = 0, cp_kv_cache_interleave_size: int = 1,
                  pad_id: int = -1) -> None:
    compute_slot_mapping_parallel(num_tokens, max_num_tokens, query_start_loc, num_reqs, positions, block_table,
                                  slot_mapping, block_size, cp_world_size, cp_rank, cp_kv_cache_interleave_size,
                                  pad_id)


@_slot_mapping.register_fake
def _(num_tokens, max_num_tokens, query_start_loc, num_reqs, positions, block_table, slot_mapping, block_size,
      cp_world_size=1, cp_rank=0, cp_kv_cache_interleave_size=1, pad_id=-1):
    return None


@_op("indexer_k_quant_and_cache", ("kv_cache",))
def _indexer_k_quant_and_cache(k: torch.Tensor, kv_cache: torch.Tensor, slot_mapping: torch.Tensor,
                               quant_block_size: int, scale_fmt: Optional[str]) -> None:
    indexer_k_quant_and_cache(k, kv_cache, slot_mapping, quant_block_size, scale_fmt)


@_indexer_k_quant_and_cache.register_fake
def _(k, kv_cache, slot_mapping, quant_block_size, scale_fmt):
    return None


@_op("cp_gather_indexer_k_quant_cache", ("k_fp8", "k_fp8_scale"))
def _cp_gather_indexer_k_quant_cache(k_cache: torch.Tensor, k_fp8: torch.Tensor, k_fp8_scale: torch.Tensor,
                                     block_table: torch.Tensor, cu_seqlen: torch.Tensor) -> None:
    cp_gather_indexer_k_quant_cache(k_cache, k_fp8, k_fp8_scale, block_table, cu_seqlen)


@_cp_gather_indexer_k_quant_cache.register_fake
def _(k_cache, k_fp8, k_fp8_scale, block_table, cu_seqlen):
    return None


@_op("compute_global_topk_indices_and_lens")
def _global_topk_indices(topk_indices: torch.Tensor, token_to_req_indices: torch.Tensor, block_table: torch.Tensor,
                         block_size: int,
                         is_valid_token: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    return compute_global_topk_indices_and_lens(topk_indices, token_to_req_indices, block_table, block_size,
                                                is_valid_token)


@_global_topk_indices.register_fake
def _(topk_indices, token_to_req_indices, block_table, block_size, is_valid_token=None):
    return (torch.empty_like(topk_indices, dtype=torch.int32),
            topk_indices.new_empty((topk_indices.shape[0],), dtype=torch.int32))


@_op("combine_topk_swa_indices")
def _combine_topk_swa(topk_indices: torch.Tensor, query_start_loc: torch.Tensor, seq_lens: torch.Tensor,
                      gather_lens: torch.Tensor, window_size: int, compress_ratio: int, topk: int, M: int,
                      N: int) -> Tuple[torch.Tensor, torch.Tensor]:
    return combine_topk_swa_indices(topk_indices, query_start_loc, seq_lens, gather_lens, window_size,
                                    compress_ratio, topk, M, N)


@_combine_topk_swa.register_fake
def _(topk_indices, query_start_loc, seq_lens, gather_lens, window_size, compress_ratio, topk, M, N):
    width = (topk + window_size + 127) // 128 * 128
    t = topk_indices.shape[0]
    return topk_indices.new_empty((t, width), dtype=torch.int32), topk_indices.new_empty((t,), dtype=torch.int32)


@_op("top_k_per_row_decode", ("indices",))
def _top_k_decode(logits: torch.Tensor, next_n: int, seq_lens: torch.Tensor, indices: torch.Tensor, num_rows: int,
                  stride0: int, stride1: int, top_k: int) -> None:
    top_k_per_row_decode(logits, next_n, seq_lens, indices, num_rows, stride0, stride1, top_k)


@_top_k_decode.register_fake
def _(logits, next_n, seq_lens, indices, num_rows, stride0, stride1, top_k):
    return None


@_op("top_k_per_row_prefill", ("indices",))
def _top_k_prefill(logits: torch.Tensor, row_starts: torch.Tensor, row_ends: torch.Tensor, indices: torch.Tensor,
                   num_rows: int, stride0: int, stride1: int, top_k: int) -> None:
    top_k_per_row_prefill(logits, row_starts, row_ends, indices, num_rows, stride0, stride1, top_k)


@_top_k_prefill.register_fake
def _(logits, row_starts, row_ends, indices, num_rows, stride0, stride1, top_k):
    return None


@_op("persistent_topk", ("output", "workspace"))
def _persistent_topk(logits: torch.Tensor, lengths: torch.Tensor, output: torch.Tensor, workspace: torch.Tensor,
                     k: int = 512, max_seq_len: Optional[int] = None) -> None:
    persistent_topk(logits, lengths, output, workspace, k, max_seq_len)


@_persistent_topk.register_fake
def _(logits, lengths, output, workspace, k=512, max_seq_len=None):
    return None


@_op("fp8_einsum")
def _fp8_einsum(equation: str, x: torch.Tensor, xs: torch.Tensor, y: torch.Tensor, ys: torch.Tensor,
                block_size: List[int], output_dtype: torch.dtype) -> torch.Tensor:
    return fp8_einsum(equation, x, xs, y, ys, block_size, output_dtype)


@_fp8_einsum.register_fake
def _(equation, x, xs, y, ys, block_size, output_dtype):
    return x.new_empty((x.shape[0], x.shape[1], y.shape[1]), dtype=output_dtype)


@_op("fp8_einsum_out", ("out",))
def _fp8_einsum_out(equation: str, x: torch.Tensor, xs: torch.Tensor, y: torch.Tensor, ys: torch.Tensor,
                    block_size: List[int], output_dtype: torch.dtype, out: torch.Tensor) -> None:
    fp8_einsum(equation, x, xs, y, ys, block_size, output_dtype, out=out)


@_fp8_einsum_out.register_fake
def _(equation, x, xs, y, ys, block_size, output_dtype, out):
    return None


@_op("flash_mla_sparse_fwd")
def _flash_mla_sparse_fwd(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor, sm_scale: float, d_v: int = 512,
                          attn_sink: Optional[torch.Tensor] = None,
                          topk_length: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return flash_mla_sparse_fwd(q, kv, indices, sm_scale, d_v, attn_sink, topk_length)


@_flash_mla_sparse_fwd.register_fake
def _(q, kv, indices, sm_scale, d_v=512, attn_sink=None, topk_length=None):
    s_q, h_q = q.shape[0], q.shape[1]
    return (q.new_empty((s_q, h_q, d_v)), q.new_empty((s_q, h_q), dtype=torch.float32),
            q.new_empty((s_q, h_q), dtype=torch.float32))


REGISTERED: List[str] = [
    "fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert",
    "fused_inv_rope_fp8_quant",
    "fused_q_kv_rmsnorm",
    "dequantize_and_gather_k_cache",
    "fused_indexer_q_rope_quant",
    "compute_slot_mapping_parallel",
    "indexer_k_quant_and_cache",
    "cp_gather_indexer_k_quant_cache",
    "compute_global_topk_indices_and_lens",
    "combine_topk_swa_indices",
    "top_k_per_row_decode",
    "top_k_per_row_prefill",
    "fp8_einsum",
    "fp8_einsum_out",
    "persistent_topk",
    "flash_mla_sparse_fwd",
]
