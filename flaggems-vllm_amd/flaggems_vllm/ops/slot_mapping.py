"""Paged-KV slot-mapping generation, parallel over tokens.

Drop-in for the reference's ``compute_slot_mapping_parallel``
(src/flaggems_vllm/runtime/backend/_ascend/ops/slot_mapping.py:109-144, an
Ascend backend op exported as ``flaggems_vllm.compute_slot_mapping_parallel``):
same signature and semantics, including the context-parallel interleave
arithmetic and the pad region, written in place into ``slot_mapping`` by the
gfx950 kernel ``slot_mapping_kernel`` (C ABI ``fgv_compute_slot_mapping``).
Its output is the ``slot_mapping`` of
fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.  The checks and the launch
run in C++ (``torch_ops.cpp``, ``slot_mapping``).
"""
import torch

from .. import _native


def compute_slot_mapping_parallel(
    num_tokens: int,
    max_num_tokens: int,
    query_start_loc: torch.Tensor,
    num_reqs: int,
    positions: torch.Tensor,
    block_table: torch.Tensor,
    slot_mapping: torch.Tensor,
    block_size: int,
    cp_world_size: int = 1,
    cp_rank: int = 0,
    cp_kv_cache_interleave_size: int = 1,
    pad_id: int = -1,
) -> None:
    """Fill ``slot_mapping[:max_num_tokens]``: the cache slot of each token of
    each request, and ``pad_id`` for tokens num_tokens..max_num_tokens-1."""
    rc = _native.torch_ext().slot_mapping(int(num_tokens), int(max_num_tokens), query_start_loc, int(num_reqs),
                                          positions, block_table, slot_mapping, int(block_size), int(cp_world_size),
                                          int(cp_rank), int(cp_kv_cache_interleave_size), int(pad_id))
    if rc:
        _native.raise_status(rc, "compute_slot_mapping_parallel")


__all__ = ["compute_slot_mapping_parallel"]
