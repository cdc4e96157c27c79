"""Paged-KV slot-mapping generation, parallel over tokens.

Drop-in for the reference's ``compute_slot_mapping_parallel``
(src/flaggems_vllm/runtime/backend/_ascend/ops/slot_mapping.py:109-144, an
Ascend backend op exported as ``flaggems_vllm.compute_slot_mapping_parallel``):
same signature and semantics, including the context-parallel interleave
arithmetic and the pad region, written in place into ``slot_mapping`` by the
gfx950 kernel ``slot_mapping_kernel`` (C ABI ``fgv_compute_slot_mapping``).
Its output is the ``slot_mapping`` of
fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.
"""
import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of


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
    assert slot_mapping.dtype == torch.int64 and slot_mapping.stride(-1) == 1
    assert slot_mapping.numel() >= max_num_tokens
    assert query_start_loc.dtype == torch.int32 and query_start_loc.numel() >= num_reqs + 1
    assert positions.dtype in (torch.int32, torch.int64) and positions.stride(-1) == 1
    assert block_table.dtype == torch.int32 and block_table.ndim == 2
    assert block_table.stride(-1) == 1
    assert slot_mapping.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    for t in (query_start_loc, positions, block_table):
        assert t.device == slot_mapping.device, "all tensors must be on slot_mapping's device"
    query_start_loc = query_start_loc.contiguous()
    with on_device_of(slot_mapping):
        rc = _native.lib().fgv_compute_slot_mapping(
            int(num_tokens), int(max_num_tokens), query_start_loc.data_ptr(), int(num_reqs),
            positions.data_ptr(), int(positions.dtype == torch.int64),
            block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
            slot_mapping.data_ptr(), int(block_size),
            int(cp_world_size), int(cp_rank), int(cp_kv_cache_interleave_size), int(pad_id),
            current_stream_ptr(slot_mapping.device),
        )
    _native.check(rc, "compute_slot_mapping_parallel")


__all__ = ["compute_slot_mapping_parallel"]
