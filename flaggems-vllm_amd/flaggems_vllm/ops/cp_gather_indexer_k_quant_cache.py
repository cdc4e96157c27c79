"""Gather a batch's cached sparse-indexer keys (FP8 codes + float32 scales).

Drop-in for the reference op of the same name
(src/flaggems_vllm/ops/cp_gather_indexer_k_quant_cache.py:114-176): same
positional signature, k_fp8 and k_fp8_scale written in place, same ValueError
when head_dim is not a multiple of the quant block size implied by
k_fp8_scale.  One launch of the gfx950 kernel ``indexer_k_gather_kernel``
through the C ABI ``fgv_cp_gather_indexer_k_quant_cache`` on the current
stream.  It reads the cache that indexer_k_quant_and_cache writes.

Row t of k_fp8 (and of k_fp8_scale) belongs to request b when
cu_seqlen[b] <= t < cu_seqlen[b + 1]; it receives position t - cu_seqlen[b]
of that request, looked up through block_table[b].  Rows outside every
request are left untouched.

Beyond the reference: the quant block size is derived from k_fp8_scale's row
size in bytes (the reference assumes a byte-typed scale tensor, as vLLM
allocates it, and a float32 one then gives the same result here); row
strides of both outputs are honoured; rows whose block-table index or block
is out of range are left untouched instead of read out of bounds; int64
block_table / cu_seqlen are converted to int32.
"""
import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 else t.to(torch.int32)


def cp_gather_indexer_k_quant_cache(
    k_cache: torch.Tensor,
    k_fp8: torch.Tensor,
    k_fp8_scale: torch.Tensor,
    block_table: torch.Tensor,
    cu_seqlen: torch.Tensor,
) -> None:
    num_tokens = k_fp8.size(0)
    head_dim = k_fp8.shape[-1]
    scale_row_bytes = k_fp8_scale.size(1) * k_fp8_scale.element_size()
    quant_block_size = head_dim * 4 // scale_row_bytes
    if quant_block_size == 0 or head_dim % quant_block_size != 0:
        raise ValueError("head_dim must be divisible by quant_block_size")
    assert k_cache.dim() == 3 and k_cache.element_size() == 1, (
        "k_cache must be [num_blocks, block_size, bytes per token] of a 1-byte type"
    )
    assert k_cache[0].is_contiguous(), "each k_cache block must be contiguous bytes"
    assert k_fp8.dim() == 2 and k_fp8.element_size() == 1 and k_fp8.stride(-1) == 1
    assert k_fp8_scale.dim() == 2 and k_fp8_scale.stride(-1) == 1
    assert k_fp8_scale.size(0) >= num_tokens, "k_fp8_scale has fewer rows than k_fp8"
    assert block_table.dim() == 2 and block_table.stride(-1) == 1, "block_table rows must be contiguous"
    batch_size = block_table.shape[0]
    assert cu_seqlen.dim() == 1 and cu_seqlen.numel() >= batch_size + 1, "cu_seqlen needs batch_size + 1 entries"
    for t in (k_fp8, k_fp8_scale, block_table, cu_seqlen):
        assert t.device == k_cache.device, "all tensors must be on k_cache's device"
    assert k_cache.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    if num_tokens == 0 or batch_size == 0:
        return
    block_table = _i32(block_table)
    cu_seqlen = _i32(cu_seqlen).contiguous()
    with on_device_of(k_cache):
        rc = _native.lib().fgv_cp_gather_indexer_k_quant_cache(
            k_cache.data_ptr(), k_cache.stride(0), k_cache.shape[0], k_cache.shape[1],
            head_dim, quant_block_size,
            k_fp8.data_ptr(), k_fp8.stride(0),
            k_fp8_scale.data_ptr(), k_fp8_scale.stride(0) * k_fp8_scale.element_size(),
            block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
            cu_seqlen.data_ptr(), batch_size, num_tokens,
            current_stream_ptr(k_cache.device),
        )
    _native.check(rc, "cp_gather_indexer_k_quant_cache")


__all__ = ["cp_gather_indexer_k_quant_cache"]
