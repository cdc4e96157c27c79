"""Quantise sparse-indexer keys to FP8 and insert them into the paged key cache.

Drop-in for the reference op of the same name
(src/flaggems_vllm/ops/indexer_k_quant_and_cache.py:100-132): same positional
signature, same in-place contract (kv_cache written, everything else read
only), same ValueError when head_dim is not a multiple of quant_block_size.
The work is one launch of the gfx950 kernel ``indexer_k_quant_kernel``
through the C ABI ``fgv_indexer_k_quant_and_cache`` on the current stream.

Cache layout (uint8 [num_blocks, block_size, head_dim + 4 * head_dim / 128]):
per block, block_size x head_dim float8_e4m3fn codes, then block_size x
(head_dim / 128) float32 scales.  The codes are OCP e4m3fn (max 448), the
format vLLM selects on gfx950; the reference's no-vLLM HIP fallback to
e4m3fnuz (max 224) belongs to earlier Instinct parts and is not offered.

Beyond the reference: k may have a row stride (unit last stride, stride a
multiple of 8 elements) and fp16 as well as bf16 rows; slots whose block is
past the end of kv_cache are skipped instead of written out of bounds.
quant_block_size must be 128 (the DeepSeek-V4 indexer's, and the only one
the reference's tests use).
"""
import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of


def indexer_k_quant_and_cache(
    k: torch.Tensor,
    kv_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    quant_block_size,
    scale_fmt,
) -> None:
    """kv_cache[slot] = (e4m3fn(k[t] / scale_j), scale_j) per 128-element block j,
    scale_j = max(amax_j, 1e-4) / 448, rounded up to a power of two when
    scale_fmt == "ue8m0"; tokens with slot_mapping[t] < 0 are skipped."""
    head_dim = k.shape[-1]
    if head_dim % quant_block_size != 0:
        raise ValueError("head_dim must be divisible by quant_block_size")
    num_tokens = slot_mapping.shape[0]
    assert k.dtype in (torch.bfloat16, torch.float16), "k must be bfloat16 or float16"
    assert kv_cache.dim() == 3 and kv_cache.element_size() == 1, (
        "kv_cache must be [num_blocks, block_size, bytes per token] of a 1-byte type"
    )
    assert kv_cache[0].is_contiguous(), "each kv_cache block must be contiguous bytes"
    assert slot_mapping.dim() == 1 and slot_mapping.dtype == torch.int64
    assert slot_mapping.stride(0) == 1 or num_tokens <= 1
    k2 = k.reshape(-1, head_dim) if k.dim() != 2 else k
    assert k2.shape[0] >= num_tokens, "k has fewer rows than slot_mapping"
    assert k2.stride(-1) == 1, "k rows must be contiguous"
    for t in (kv_cache, slot_mapping):
        assert t.device == k.device, "all tensors must be on k's device"
    assert k.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    if num_tokens == 0:
        return
    num_blocks, block_size = kv_cache.shape[0], kv_cache.shape[1]
    with on_device_of(k):
        rc = _native.lib().fgv_indexer_k_quant_and_cache(
            k2.data_ptr(), k2.stride(0), int(k.dtype == torch.float16),
            num_tokens, head_dim, int(quant_block_size),
            kv_cache.data_ptr(), kv_cache.stride(0), num_blocks, block_size,
            slot_mapping.data_ptr(), int(scale_fmt == "ue8m0"),
            current_stream_ptr(k.device),
        )
    _native.check(rc, "indexer_k_quant_and_cache")


__all__ = ["indexer_k_quant_and_cache"]
