"""Dequantise and gather DeepSeek-V4 cached K rows into bf16.

Drop-in for the reference op of the same name
(src/flaggems_vllm/ops/deepseek_v4_attention_dequantize_and_gather_k_cache.py:123-172):
same signature and defaults, same AssertionErrors, ``out`` written in place on
the current stream by the gfx950 kernel ``dequantize_gather_kernel`` through
the C ABI ``fgv_dequantize_and_gather_k_cache``.  It reads the 584-byte token
layout that fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert writes.

Beyond the reference: rows whose block-table index or physical block is out
of range are left untouched instead of being read out of bounds; int64 index
tensors are converted to int32.  nope_dim and rope_dim must be multiples of 8.
"""
from typing import Optional

import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of


def _default_scale_slots(nope_dim: int) -> int:
    return (nope_dim + 63) // 64 + (1 if nope_dim % 64 == 0 else 0)


def _i32(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if t is None:
        return None
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t


def dequantize_and_gather_k_cache(
    out: torch.Tensor,
    k_cache: torch.Tensor,
    seq_lens: torch.Tensor,
    gather_lens: Optional[torch.Tensor],
    block_table: torch.Tensor,
    block_size: int,
    offset: int = 0,
    rope_dim: int = 64,
    nope_dim: Optional[int] = None,
    scale_slots: Optional[int] = None,
) -> None:
    """out[r, offset + i] = dequantised cache row of position
    seq_lens[r] - gather_lens[r] + i (gather_lens=None: the whole sequence)."""
    assert out.ndim == 3 and out.dtype == torch.bfloat16
    assert seq_lens.ndim == 1 and block_table.ndim == 2
    assert seq_lens.shape[0] == block_table.shape[0] <= out.shape[0]
    output_dim = out.shape[-1]
    if nope_dim is None:
        nope_dim = output_dim - rope_dim
    if scale_slots is None:
        scale_slots = _default_scale_slots(nope_dim)
    assert nope_dim + rope_dim <= output_dim
    assert k_cache.ndim in (2, 3), f"k_cache must be 2D or 3D, got shape={tuple(k_cache.shape)}"
    assert out.stride(-1) == 1, "out rows must be contiguous"
    assert k_cache[0].is_contiguous(), "each k_cache block must be contiguous bytes"
    assert block_table.stride(-1) == 1, "block_table rows must be contiguous"
    assert out.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    for t in (k_cache, seq_lens, block_table) + ((gather_lens,) if gather_lens is not None else ()):
        assert t.device == out.device, "all tensors must be on out's device"

    seq_lens = _i32(seq_lens).contiguous()
    gather_lens = _i32(gather_lens)
    if gather_lens is not None:
        gather_lens = gather_lens.contiguous()
    block_table = _i32(block_table)
    num_reqs = seq_lens.shape[0]
    if num_reqs == 0:
        return
    with on_device_of(out):
        rc = _native.lib().fgv_dequantize_and_gather_k_cache(
            out.data_ptr(), out.stride(0), out.stride(1), out.shape[1],
            k_cache.data_ptr(), k_cache.stride(0), k_cache.shape[0],
            seq_lens.data_ptr(), gather_lens.data_ptr() if gather_lens is not None else None,
            block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
            num_reqs, int(block_size), int(offset),
            int(nope_dim), int(rope_dim), int(scale_slots),
            current_stream_ptr(out.device),
        )
    _native.check(rc, "dequantize_and_gather_k_cache")


__all__ = ["dequantize_and_gather_k_cache"]
