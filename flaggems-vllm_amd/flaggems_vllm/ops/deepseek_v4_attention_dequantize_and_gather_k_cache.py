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
The checks and the launch run in C++ (``torch_ops.cpp``, ``dequantize_gather``);
scale_slots defaults to (nope_dim + 63) // 64, plus one when 64 divides
nope_dim.
"""
from typing import Optional

import torch

from .. import _native


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
    rc = _native.torch_ext().dequantize_gather(out, k_cache, seq_lens, gather_lens, block_table, int(block_size),
                                               int(offset), int(rope_dim), nope_dim, scale_slots)
    if rc:
        _native.raise_status(rc, "dequantize_and_gather_k_cache")


__all__ = ["dequantize_and_gather_k_cache"]
