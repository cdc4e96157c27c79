"""Request-local top-k indices to global cache slots, with the row lengths.

Drop-in for the reference's ``compute_global_topk_indices_and_lens``
(src/flaggems_vllm/ops/deepseek_v4_attention_compute_global_topk_indices_and_lens.py:122-160):
same signature, outputs and layouts (``global_indices`` is
``empty_like(topk_indices)``, ``lens`` is [num_tokens] int32).  The work is
the gfx950 kernel ``global_topk_indices_kernel`` (C ABI
``fgv_compute_global_topk_indices_and_lens``).  Its outputs are the
``indices`` / ``topk_length`` of flash_mla_with_kvcache's sparse decode.
"""
from typing import Optional, Tuple

import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of


def compute_global_topk_indices_and_lens(
    topk_indices: torch.Tensor,
    token_to_req_indices: torch.Tensor,
    block_table: torch.Tensor,
    block_size: int,
    is_valid_token: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    assert topk_indices.ndim == 2
    assert topk_indices.dtype == torch.int32, "topk_indices must be int32"
    assert token_to_req_indices.dtype == torch.int32 and token_to_req_indices.numel() >= topk_indices.shape[0]
    assert block_table.dtype == torch.int32 and block_table.ndim == 2 and block_table.stride(-1) == 1
    assert topk_indices.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    num_tokens, topk = topk_indices.shape
    global_indices = torch.empty_like(topk_indices, dtype=torch.int32)
    lens = torch.empty((num_tokens,), device=topk_indices.device, dtype=torch.int32)
    req = token_to_req_indices.contiguous()
    valid = None
    if is_valid_token is not None:
        assert is_valid_token.dtype == torch.int32 and is_valid_token.numel() >= num_tokens
        valid = is_valid_token.contiguous()
    with on_device_of(topk_indices):
        rc = _native.lib().fgv_compute_global_topk_indices_and_lens(
            topk_indices.data_ptr(), topk_indices.stride(0), topk_indices.stride(1), num_tokens, topk,
            req.data_ptr(), block_table.data_ptr(), block_table.stride(0), block_table.shape[0],
            block_table.shape[1], int(block_size), valid.data_ptr() if valid is not None else None,
            global_indices.data_ptr(), global_indices.stride(0), global_indices.stride(1), lens.data_ptr(),
            current_stream_ptr(topk_indices.device),
        )
    _native.check(rc, "compute_global_topk_indices_and_lens")
    return global_indices, lens


__all__ = ["compute_global_topk_indices_and_lens"]
