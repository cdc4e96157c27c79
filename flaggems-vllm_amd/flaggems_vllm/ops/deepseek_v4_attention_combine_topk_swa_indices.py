"""Top-k and sliding-window indices combined into one index row per token.

Drop-in for the reference's ``combine_topk_swa_indices``
(src/flaggems_vllm/ops/deepseek_v4_attention_combine_topk_swa_indices.py:105-150):
same signature and outputs, ``combined`` [num_tokens, topk + window_size
rounded up to 128] int32 (rows of tokens outside every request are left
unwritten, as the reference leaves them) and ``lens`` [num_tokens] int32.  The
work is the gfx950 kernel ``combine_topk_swa_kernel`` (C ABI
``fgv_combine_topk_swa_indices``).
"""
from typing import Tuple

import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of


def combine_topk_swa_indices(
    topk_indices: torch.Tensor,
    query_start_loc: torch.Tensor,
    seq_lens: torch.Tensor,
    gather_lens: torch.Tensor,
    window_size: int,
    compress_ratio: int,
    topk: int,
    M: int,
    N: int,
) -> Tuple[torch.Tensor, torch.Tensor]:
    assert topk_indices.ndim == 2
    assert topk_indices.dtype == torch.int32, "topk_indices must be int32"
    for t in (query_start_loc, seq_lens, gather_lens):
        assert t.dtype == torch.int32, "query_start_loc, seq_lens and gather_lens must be int32"
    assert topk_indices.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    num_tokens = topk_indices.shape[0]
    num_reqs = seq_lens.shape[0]
    assert query_start_loc.numel() >= num_reqs + 1 and gather_lens.numel() >= num_reqs
    L = _native.lib()
    width = L.fgv_combine_topk_swa_width(int(topk), int(window_size))
    assert width >= 0, "topk and window_size must be non-negative"
    combined = torch.empty((num_tokens, width), device=topk_indices.device, dtype=torch.int32)
    lens = torch.empty((num_tokens,), device=topk_indices.device, dtype=torch.int32)
    qsl, seq, gat = query_start_loc.contiguous(), seq_lens.contiguous(), gather_lens.contiguous()
    with on_device_of(topk_indices):
        rc = L.fgv_combine_topk_swa_indices(
            topk_indices.data_ptr(), topk_indices.stride(0), topk_indices.stride(1), num_tokens,
            topk_indices.shape[1], qsl.data_ptr(), seq.data_ptr(), gat.data_ptr(), num_reqs,
            int(window_size), int(compress_ratio), int(topk), int(M), int(N),
            combined.data_ptr(), combined.stride(0), combined.stride(1), lens.data_ptr(),
            current_stream_ptr(topk_indices.device),
        )
    _native.check(rc, "combine_topk_swa_indices")
    return combined, lens


__all__ = ["combine_topk_swa_indices"]
