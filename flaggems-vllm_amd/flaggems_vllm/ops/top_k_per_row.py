"""Top-k per row of the sparse indexer's logits, decode and prefill forms.

Drop-ins for the reference's ``top_k_per_row_decode``
(src/flaggems_vllm/ops/top_k_per_row_decode.py:1263-1399) and
``top_k_per_row_prefill`` (src/flaggems_vllm/ops/top_k_per_row_prefill.py:1232-1331):
same signatures, writing ``indices`` in place.  The work is the gfx950 radix
select ``top_k_per_row_kernel`` (C ABI ``fgv_top_k_per_row_decode`` /
``fgv_top_k_per_row_prefill``).  As in the reference the order of a row's
indices is unspecified; values equal to the k-th largest are taken lowest
index first, so the selected set depends on the values only.
"""
import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of


def _check(logits, indices, num_rows, top_k):
    assert num_rows == logits.shape[0]
    assert logits.dtype == torch.float32 and logits.ndim == 2, "logits must be float32 [num_rows, vocab]"
    assert indices.dtype == torch.int32 and indices.ndim == 2, "indices must be int32 [num_rows, top_k]"
    assert indices.shape[0] >= num_rows and indices.shape[1] >= top_k
    assert logits.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    assert indices.device == logits.device


def _workspace(logits, num_rows, top_k):
    """The split's candidate buffer for rows wider than 16384 values (None if
    the sizes need none), allocated per call as the reference allocates its
    split buffers (ops/top_k_per_row_decode.py:1303-1312)."""
    n = _native.lib().fgv_top_k_per_row_workspace_bytes(int(num_rows), logits.shape[1], int(top_k))
    return torch.empty(n, dtype=torch.uint8, device=logits.device) if n > 0 else None


def top_k_per_row_decode(logits, next_n, seq_lens, indices, num_rows, stride0, stride1, top_k):
    """Row r holds candidates [0, seq_lens[r // next_n] - next_n + r % next_n + 1)."""
    _check(logits, indices, num_rows, top_k)
    assert seq_lens.dtype == torch.int32 and seq_lens.numel() >= (num_rows + next_n - 1) // next_n
    seq = seq_lens.contiguous()
    ws = _workspace(logits, num_rows, top_k)
    with on_device_of(logits):
        rc = _native.lib().fgv_top_k_per_row_decode(
            logits.data_ptr(), int(stride0), int(stride1), int(num_rows), logits.shape[1], int(next_n),
            seq.data_ptr(), indices.data_ptr(), indices.stride(0), indices.stride(1), int(top_k),
            ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
            current_stream_ptr(logits.device))
    _native.check(rc, "top_k_per_row_decode")


def top_k_per_row_prefill(logits, row_starts, row_ends, indices, num_rows, stride0, stride1, top_k):
    """Row r holds candidates [row_starts[r], row_ends[r]); indices are relative to row_starts[r]."""
    _check(logits, indices, num_rows, top_k)
    assert row_starts.dtype == torch.int32 and row_ends.dtype == torch.int32
    assert row_starts.numel() >= num_rows and row_ends.numel() >= num_rows
    starts, ends = row_starts.contiguous(), row_ends.contiguous()
    ws = _workspace(logits, num_rows, top_k)
    with on_device_of(logits):
        rc = _native.lib().fgv_top_k_per_row_prefill(
            logits.data_ptr(), int(stride0), int(stride1), int(num_rows), logits.shape[1], starts.data_ptr(),
            ends.data_ptr(), indices.data_ptr(), indices.stride(0), indices.stride(1), int(top_k),
            ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
            current_stream_ptr(logits.device))
    _native.check(rc, "top_k_per_row_prefill")


__all__ = ["top_k_per_row_decode", "top_k_per_row_prefill"]
