"""vLLM-compatible decode top-k over rows of per-row lengths.

Drop-in for the reference's ``persistent_topk``
(src/flaggems_vllm/ops/persistent_topk.py:2179-2342): same signature, the same
assertions, ``output`` written in place.  Row r's candidates are
``logits[r, :lengths.reshape(-1)[r]]`` (``lengths`` [num_rows], or [B, next_n]
for MTP, one length per row) clamped to the row width; ``output[r]`` receives
the column indices of the row's top ``k`` values, in no particular order, or
``0 .. len-1`` then -1 for a row of at most ``k`` values.  The work is the
same gfx950 radix select as ``top_k_per_row_decode`` (C ABI
``fgv_top_k_per_row_decode`` with next_n = 1); the caller's ``workspace``
carries the split of few long rows when it is large enough
(``fgv_top_k_per_row_workspace_bytes``) and 16-byte aligned, and the rows are
streamed otherwise, with the same index sets.  Values equal to the k-th
largest are taken lowest index first.
"""
import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of


def persistent_topk(logits: torch.Tensor, lengths: torch.Tensor, output: torch.Tensor, workspace: torch.Tensor,
                    k: int = 512, max_seq_len: int = None) -> None:
    assert logits.is_cuda, "persistent_topk: logits must be CUDA tensor"
    assert lengths.is_cuda, "persistent_topk: lengths must be CUDA tensor"
    assert output.is_cuda, "persistent_topk: output must be CUDA tensor"
    assert logits.dtype == torch.float32, "persistent_topk: only float32 supported"
    assert lengths.dtype == torch.int32, "persistent_topk: lengths must be int32"
    assert output.dtype == torch.int32, "persistent_topk: output must be int32"
    assert logits.dim() == 2, "persistent_topk: logits must be 2D"
    assert lengths.dim() in (1, 2), "persistent_topk: lengths must be 1D or 2D"
    assert lengths.is_contiguous(), "persistent_topk: lengths must be contiguous"
    assert output.dim() == 2, "persistent_topk: output must be 2D"
    num_rows = logits.size(0)
    seq_lens = lengths.reshape(-1)
    assert seq_lens.numel() == num_rows, (
        f"persistent_topk: lengths size mismatch: {seq_lens.numel()} vs {num_rows}")
    assert output.size(0) == num_rows and output.size(1) == k, (
        f"persistent_topk: output size mismatch: ({output.size(0)}, {output.size(1)}) vs ({num_rows}, {k})")
    assert k in (512, 1024, 2048), f"persistent_topk supports k=512, k=1024, or k=2048, got k={k}"
    width = logits.shape[1]
    L = _native.lib()
    need = L.fgv_top_k_per_row_workspace_bytes(num_rows, width, k)
    use_ws = (need > 0 and workspace is not None and workspace.is_cuda and workspace.device == logits.device
              and workspace.numel() * workspace.element_size() >= need and workspace.data_ptr() % 16 == 0)
    with on_device_of(logits):
        rc = L.fgv_top_k_per_row_decode(
            logits.data_ptr(), logits.stride(0), logits.stride(1), num_rows, width, 1, seq_lens.data_ptr(),
            output.data_ptr(), output.stride(0), output.stride(1), k,
            workspace.data_ptr() if use_ws else None, need if use_ws else 0, current_stream_ptr(logits.device))
    _native.check(rc, "persistent_topk")


__all__ = ["persistent_topk"]
