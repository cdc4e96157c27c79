"""Block-scaled FP8 einsum ``bhr,hdr->bhd``: the grouped output projection
that consumes ``fused_inv_rope_fp8_quant``'s e4m3fn activations and scales.

Drop-in for the reference's ``fp8_einsum`` (src/flaggems_vllm/ops/fp8_einsum.py:20-115):
same signature, the same checks in the same order with the same exception
types (NotImplementedError for what the op does not support, ValueError for
inconsistent arguments), a new tensor or ``out`` returned.  The reference's
Hopper requirement becomes a HIP device requirement.  The work is the gfx950
kernels of ``fp8_einsum.hip`` (C ABI ``fgv_fp8_einsum_bhr_hdr_ws``): 16x16x128
FP8 MFMAs, one per 128-wide K block, each block's partial sum scaled by
``xs * ys`` into a float32 accumulator; mid-size b splits the K blocks over
several workgroups per output tile, with the partial tiles in a workspace
this wrapper allocates.
"""
from typing import Optional, Sequence

import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of

_OUT_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def fp8_einsum(
    equation: str,
    x: torch.Tensor,
    xs: torch.Tensor,
    y: torch.Tensor,
    ys: torch.Tensor,
    block_size: Sequence[int] = (128, 128),
    output_dtype: torch.dtype = torch.bfloat16,
    *,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """``out[b,h,d] = sum_r (x[b,h,r] xs[b,h,r/128]) (y[h,d,r] ys[h,d/128,r/128])``.

    ``x[b,h,r]`` and ``y[h,d,r]`` are float8_e4m3fn with a contiguous last
    dimension; ``xs`` and ``ys`` float32; r and d multiples of 128.  Output
    bfloat16 (default), float16 or float32.  Inference only.
    """
    if equation != "bhr,hdr->bhd":
        raise NotImplementedError("fp8_einsum only supports 'bhr,hdr->bhd'")
    if tuple(block_size) != (128, 128):
        raise NotImplementedError("fp8_einsum requires 128x128 scale blocks")
    if output_dtype not in _OUT_CODES:
        raise NotImplementedError("output_dtype must be bfloat16, float16 or float32")
    inputs = (x, xs, y, ys)
    if any(t.layout != torch.strided or t.ndim != 3 for t in inputs):
        raise ValueError("inputs must be strided rank-3 tensors")
    if any(t.device != x.device for t in inputs):
        raise ValueError("all inputs must be on the same device")
    if x.device.type != "cuda":
        raise NotImplementedError("fp8_einsum runs on the GPU (HIP) only")
    if x.dtype != torch.float8_e4m3fn or y.dtype != torch.float8_e4m3fn:
        raise NotImplementedError("x and y must have dtype float8_e4m3fn")
    if xs.dtype != torch.float32 or ys.dtype != torch.float32:
        raise NotImplementedError("xs and ys must have dtype float32")
    if any(t.requires_grad for t in inputs):
        raise NotImplementedError("fp8_einsum does not support autograd")

    b, h, r = x.shape
    h2, d, r2 = y.shape
    if h2 != h or r2 != r:
        raise ValueError("x and y head/reduction dimensions must match")
    if r % 128 or d % 128:
        raise NotImplementedError("r and d must be multiples of 128")
    if xs.shape != (b, h, r // 128) or ys.shape != (h, d // 128, r // 128):
        raise ValueError("scale shapes do not match the 128x128 block grid")
    if x.stride(-1) != 1 or y.stride(-1) != 1:
        raise NotImplementedError("x and y must have a contiguous last dimension")

    if out is None:
        out = torch.empty((b, h, d), device=x.device, dtype=output_dtype)
    else:
        if out.shape != (b, h, d) or out.device != x.device or out.dtype != output_dtype:
            raise ValueError("out must match the output shape, device and dtype")
        if out.layout != torch.strided or out.requires_grad:
            raise ValueError("out must be a strided tensor without autograd")
        # a dense last dimension and rows at least a row apart: no two outputs
        # share an element, padded buffers allowed
        if out.stride(-1) != 1 or out.stride(1) < d or out.stride(0) < h * out.stride(1):
            raise ValueError("out must have non-overlapping rows in [b,h,d] order")
        if out.numel() and any(out.untyped_storage().data_ptr() == t.untyped_storage().data_ptr() for t in inputs):
            raise ValueError("out must not share storage with an input")

    if out.numel() == 0:
        return out
    with on_device_of(x):
        # fp32 partial tiles of the split-K schedule (mid-size b), from torch's
        # caching allocator; 0 bytes when the sizes take an unsplit kernel
        ws_bytes = _native.lib().fgv_fp8_einsum_workspace_bytes(b, h, r, d)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes > 0 else None
        rc = _native.lib().fgv_fp8_einsum_bhr_hdr_ws(
            x.data_ptr(), x.stride(0), x.stride(1), xs.data_ptr(), xs.stride(0), xs.stride(1), xs.stride(2),
            y.data_ptr(), y.stride(0), y.stride(1), ys.data_ptr(), ys.stride(0), ys.stride(1), ys.stride(2),
            b, h, r, d, out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), _OUT_CODES[output_dtype],
            ws.data_ptr() if ws is not None else None, ws_bytes, current_stream_ptr(x.device))
    _native.check(rc, "fp8_einsum")
    return out


__all__ = ["fp8_einsum"]
