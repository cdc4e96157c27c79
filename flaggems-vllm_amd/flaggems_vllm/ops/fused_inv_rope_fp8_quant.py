"""Fused DeepSeek-V4 inverse RoPE + per-128 FP8 e4m3fn group quant.

Drop-in for the reference op of the same name
(src/flaggems_vllm/ops/fused_inv_rope_fp8_quant.py:157-256): same signature
and defaults, same output tensors and strides, same AssertionErrors.  The
work is one launch of the gfx950 HIP kernel ``inv_rope_fp8_quant_kernel``
through the C ABI ``fgv_inv_rope_fp8_quant`` on the current stream.

Differences from the reference, all deliberate:
* ``dtype=None`` means float8_e4m3fn: gfx950 converts to OCP e4m3 natively,
  whereas the reference falls back to float32 (and then fails its own assert)
  on every vendor but NVIDIA and MetaX
  (src/flaggems_vllm/utils/device_info.py:85-97).
* The rotated rope values are rounded to bf16 before the amax and the quant,
  as the reference's torch oracle does
  (tests/test_fused_inv_rope_fp8_quant.py:167-170), so codes and scales match
  that oracle bit for bit.
* Only the DeepSeek-V4 geometry is implemented: head_dim 512 = 448 nope + 64
  rope, quant_group_size 128.
"""
import logging
from typing import Optional, Tuple

import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of

SUPPORTED_FP8_DTYPE = torch.float8_e4m3fn

logger = logging.getLogger(__name__)


def _get_tma_aligned_size(size: int, align: int) -> int:
    return ((size + align - 1) // align) * align


def fused_inv_rope_fp8_quant(
    o: torch.Tensor,
    positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    n_groups: int,
    heads_per_group: int,
    nope_dim: int = 448,
    rope_dim: int = 64,
    quant_group_size: int = 128,
    eps: float = 1e-10,
    dtype: Optional[torch.dtype] = None,
    tma_aligned_scales: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Inverse GPT-J RoPE on the last 64 dims of each head, then FP8 quant.

    Args:
        o: [num_tokens, num_heads, head_dim] bf16 attention output.
        positions: [num_tokens] int64.
        cos_sin_cache: [max_position, rope_dim] float32, cos || sin.

    Returns:
        o_fp8: [num_tokens, n_groups, heads_per_group * head_dim] float8_e4m3fn
            with strides (d, num_tokens * d, 1).
        o_scale: [num_tokens, n_groups, num_scale_blocks] float32, or the packed
            UE8M0 int32 view [num_tokens, n_groups, ceil(blocks / 4)] when
            tma_aligned_scales; token-fastest storage padded to 4 tokens.
    """
    logger.debug("GEMS FUSED INV ROPE FP8 QUANT")

    fp8_dtype = SUPPORTED_FP8_DTYPE if dtype is None else dtype
    assert fp8_dtype == torch.float8_e4m3fn, "only torch.float8_e4m3fn is supported"
    assert o.ndim == 3, "`o` must be [num_tokens, num_heads, head_dim]"
    assert positions.ndim == 1, "`positions` must be 1D"
    assert cos_sin_cache.ndim == 2, "`cos_sin_cache` must be 2D"
    assert o.stride(-1) == 1, "head_dim must be contiguous"
    assert positions.shape[0] == o.shape[0], "positions and o token count mismatch"

    num_tokens, num_heads, head_dim = o.shape
    assert num_heads == n_groups * heads_per_group
    assert head_dim == nope_dim + rope_dim
    assert head_dim % quant_group_size == 0
    assert nope_dim % quant_group_size == (quant_group_size - rope_dim)
    assert rope_dim % 2 == 0
    assert cos_sin_cache.shape[-1] == rope_dim
    assert cos_sin_cache.dtype == torch.float32
    assert (nope_dim, rope_dim, quant_group_size) == (448, 64, 128), (
        "this build implements the DeepSeek-V4 geometry: nope_dim=448, rope_dim=64, "
        "quant_group_size=128"
    )
    assert o.dtype == torch.bfloat16, "`o` must be bfloat16"
    assert cos_sin_cache.stride(1) == 1, "cos_sin_cache rows must be contiguous"
    assert o.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    assert positions.device == o.device and cos_sin_cache.device == o.device

    chunks_per_head = head_dim // quant_group_size
    if tma_aligned_scales:
        assert (
            chunks_per_head <= 4
        ), "packed UE8M0 path currently expects at most 4 scale blocks per head"

    if positions.dtype != torch.int64 or positions.stride(0) != 1:
        positions = positions.to(torch.int64).contiguous()

    d = heads_per_group * head_dim
    num_scale_blocks = d // quant_group_size
    tma_aligned_t = _get_tma_aligned_size(num_tokens, 4)
    if tma_aligned_scales:
        scale_inner = (num_scale_blocks + 3) // 4
        scale_dtype = torch.int32
    else:
        scale_inner = num_scale_blocks
        scale_dtype = torch.float32

    fp8_q = torch.empty((n_groups, num_tokens, d), dtype=fp8_dtype, device=o.device)
    scale = torch.empty(
        n_groups * scale_inner * tma_aligned_t, dtype=scale_dtype, device=o.device
    ).as_strided(
        (n_groups, num_tokens, scale_inner),
        (scale_inner * tma_aligned_t, 1, tma_aligned_t),
    )

    if tma_aligned_t > 0:
        with on_device_of(o):
            rc = _native.lib().fgv_inv_rope_fp8_quant(
                o.data_ptr(), o.stride(0), o.stride(1),
                positions.data_ptr(),
                cos_sin_cache.data_ptr(), cos_sin_cache.stride(0), cos_sin_cache.shape[0],
                num_tokens, n_groups, heads_per_group,
                fp8_q.data_ptr(), fp8_q.stride(0), fp8_q.stride(1),
                scale.data_ptr(), scale.stride(0), scale.stride(2),
                tma_aligned_t, float(eps), int(bool(tma_aligned_scales)),
                current_stream_ptr(o.device),
            )
        _native.check(rc, "fused_inv_rope_fp8_quant")

    return fp8_q.transpose(0, 1), scale.transpose(0, 1)
