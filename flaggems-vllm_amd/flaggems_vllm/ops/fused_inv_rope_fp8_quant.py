"""Fused DeepSeek-V4 inverse RoPE + per-128 FP8 e4m3fn group quant.

Drop-in for the reference op of the same name
(src/flaggems_vllm/ops/fused_inv_rope_fp8_quant.py:157-256): same signature
and defaults, same output tensors and strides, same AssertionErrors.  The
checks, the two output allocations and the launch run in C++
(``torch_ops.cpp``, ``inv_rope_fp8_quant``): one launch of the gfx950 HIP
kernel ``inv_rope_fp8_quant_kernel`` through the C ABI
``fgv_inv_rope_fp8_quant`` on the current stream.

Differences from the reference, all deliberate:
* ``dtype=None`` means float8_e4m3fn: gfx950 converts to OCP e4m3 natively,
  whereas the reference falls back to float32 (and then fails its own assert)
  on every vendor but NVIDIA and MetaX
  (src/flaggems_vllm/utils/device_info.py:85-97).
* The rotated rope values are rounded to bf16 before the amax and the quant,
  as the reference's torch oracle does
  (tests/test_fused_inv_rope_fp8_quant.py:167-170), so codes and scales match
  that oracle bit for bit.
* Every geometry the reference asserts accept (head_dim = nope_dim +
  rope_dim, quant_group_size | head_dim, the rope dims inside the last
  chunk), for head_dim a power of two in [8, 512] and quant_group_size a power
  of two >= 8 (the reference's Triton kernel needs powers of two too).
  DeepSeek-V4's (448, 64, 128) runs its own kernel, the rest a general one.
  Packed scales with fewer than four chunks per head need heads_per_group 1:
  the reference's packed scale tensor only then has a word for every head.
"""
import logging
from typing import Optional, Tuple

import torch

from .. import _native

SUPPORTED_FP8_DTYPE = torch.float8_e4m3fn

logger = logging.getLogger(__name__)


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
    rc, fp8_q, scale = _native.torch_ext().inv_rope_fp8_quant(
        o, positions, cos_sin_cache, n_groups, heads_per_group, nope_dim, rope_dim, quant_group_size, eps,
        dtype is None or dtype == SUPPORTED_FP8_DTYPE, bool(tma_aligned_scales))
    if rc:
        _native.raise_status(rc, "fused_inv_rope_fp8_quant")
    return fp8_q, scale
