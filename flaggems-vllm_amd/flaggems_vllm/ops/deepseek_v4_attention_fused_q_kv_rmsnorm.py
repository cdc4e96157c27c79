"""DeepSeek-V4 fused q/kv weighted RMSNorm.

Drop-in for the reference op of the same name
(src/flaggems_vllm/ops/deepseek_v4_attention_fused_q_kv_rmsnorm.py:65-103): same
signature, same AssertionErrors, outputs allocated like ``torch.empty_like``
and written by the gfx950 kernel ``fused_q_kv_rmsnorm_kernel`` through the C
ABI ``fgv_fused_q_kv_rmsnorm`` in one launch on the current stream.  The
checks, the allocation and the launch run in C++ (``torch_ops.cpp``,
``q_kv_rmsnorm``).

This build implements bf16 activations with bf16 or float32 weights and row
sizes that are multiples of 8 up to 2^24 (DeepSeek-V4: 1536 and 512).
"""
from typing import Tuple

import torch

from .. import _native


def fused_q_kv_rmsnorm(
    qr: torch.Tensor,
    kv: torch.Tensor,
    q_weight: torch.Tensor,
    kv_weight: torch.Tensor,
    eps: float,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(RMSNorm(qr) * q_weight, RMSNorm(kv) * kv_weight), row by row."""
    rc, qr_out, kv_out = _native.torch_ext().q_kv_rmsnorm(qr, kv, q_weight, kv_weight, float(eps))
    if rc:
        _native.raise_status(rc, "fused_q_kv_rmsnorm")
    return qr_out, kv_out


__all__ = ["fused_q_kv_rmsnorm"]
