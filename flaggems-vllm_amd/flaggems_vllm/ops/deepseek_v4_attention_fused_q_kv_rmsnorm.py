"""DeepSeek-V4 fused q/kv weighted RMSNorm.

Drop-in for the reference op of the same name
(src/flaggems_vllm/ops/deepseek_v4_attention_fused_q_kv_rmsnorm.py:65-103): same
signature, same AssertionErrors, outputs allocated with ``torch.empty_like``
and written by the gfx950 kernel ``fused_q_kv_rmsnorm_kernel`` through the C
ABI ``fgv_fused_q_kv_rmsnorm`` in one launch on the current stream.

This build implements bf16 activations with bf16 or float32 weights and row
sizes that are multiples of 8 up to 4096 (DeepSeek-V4: 1536 and 512).
"""
from typing import Tuple

import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of


def fused_q_kv_rmsnorm(
    qr: torch.Tensor,
    kv: torch.Tensor,
    q_weight: torch.Tensor,
    kv_weight: torch.Tensor,
    eps: float,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(RMSNorm(qr) * q_weight, RMSNorm(kv) * kv_weight), row by row."""
    assert qr.ndim == 2 and kv.ndim == 2
    assert qr.shape[0] == kv.shape[0]
    assert qr.stride(-1) == 1 and kv.stride(-1) == 1
    assert q_weight.is_contiguous() and kv_weight.is_contiguous()

    q_size = qr.shape[1]
    kv_size = kv.shape[1]
    num_tokens = qr.shape[0]
    qr_out = torch.empty_like(qr)
    kv_out = torch.empty_like(kv)
    if num_tokens == 0:
        return qr_out, kv_out

    assert qr.dtype == torch.bfloat16 and kv.dtype == torch.bfloat16, "bf16 activations"
    assert q_weight.dtype == kv_weight.dtype and q_weight.dtype in (torch.bfloat16, torch.float32)
    assert q_weight.numel() == q_size and kv_weight.numel() == kv_size
    assert qr.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    for t in (kv, q_weight, kv_weight):
        assert t.device == qr.device, "all tensors must be on qr's device"
    with on_device_of(qr):
        rc = _native.lib().fgv_fused_q_kv_rmsnorm(
            qr.data_ptr(), qr.stride(0), qr_out.data_ptr(), qr_out.stride(0),
            q_weight.data_ptr(), q_size,
            kv.data_ptr(), kv.stride(0), kv_out.data_ptr(), kv_out.stride(0),
            kv_weight.data_ptr(), kv_size,
            num_tokens, float(eps), int(q_weight.dtype == torch.float32),
            current_stream_ptr(qr.device),
        )
    _native.check(rc, "fused_q_kv_rmsnorm")
    return qr_out, kv_out


__all__ = ["fused_q_kv_rmsnorm"]
