"""Sparse MLA prefill over bf16 key/value rows.

Drop-in for the reference's ``flash_mla_sparse_fwd``
(src/flaggems_vllm/ops/flashmla_sparse.py:1045-1206): the same signature,
the same assertions in the same order, and the same three outputs (O, the
largest score and the log-sum-exp per query head).  The launch goes to the
gfx950 kernel ``sparse_mla_prefill_kernel`` (C ABI ``fgv_flash_mla_sparse_fwd``):
one workgroup per (token, 64-head block), the selected kv rows DMA'd into LDS
in chunks of 32 and attended on bf16 MFMAs, d_qk 512 or 576 (the last 64 dims
enter the scores only).
"""
from typing import Optional, Tuple

import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of


def flash_mla_sparse_fwd(
    q: torch.Tensor,
    kv: torch.Tensor,
    indices: torch.Tensor,
    sm_scale: float,
    d_v: int = 512,
    attn_sink: Optional[torch.Tensor] = None,
    topk_length: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Sparse attention prefill.

    q [s_q, h_q, d_qk] bf16, kv [s_kv, 1, d_qk] bf16, indices [s_q, 1, topk]
    int32 (entries < 0 or >= s_kv are not attended), optional attn_sink [h_q]
    float32 (rescales O by exp(lse) / (exp(lse) + exp(sink)); no effect on
    lse and max_logits) and topk_length [s_q] int32 (token t attends only its
    first topk_length[t] indices).  Returns (out [s_q, h_q, 512] bf16,
    max_logits [s_q, h_q] float32, lse [s_q, h_q] float32); a head that
    attends nothing gets out 0, max_logits -inf and lse +inf.
    """
    assert q.is_contiguous() and kv.is_contiguous() and indices.is_contiguous()
    assert q.dtype == torch.bfloat16 and kv.dtype == torch.bfloat16 and indices.dtype == torch.int32
    SQ, HQ, DQK = q.shape
    SKV, HKV, _ = kv.shape

    assert d_v == 512, "Unsupported d_v"

    assert kv.shape[-1] == DQK
    _, _, TOPK = indices.shape
    assert indices.shape == (SQ, HKV, TOPK)
    if attn_sink is not None:
        assert attn_sink.is_contiguous()
        assert attn_sink.dtype == torch.float32
        assert attn_sink.shape == (HQ,), "attn_sink error shape"
    if topk_length is not None:
        assert topk_length.is_contiguous()
        assert topk_length.dtype == torch.int32
        assert topk_length.shape == (SQ,), "topk_length error shape"

    assert HKV == 1, "h_kv is expected to be 1"
    assert HQ == 64 or HQ == 128, "Unsupported h_q"
    assert DQK == 576 or DQK == 512, "Unsupported d_qk"

    assert q.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    for t in (kv, indices, attn_sink, topk_length):
        assert t is None or t.device == q.device, "all tensors must be on q's device"

    output = torch.empty((SQ, HQ, d_v), device=q.device, dtype=q.dtype)
    max_logits = torch.empty((SQ, HQ), device=q.device, dtype=torch.float32)
    lse = torch.empty((SQ, HQ), device=q.device, dtype=torch.float32)
    if SQ == 0:
        return output, max_logits, lse

    ptr = lambda t: t.data_ptr() if t is not None else None
    with on_device_of(q):
        rc = _native.lib().fgv_flash_mla_sparse_fwd(
            q.data_ptr(), q.stride(0), q.stride(1),
            kv.data_ptr(), kv.stride(0), SKV,
            indices.data_ptr(), indices.stride(0), TOPK,
            ptr(topk_length), ptr(attn_sink), float(sm_scale),
            SQ, HQ, DQK,
            output.data_ptr(), output.stride(0), output.stride(1),
            max_logits.data_ptr(), max_logits.stride(0),
            lse.data_ptr(), lse.stride(0),
            current_stream_ptr(q.device),
        )
    _native.check(rc, "flash_mla_sparse_fwd")
    return output, max_logits, lse


__all__ = ["flash_mla_sparse_fwd"]
