"""Sparse-indexer logits of FP8 or MXFP4 queries against FP8 index keys.

Drop-in for the reference op of the same name
(src/flaggems_vllm/ops/fp8_fp4_mqa_logits.py:523-651): same signature and
return value, a new float32 ``[M, N]`` tensor on the queries' device,

    logits[m, n] = sum_h ReLU((q[m, h] . k[n]) * k_scale[n]) * weights[m, h]

with ``-inf`` where ``n < cu_seqlen_ks[m]`` or ``n >= cu_seqlen_ke[m]`` when
``clean_logits``.  One launch of the gfx950 kernel ``mqa_logits_kernel``
through the C ABI ``fgv_fp8_fp4_mqa_logits`` on the current stream: FP8 q on
the 16x16x128 FP8 MFMA, MXFP4 q as its FP4 operand with the UE8M0 bytes as
hardware block scales.  With ``clean_logits`` the key tiles no query of a
workgroup can see are written as ``-inf`` without being computed.

Inputs as fused_indexer_q_rope_quant and cp_gather_indexer_k_quant_cache
produce them: q ``(values [M, H, 128] float8_e4m3fn, None)`` or
``(packed [M, H, 64] uint8, scale [M, H] or [M, H, 1] int32)``; kv
``(k [N, 128] float8_e4m3fn or uint8, k_scale [N] float32)``, k_scale
positive; weights ``[M, H]`` float32.  num_heads 16/32/64/128 and head_dim
128 (DeepSeek-V4's indexer; the MXFP4 scale word holds four blocks, so the
reference's MXFP4 path is also head_dim 128).  Where the reference takes
ReLU of ``dot * k_scale`` per head, this build multiplies the head sum by
k_scale once (the same value for k_scale > 0); head sums are binary32 in a
different order, within the bound the tests state.
"""
import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of

HEAD_DIM = 128


def _i32(t):
    return t if t.dtype == torch.int32 else t.to(torch.int32)


def fp8_fp4_mqa_logits(
    q: tuple,
    kv: tuple,
    weights: torch.Tensor,
    cu_seqlen_ks: torch.Tensor,
    cu_seqlen_ke: torch.Tensor,
    clean_logits: bool = True,
) -> torch.Tensor:
    q_values, q_scale = q
    k_values, k_scales = kv
    if q_scale is not None:
        M, H, D2 = q_values.shape
        D = D2 * 2
    else:
        M, H, D = q_values.shape
    N = k_values.shape[0]
    assert k_values.dim() == 2 and k_values.shape[1] == D
    assert q_values.element_size() == 1 and k_values.element_size() == 1, "q and k must be 1-byte codes"
    assert q_values.stride(-1) == 1 and k_values.stride(-1) == 1, "q and k rows must be contiguous"
    assert weights.shape == (M, H) and weights.dtype == torch.float32
    assert k_scales.numel() == N and k_scales.dtype == torch.float32
    k_scales = k_scales.reshape(N)
    assert k_scales.stride(0) == 1 or N <= 1
    for t in (k_values, k_scales, weights):
        assert t.device == q_values.device, "all tensors must be on q's device"
    assert q_values.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    qs = None
    if q_scale is not None:
        assert q_scale.dtype == torch.int32 and q_scale.numel() == M * H, "MXFP4 q_scale: int32 [M, H] (or [M, H, 1])"
        qs = q_scale.reshape(M, H)
    logits = torch.empty((M, N), dtype=torch.float32, device=q_values.device)
    if M == 0 or N == 0:
        return logits
    ks = ke = None
    if clean_logits:
        assert cu_seqlen_ks.numel() >= M and cu_seqlen_ke.numel() >= M
        ks = _i32(cu_seqlen_ks).reshape(-1).contiguous()
        ke = _i32(cu_seqlen_ke).reshape(-1).contiguous()
    with on_device_of(q_values):
        rc = _native.lib().fgv_fp8_fp4_mqa_logits(
            q_values.data_ptr(), q_values.stride(0), q_values.stride(1),
            qs.data_ptr() if qs is not None else None, qs.stride(0) if qs is not None else 0,
            qs.stride(1) if qs is not None else 0,
            k_values.data_ptr(), k_values.stride(0), k_scales.data_ptr(),
            weights.data_ptr(), weights.stride(0), weights.stride(1),
            ks.data_ptr() if ks is not None else None, ke.data_ptr() if ke is not None else None,
            logits.data_ptr(), logits.stride(0), M, N, H, D, int(bool(clean_logits)),
            current_stream_ptr(q_values.device),
        )
    _native.check(rc, "fp8_fp4_mqa_logits")
    return logits


__all__ = ["fp8_fp4_mqa_logits"]
