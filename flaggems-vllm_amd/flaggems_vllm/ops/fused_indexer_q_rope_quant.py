"""Fused RoPE + quant of the DeepSeek-V4 sparse-indexer q, with weight folding.

Drop-in for the reference op of the same name
(src/flaggems_vllm/ops/fused_indexer_q_rope_quant.py:285-410): same signature,
same outputs and weight-fold contracts, one launch of the gfx950 kernel
``indexer_q_rope_quant_kernel`` through the C ABI
``fgv_fused_indexer_q_rope_quant`` on the current stream.

* FP8 (use_fp4=False): q_fp8 [T, H, D] float8_e4m3fn with one power-of-two
  scale per (token, head) that is folded into the weights:
  weights_out = weights * q_scale * softmax_scale * head_scale.
* MXFP4 (use_fp4=True): packed E2M1 values [T, H, D/2] uint8 and one UE8M0
  byte per 32 elements, returned as the int32 view [T, H] (D = 128);
  weights_out = weights * softmax_scale * head_scale.  The reference requires
  sm100 for this path; gfx950 converts to FP4 natively.

This build implements head_dim 128, 256 or 512 with a 64-dim rope tail, bf16
q, float32 or bf16 cos/sin and bf16 or float32 weights.
"""
import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of

MXFP4_BLOCK_SIZE = 32


def fused_indexer_q_rope_quant(
    positions: torch.Tensor,
    index_q: torch.Tensor,
    index_q_cos_sin_cache: torch.Tensor,
    # Index weights
    index_weights: torch.Tensor,
    index_weights_softmax_scale: float,
    index_weights_head_scale: float,
    use_fp4: bool = False,
):
    """Returns (q_fp8, weights_out), or ((q_packed, q_scale), weights_out) with use_fp4."""
    assert positions.ndim == 1
    assert index_q.ndim == 3
    assert index_q_cos_sin_cache.ndim == 2

    num_tokens = positions.shape[0]
    num_index_q_heads = index_q.shape[1]
    index_q_head_dim = index_q.shape[2]

    index_weights_out = torch.empty_like(index_weights, dtype=torch.float32)

    assert index_q.dtype == torch.bfloat16 and index_q.stride(-1) == 1
    assert index_q.shape[0] >= num_tokens
    assert index_q_cos_sin_cache.shape[-1] == 64, "rope dim 64"
    assert index_q_cos_sin_cache.dtype in (torch.float32, torch.bfloat16)
    assert index_q_cos_sin_cache.stride(-1) == 1
    assert index_weights.dtype in (torch.bfloat16, torch.float32)
    assert index_weights.ndim == 2 and index_weights.stride(-1) == 1
    assert index_weights.shape[0] >= num_tokens and index_weights.shape[1] == num_index_q_heads
    assert index_q_head_dim in (128, 256, 512), "head_dim 128, 256 or 512"
    assert index_q.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    for t in (positions, index_q_cos_sin_cache, index_weights):
        assert t.device == index_q.device, "all tensors must be on index_q's device"
    if positions.dtype != torch.int64 or positions.stride(0) != 1:
        positions = positions.to(torch.int64).contiguous()

    if use_fp4:
        assert index_q_head_dim % MXFP4_BLOCK_SIZE == 0, (
            f"head_dim={index_q_head_dim} must be a multiple of MXFP4 block "
            f"size {MXFP4_BLOCK_SIZE}"
        )
        num_scale_blocks = index_q_head_dim // MXFP4_BLOCK_SIZE
        q_out = torch.empty((num_tokens, num_index_q_heads, index_q_head_dim // 2),
                            dtype=torch.uint8, device=index_q.device)
        scale = torch.empty((num_tokens, num_index_q_heads, num_scale_blocks),
                            dtype=torch.uint8, device=index_q.device)
    else:
        # as the reference allocates it: index_q's shape (its rows may exceed
        # num_tokens; only the first num_tokens are written) and layout
        q_out = torch.empty_like(index_q, dtype=torch.float8_e4m3fn)
        assert q_out.stride(-1) == 1
        scale = None

    with on_device_of(index_q):
        rc = _native.lib().fgv_fused_indexer_q_rope_quant(
            positions.data_ptr(), num_tokens,
            index_q.data_ptr(), index_q.stride(0), index_q.stride(1),
            num_index_q_heads, index_q_head_dim,
            index_q_cos_sin_cache.data_ptr(), index_q_cos_sin_cache.stride(0),
            index_q_cos_sin_cache.shape[0], int(index_q_cos_sin_cache.dtype == torch.bfloat16),
            index_weights.data_ptr(), index_weights.stride(0),
            int(index_weights.dtype == torch.float32),
            float(index_weights_softmax_scale), float(index_weights_head_scale),
            index_weights_out.data_ptr(), index_weights_out.stride(0),
            int(bool(use_fp4)),
            q_out.data_ptr(), q_out.stride(0), q_out.stride(1),
            scale.data_ptr() if scale is not None else None,
            scale.stride(0) if scale is not None else 0,
            scale.stride(1) if scale is not None else 0,
            current_stream_ptr(index_q.device),
        )
    _native.check(rc, "fused_indexer_q_rope_quant")
    if use_fp4:
        return (q_out, scale.view(torch.int32).squeeze(-1)), index_weights_out
    return q_out, index_weights_out


__all__ = ["fused_indexer_q_rope_quant"]
