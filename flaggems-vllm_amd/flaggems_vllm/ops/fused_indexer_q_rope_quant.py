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
q, float32 or bf16 cos/sin and bf16 or float32 weights.  The checks, the
allocations and the launch run in C++ (``torch_ops.cpp``,
``indexer_q_rope_quant``).
"""
import torch

from .. import _native

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
    rc, q_out, scale, index_weights_out = _native.torch_ext().indexer_q_rope_quant(
        positions, index_q, index_q_cos_sin_cache, index_weights, float(index_weights_softmax_scale),
        float(index_weights_head_scale), bool(use_fp4))
    if rc:
        _native.raise_status(rc, "fused_indexer_q_rope_quant")
    if use_fp4:
        return (q_out, scale), index_weights_out
    return q_out, index_weights_out


__all__ = ["fused_indexer_q_rope_quant"]
