"""Fused DeepSeek-V4 q RMSNorm + RoPE, kv RoPE + UE8M0 FP8 quant + paged insert.

Drop-in for the reference op of the same name
(src/flaggems_vllm/ops/fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:289-351):
same positional signature, same in-place contract (q and k_cache mutated, kv
and the index tensors untouched), same AssertionError for the same bad inputs.
The argument checks and the launch run in C++ (``torch_ops.cpp``,
``qnorm_rope_kv_insert``): one launch of the gfx950 HIP kernel
``qnorm_rope_kv_insert_kernel`` through the C ABI
``fgv_qnorm_rope_kv_rope_quant_insert``, on the current stream, with no host
synchronisation and no allocation.  An eager call costs a few microseconds of
host time.

Beyond the reference: q and kv may be strided views (unit last stride, row
strides multiple of 8 elements), as when they are slices of one fused
projection buffer; cos_sin_cache's row stride is honoured; slots whose block
is past the end of k_cache are skipped and positions are clamped into the
cache's rows instead of being read out of bounds.
"""
import torch

from .. import _native

HEAD_DIM = 512
ROPE_DIM = 64


def cache_geometry(k_cache: torch.Tensor):
    """(num_blocks, block stride in bytes) the kernel addresses k_cache with
    (the rule the C++ op applies before its launch).

    A [num_blocks, block_bytes] cache (or any cache with more dimensions)
    has k_cache.shape[0] blocks, stride(0) bytes apart.  A 1-D cache is one
    block of numel bytes: slots past cache_block_size then fall in block >= 1,
    which the kernel's block bound skips, so nothing is written past its end.
    """
    if k_cache.dim() > 1:
        return k_cache.shape[0], k_cache.stride(0)
    return 1, k_cache.numel()


def fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(
    q: torch.Tensor,
    kv: torch.Tensor,
    k_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    position_ids: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    eps: float,
    cache_block_size: int,
):
    """Horizontally fused DeepSeek-V4 MLA pre-processing, in place.

    Args:
        q: [num_tokens, num_heads, 512] bf16, updated in place.
        kv: [num_tokens, 512] bf16, read only.
        k_cache: [num_blocks, block_bytes] uint8 paged cache.  Per block:
            cache_block_size x 576 B token data (448 e4m3fn codes + 64 bf16
            roped values), then cache_block_size x 8 B scales (7 UE8M0 bytes
            + 1 zero byte).  Only stride(0) is used between blocks.
        slot_mapping: [num_tokens_insert] int64, num_tokens_insert <= num_tokens;
            -1 marks a token that is not inserted.
        position_ids: [num_tokens] int64.
        cos_sin_cache: [max_pos, 64] float32, cos | sin.
        eps: RMSNorm epsilon.
        cache_block_size: tokens per cache block.
    """
    rc = _native.torch_ext().qnorm_rope_kv_insert(q, kv, k_cache, slot_mapping, position_ids, cos_sin_cache,
                                                  eps, cache_block_size)
    if rc:
        _native.raise_status(rc, "fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert")
