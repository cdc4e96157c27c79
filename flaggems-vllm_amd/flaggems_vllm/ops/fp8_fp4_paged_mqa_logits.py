"""Sparse-indexer logits over the paged FP8 key cache (decode).

Drop-in for the reference op of the same name
(src/flaggems_vllm/ops/fp8_fp4_paged_mqa_logits.py:410-579): same signature
and return value, a new float32 ``[B * next_n, max_model_len]`` tensor.  Row
``b * next_n + t`` holds, for positions ``n < context_lens`` of that row, the
logit of fp8_fp4_mqa_logits against position n of sequence b's keys, read
through ``block_tables[b]`` from the cache ``[num_blocks, block_size, 1, 132]``
that indexer_k_quant_and_cache writes (block_size x 128 e4m3fn bytes, then
block_size float32 scales); every other position is 0, or ``-inf`` with
``clean_logits``.  One launch of ``paged_mqa_logits_kernel`` through the C ABI
``fgv_fp8_fp4_paged_mqa_logits``, which writes every output element (no
separate fill pass).  ``schedule_metadata`` is accepted and unused, as in the
reference.

q: ``(values [B, next_n, H, 128] float8_e4m3fn, None)`` or ``(packed
[B, next_n, H, 64] uint8, scale [B, next_n, H] int32)`` (3-D q means
next_n = 1); weights ``[B * next_n, H]`` float32; context_lens ``[B]`` or
``[B, next_n]``; block_tables ``[B, max_blocks]`` (or one row per query row).
Block indices are clamped into the cache, as the reference does.  num_heads
16/32/64/128, head_dim 128.
"""
import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of


def _i32(t):
    return t if t.dtype == torch.int32 else t.to(torch.int32)


def fp8_fp4_paged_mqa_logits(
    q,
    kv_cache,
    weights,
    context_lens,
    block_tables,
    schedule_metadata,
    max_model_len,
    clean_logits=False,
):
    del schedule_metadata  # the reference ignores it too
    q_values, q_scale = q
    is_fp4 = q_scale is not None
    if q_values.dim() == 3:
        q_values = q_values.unsqueeze(1)
    B, next_n, H, q_last_dim = q_values.shape
    rows = B * next_n
    block_size = kv_cache.shape[1]
    head_dim = kv_cache.shape[3] - 4
    if is_fp4:
        assert q_last_dim == head_dim // 2
    else:
        assert q_last_dim == head_dim
    assert kv_cache.dim() == 4 and kv_cache.element_size() == 1 and kv_cache[0].is_contiguous()
    assert weights.shape == (rows, H) and weights.dtype == torch.float32
    q_rows = q_values.reshape(rows, H, q_last_dim)
    assert q_rows.stride(-1) == 1
    qs = q_scale.reshape(rows, H) if is_fp4 else None
    if qs is not None:
        assert qs.dtype == torch.int32
    ctx = _i32(context_lens)
    if ctx.dim() == 2:
        ctx, per_len = ctx.reshape(-1)[:rows].contiguous(), 1
    else:
        ctx, per_len = ctx.contiguous(), next_n
    bt = _i32(block_tables)
    if bt.dim() == 2 and bt.shape[0] == B:
        per_table = next_n
    else:
        bt, per_table = bt.reshape(rows, -1), 1
    assert bt.stride(-1) == 1, "block_tables rows must be contiguous"
    for t in (kv_cache, weights, ctx, bt):
        assert t.device == q_values.device, "all tensors must be on q's device"
    assert q_values.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    logits = torch.empty((rows, max_model_len), dtype=torch.float32, device=q_values.device)
    if rows == 0 or max_model_len == 0:
        return logits
    with on_device_of(q_values):
        rc = _native.lib().fgv_fp8_fp4_paged_mqa_logits(
            q_rows.data_ptr(), q_rows.stride(0), q_rows.stride(1),
            qs.data_ptr() if qs is not None else None, qs.stride(0) if qs is not None else 0,
            qs.stride(1) if qs is not None else 0,
            kv_cache.data_ptr(), kv_cache.stride(0), kv_cache.shape[0], block_size, head_dim,
            weights.data_ptr(), weights.stride(0), weights.stride(1),
            ctx.data_ptr(), per_len, bt.data_ptr(), bt.stride(0), bt.shape[1], per_table,
            logits.data_ptr(), logits.stride(0), rows, H, int(max_model_len), int(bool(clean_logits)),
            current_stream_ptr(q_values.device),
        )
    _native.check(rc, "fp8_fp4_paged_mqa_logits")
    return logits


__all__ = ["fp8_fp4_paged_mqa_logits"]
