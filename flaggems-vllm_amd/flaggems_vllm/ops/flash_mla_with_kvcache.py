"""Sparse MLA decode over DeepSeek-V4's 584-byte MODEL1 cache.

Drop-in for the reference's ``flash_mla_with_kvcache`` /
``get_mla_metadata`` / ``FlashMLASchedMeta``
(src/flaggems_vllm/ops/flash_mla_with_kvcache.py:69-95, 852-1073) on the path
this package covers: sparse attention (``indices`` given) over FP8 MODEL1
caches (head_dim_k 512, 584 bytes per token), with optional top-k lengths,
attention sink, extra cache and caller-provided ``out``.  The argument checks
and the scheduler-metadata bookkeeping follow the reference's assertions one
for one; the launch goes to the gfx950 kernel ``sparse_mla_decode_kernel``
(C ABI ``fgv_sparse_mla_decode_model1``).

Not on this path, and rejected with NotImplementedError: dense paged decode
(``indices`` None) and the 656-byte V3.2 cache (head_dim_k 576).
"""
import dataclasses
from typing import Optional, Tuple

import torch

from .. import _native
from ._common import current_stream_ptr, on_device_of

MODEL1_TOKEN_BYTES = 584


@dataclasses.dataclass
class FlashMLASchedMeta:
    """Scheduler metadata handle (reference :69-89).  The first call records
    the call's configuration; later calls with the same handle must match it."""

    @dataclasses.dataclass
    class Config:
        b: int
        s_q: int
        h_q: int
        page_block_size: int
        h_k: int
        causal: bool
        is_fp8_kvcache: bool
        topk: Optional[int]
        extra_page_block_size: Optional[int]
        extra_topk: Optional[int]

    have_initialized: bool = False
    config: Optional[Config] = None
    tile_scheduler_metadata: Optional[torch.Tensor] = None
    num_splits: Optional[torch.Tensor] = None


def get_mla_metadata(*args, **kwargs) -> Tuple[FlashMLASchedMeta, None]:
    """A fresh FlashMLASchedMeta (reference :92-94); the kernel needs no
    precomputed schedule."""
    return FlashMLASchedMeta(), None


_MISMATCH = (" Your input arguments are inconsistent with sched_meta. Please make sure the input "
             "arguments are consistent across different invocations of flash_mla_with_kvcache on "
             "the same sched_meta.")


def _check_sched_meta(meta, cfg):
    if not meta.have_initialized:
        meta.have_initialized = True
        meta.config = cfg
        return
    assert meta.config is not None
    c = meta.config
    assert c.b == cfg.b, "sched_meta.config.b must be equal to batch_size." + _MISMATCH
    assert c.s_q == cfg.s_q, "sched_meta.config.s_q must be equal to seq_len_q." + _MISMATCH
    assert c.h_q == cfg.h_q, "sched_meta.config.h_q must be equal to num_heads_q." + _MISMATCH
    assert c.page_block_size == cfg.page_block_size, (
        "sched_meta.config.page_block_size must be equal to page_block_size." + _MISMATCH)
    assert c.h_k == cfg.h_k, "sched_meta.config.h_k must be equal to num_heads_k." + _MISMATCH
    assert c.causal == cfg.causal, "sched_meta.config.causal must be equal to causal." + _MISMATCH
    assert c.is_fp8_kvcache == cfg.is_fp8_kvcache, (
        "sched_meta.config.is_fp8_kvcache must be equal to is_fp8_kvcache." + _MISMATCH)
    assert c.topk == cfg.topk, (
        "sched_meta.config.topk must be equal to the last dim of indices." + _MISMATCH)
    assert c.extra_page_block_size == cfg.extra_page_block_size, (
        "sched_meta.config.extra_page_block_size must be equal to the page_block_size of "
        "extra_k_cache." + _MISMATCH)
    assert c.extra_topk == cfg.extra_topk, (
        "sched_meta.config.extra_topk must be equal to the last dim of "
        "extra_indices_in_kvcache." + _MISMATCH)


def _as_bytes(cache: torch.Tensor) -> torch.Tensor:
    return cache if cache.dtype == torch.uint8 else cache.view(torch.uint8)


def flash_mla_with_kvcache(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    block_table: Optional[torch.Tensor],
    cache_seqlens: Optional[torch.Tensor],
    head_dim_v: int,
    tile_scheduler_metadata: FlashMLASchedMeta,
    num_splits: None = None,
    softmax_scale: Optional[float] = None,
    causal: bool = False,
    is_fp8_kvcache: bool = False,
    indices: Optional[torch.Tensor] = None,
    attn_sink: Optional[torch.Tensor] = None,
    extra_k_cache: Optional[torch.Tensor] = None,
    extra_indices_in_kvcache: Optional[torch.Tensor] = None,
    topk_length: Optional[torch.Tensor] = None,
    extra_topk_length: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Returns ``(out, softmax_lse)``: out [batch, seq_q, num_heads_q,
    head_dim_v] in q's dtype and lse [batch, num_heads_q, seq_q] float32
    (natural log, sink excluded, +inf for rows that attend nothing)."""
    meta = tile_scheduler_metadata
    assert isinstance(meta, FlashMLASchedMeta)
    assert num_splits is None
    assert q.ndim == 4
    assert k_cache.ndim == 4
    topk = indices.shape[-1] if indices is not None else None
    extra_page = extra_k_cache.shape[1] if extra_k_cache is not None else None
    extra_topk = extra_indices_in_kvcache.shape[-1] if extra_indices_in_kvcache is not None else None
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** (-0.5)
    if not meta.have_initialized and indices is not None:
        assert not causal, "causal must be False when sparse attention is enabled"
    _check_sched_meta(meta, FlashMLASchedMeta.Config(
        q.shape[0], q.shape[1], q.shape[2], k_cache.shape[1], k_cache.shape[2], causal,
        is_fp8_kvcache, topk, extra_page, extra_topk))

    batch, seq_q, num_heads_q, head_dim_k = q.shape
    num_heads_k = k_cache.shape[2]
    if out is None:
        out = torch.empty((batch, seq_q, num_heads_q, head_dim_v), dtype=q.dtype, device=q.device)
    else:
        assert out.shape == (batch, seq_q, num_heads_q, head_dim_v)
        assert out.dtype == q.dtype
        assert out.device == q.device
        assert out.stride(-1) == 1
    lse = torch.empty((batch, num_heads_q, seq_q), dtype=torch.float32, device=q.device)

    if indices is None:
        assert (attn_sink is None and extra_k_cache is None and extra_indices_in_kvcache is None
                and topk_length is None and extra_topk_length is None), (
            "indices, attn_sink, extra_k_cache, extra_indices_in_kvcache, topk_length and "
            "extra_topk_length must be None when dense attention is used.")
        assert block_table is not None and cache_seqlens is not None, (
            "block_table and cache_seqlens must be provided when dense attention is used.")
        raise NotImplementedError("dense paged MLA decode is not part of this package")

    assert not causal, "causal must be False when sparse attention is enabled"
    assert is_fp8_kvcache, "is_fp8_kvcache must be True for sparse attention"
    assert num_heads_k == 1, "Currently only MQA (h_kv == 1) is supported for sparse decoding"
    assert head_dim_v == 512, "Only head_size_v == 512 is supported"
    assert num_heads_q in (64, 128), "Only h_q == 64 or 128 is supported"
    assert head_dim_k in (512, 576), "Only head_size_k == 512 or 576 is supported for sparse decoding"
    assert q.dtype == torch.bfloat16
    assert k_cache.dtype in (torch.float8_e4m3fn, torch.int8, torch.uint8)
    assert topk is not None and topk > 0
    assert topk % 64 == 0, "topk must be divisible by 64"
    assert indices.ndim == 3 and indices.shape[:2] == (batch, seq_q)
    assert indices.dtype == torch.int32
    assert indices.stride(-1) == 1
    if topk_length is not None:
        assert topk_length.shape == (batch,)
        assert topk_length.dtype == torch.int32
        assert topk_length.is_contiguous()
    if attn_sink is not None:
        assert attn_sink.shape == (num_heads_q,)
        assert attn_sink.dtype == torch.float32
    if extra_k_cache is not None:
        assert extra_indices_in_kvcache is not None, (
            "extra_indices_in_kvcache must be provided when extra_k_cache is provided")
        assert extra_k_cache.dtype in (torch.float8_e4m3fn, torch.int8, torch.uint8)
    else:
        assert extra_indices_in_kvcache is None, (
            "extra_indices_in_kvcache must not be provided when extra_k_cache is not provided")
        assert extra_topk_length is None, (
            "extra_topk_length must not be provided when extra_k_cache is not provided")
    if extra_indices_in_kvcache is not None:
        assert extra_indices_in_kvcache.ndim == 3
        assert extra_indices_in_kvcache.shape[:2] == (batch, seq_q)
        assert extra_indices_in_kvcache.dtype == torch.int32
        assert extra_indices_in_kvcache.stride(-1) == 1
        assert extra_indices_in_kvcache.shape[-1] % 64 == 0
    if extra_topk_length is not None:
        assert extra_topk_length.shape == (batch,)
        assert extra_topk_length.dtype == torch.int32
        assert extra_topk_length.is_contiguous()
    if head_dim_k == 576:
        assert k_cache.shape[-1] == 656, "V32 sparse FP8 cache must use 656 bytes per token"
        assert k_cache.stride(1) == 656, "The whole block must be contiguous for V32 KV cache"
        assert topk_length is None, "V3.2/V32 does not support dynamic topk length"
        assert extra_k_cache is None, "V3.2/V32 does not support extra KV cache"
        assert extra_indices_in_kvcache is None, "V3.2/V32 does not support extra indices"
        assert extra_topk_length is None, "V3.2/V32 does not support extra topk length"
        raise NotImplementedError("the 656-byte V3.2 sparse cache is not part of this package")
    assert k_cache.shape[-1] == MODEL1_TOKEN_BYTES, "MODEL1 sparse FP8 cache must use 584 bytes per token"
    assert k_cache.stride(1) == MODEL1_TOKEN_BYTES, "The whole block must be contiguous for MODEL1 KV cache"
    if extra_k_cache is not None:
        assert extra_k_cache.ndim == 4
        assert extra_k_cache.shape[2] == 1
        assert extra_k_cache.shape[-1] == MODEL1_TOKEN_BYTES
        assert extra_k_cache.stride(1) == MODEL1_TOKEN_BYTES

    assert q.device.type == "cuda", "flaggems_vllm runs on the GPU (HIP) only"
    for t in (k_cache, indices, topk_length, attn_sink, extra_k_cache, extra_indices_in_kvcache,
              extra_topk_length):
        assert t is None or t.device == q.device, "all tensors must be on q's device"
    assert q.stride(-1) == 1

    kc = _as_bytes(k_cache)
    ek = _as_bytes(extra_k_cache) if extra_k_cache is not None else None
    ei = extra_indices_in_kvcache
    ptr = lambda t: t.data_ptr() if t is not None else None
    with on_device_of(q):
        # a workspace for the balanced split schedule of long lists (cf. the
        # reference's lse_part / o_part, flash_mla_with_kvcache_model1.py:1588-1595)
        # and for a bf16 copy of an extra cache that is gathered many times over
        ws_bytes = _native.lib().fgv_sparse_mla_decode_workspace_bytes(
            batch, seq_q, num_heads_q, topk, extra_topk or 0,
            ek.shape[0] * ek.shape[1] if ek is not None else 0)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes > 0 else None
        rc = _native.lib().fgv_sparse_mla_decode_model1(
            q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
            kc.data_ptr(), kc.stride(0), kc.shape[0], kc.shape[1],
            indices.data_ptr(), indices.stride(0), indices.stride(1), topk, ptr(topk_length),
            ptr(ek), ek.stride(0) if ek is not None else 0, ek.shape[0] if ek is not None else 0,
            ek.shape[1] if ek is not None else 1,
            ptr(ei), ei.stride(0) if ei is not None else 0, ei.stride(1) if ei is not None else 0,
            extra_topk or 0, ptr(extra_topk_length),
            ptr(attn_sink), float(softmax_scale),
            out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
            lse.data_ptr(), lse.stride(0), lse.stride(1),
            batch, seq_q, num_heads_q, ptr(ws), ws_bytes, current_stream_ptr(q.device),
        )
    _native.check(rc, "flash_mla_with_kvcache")
    return out, lse


__all__ = ["FlashMLASchedMeta", "flash_mla_with_kvcache", "get_mla_metadata"]
