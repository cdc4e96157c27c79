"""CPU oracle for the DeepSeek-V4 attention pre-processing path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` import this package, and only as the
checker.  The product (``flaggems_vllm`` and its HIP library) never imports it.

Two restatements of the reference live here:

* ``liboracle_dsv4.so`` (``dsv4_oracle.c``): scalar C, the bit-level checker.
  Its RMSNorm factor is the correctly rounded one (see the C header), which the
  HIP kernel shares, so q is compared bit for bit against it.
* ``torch_ref``: the reference's own PyTorch formulation
  (tests/test_fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:68-333,
  tests/test_fused_inv_rope_fp8_quant.py:132-198) restated on CPU tensors.  It
  is what the north-star tolerance (q within 1 bf16 ulp) is measured against,
  and it is the "reference PyTorch path" timed as the CPU baseline.

The C library is pinned by tests/test_oracle_pins.py; the torch restatement is
pinned against the C library and against closed forms there as well.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# FGV_ORACLE_LIB selects another build of the same source, e.g. the
# AddressSanitizer/UBSan one from `make -C oracle sanitize`.
_LIB_PATH = os.environ.get("FGV_ORACLE_LIB") or os.path.join(_HERE, "liboracle_dsv4.so")
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def build():
    """Compile the C oracle in place (gcc, via the Makefile next to it)."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"oracle library {_LIB_PATH} is not built; run `make -C oracle`"
            )
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_e4m3fn.restype = ctypes.c_uint8
        L.oracle_e4m3fn.argtypes = [ctypes.c_float]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_kv_ue8m0_exponent.restype = ctypes.c_int
        L.oracle_kv_ue8m0_exponent.argtypes = [ctypes.c_float]
        L.oracle_rms_factor.restype = ctypes.c_float
        L.oracle_rms_factor.argtypes = [_P, ctypes.c_float]
        L.oracle_e4m3fn_array.restype = None
        L.oracle_e4m3fn_array.argtypes = [_P, _P, _I64]
        L.oracle_f32_to_bf16_array.restype = None
        L.oracle_f32_to_bf16_array.argtypes = [_P, _P, _I64]
        L.oracle_qnorm_rope_kv_insert.restype = None
        L.oracle_qnorm_rope_kv_insert.argtypes = [
            _P, _I64, _I64,  # q, q_st, q_sh
            _P, _I64,  # kv, kv_st
            _P, _I64, _I64,  # k_cache, block_stride, num_blocks
            _P, _I64,  # slot_mapping, num_tokens_insert
            _P,  # position_ids
            _P, _I64, _I64,  # cos_sin, cs_stride, max_pos
            _I64, _I64,  # num_tokens, num_heads
            ctypes.c_float, _I64, ctypes.c_int,  # eps, block_size, nthreads
        ]
        L.oracle_inv_rope_fp8_quant.restype = None
        L.oracle_inv_rope_fp8_quant.argtypes = [
            _P, _I64, _I64,  # o, o_st, o_sh
            _P, _P, _I64, _I64,  # positions, cos_sin, cs_stride, max_pos
            _I64, _I64, _I64,  # num_tokens, n_groups, heads_per_group
            _I64, _I64, _I64,  # nope_dim, rope_dim, quant_group_size
            _P, _I64, _I64,  # fp8, fp8_sg, fp8_st
            _P, _I64, _I64, _I64,  # scale, sc_sg, sc_sk, tpad
            ctypes.c_float, ctypes.c_int, ctypes.c_int,  # eps, tma, nthreads
        ]
        L.oracle_e4m3fn_to_f32.restype = ctypes.c_float
        L.oracle_e4m3fn_to_f32.argtypes = [ctypes.c_uint8]
        L.oracle_e4m3fn_decode_array.restype = None
        L.oracle_e4m3fn_decode_array.argtypes = [_P, _P, _I64]
        L.oracle_dequantize_and_gather_k_cache.restype = None
        L.oracle_dequantize_and_gather_k_cache.argtypes = [
            _P, _I64, _I64, _I64,  # out, out_s0, out_s1, out_rows
            _P, _I64, _I64,  # cache, block_stride, num_blocks
            _P, _P,  # seq_lens, gather_lens
            _P, _I64, _I64,  # block_table, bt_stride, max_blocks
            _I64, _I64, _I64,  # num_reqs, bs, offset
            _I64, _I64, _I64,  # nope, rope, scale_slots
        ]
        L.oracle_fused_q_kv_rmsnorm.restype = None
        L.oracle_fused_q_kv_rmsnorm.argtypes = [
            _P, _I64, _P, _I64, _P, _I64,
            _P, _I64, _P, _I64, _P, _I64,
            _I64, ctypes.c_float, ctypes.c_int, ctypes.c_int,
        ]
        L.oracle_e2m1.restype = ctypes.c_uint8
        L.oracle_e2m1.argtypes = [ctypes.c_float]
        L.oracle_e2m1_array.restype = None
        L.oracle_e2m1_array.argtypes = [_P, _P, _I64]
        L.oracle_fused_indexer_q_rope_quant.restype = None
        L.oracle_fused_indexer_q_rope_quant.argtypes = [
            _P, _I64, _P, _I64, _I64, _I64, _I64,
            _P, _I64, _I64, ctypes.c_int, _P, _I64, ctypes.c_int,
            ctypes.c_float, ctypes.c_float, _P, _I64, ctypes.c_int,
            _P, _I64, _I64, _P, _I64, _I64,
        ]
        L.oracle_compute_slot_mapping.restype = None
        L.oracle_compute_slot_mapping.argtypes = [
            _I64, _I64, _P, _I64, _P, ctypes.c_int, _P, _I64, _I64, _P, _I64,
            _I64, _I64, _I64, _I64,
        ]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_indexer_k_quant_and_cache.restype = None
        L.oracle_indexer_k_quant_and_cache.argtypes = [
            _P, _I64, ctypes.c_int, _I64, _I64, _I64,  # k, k_st, fp16, T, head_dim, qbs
            _P, _I64, _I64, _I64,  # cache, block_stride, num_blocks, block_size
            _P, ctypes.c_int,  # slots, ue8m0
        ]
        L.oracle_cp_gather_indexer_k_quant_cache.restype = None
        L.oracle_cp_gather_indexer_k_quant_cache.argtypes = [
            _P, _I64, _I64, _I64, _I64, _I64,  # cache, block_stride, num_blocks, block_size, head_dim, qbs
            _P, _I64, _P, _I64,  # k_out, stride, scale_out, stride (bytes)
            _P, _I64, _I64,  # block_table, stride, max_blocks
            _P, _I64, _I64,  # cu, batch, T
        ]
        L.oracle_mqa_logits.restype = None
        L.oracle_mqa_logits.argtypes = [
            _P, _I64, _I64, _P, _I64, _I64,  # q, strides (bytes), q_scale, strides
            _P, _I64, _P, _P, _I64, _I64,  # k, stride, k_scale, w, strides
            _P, _P, ctypes.c_int, _I64, _I64, _I64,  # ks, ke, clean, N, H, D
            _P, _I64, _P, _P,  # rows, nrows, out, bound
        ]
        L.oracle_paged_mqa_logits.restype = None
        L.oracle_paged_mqa_logits.argtypes = [
            _P, _I64, _I64, _P, _I64, _I64,  # q, strides, q_scale, strides
            _P, _I64, _I64, _I64,  # kv, block stride, num_blocks, block_size
            _P, _I64, _I64,  # w, strides
            _P, _I64, _P, _I64, _I64, _I64,  # ctx, per len, bt, stride, max blocks, per table
            _I64, _I64, _I64, ctypes.c_float,  # H, D, max_model_len, fill
            _P, _I64, _P, _P,  # rows, nrows, out, bound
        ]
        L.oracle_model1_token_row.restype = None
        L.oracle_model1_token_row.argtypes = [_P, _I64, _I64, _I64, _P]
        L.oracle_sparse_mla_decode_model1.restype = None
        L.oracle_sparse_mla_decode_model1.argtypes = [
            _P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _P,
            _P, _I64, _I64, _I64, _P, _I64, _P, _P, ctypes.c_double, _P, _P,
        ]
        L.oracle_sparse_mla_prefill.restype = None
        L.oracle_sparse_mla_prefill.argtypes = [
            _P, _P, _I64, _I64, _P, _I64, _P, _P, ctypes.c_double, _I64, _I64, _I64, _P, _P, _P,
        ]
        L.oracle_compute_global_topk_indices.restype = None
        L.oracle_compute_global_topk_indices.argtypes = [
            _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _P]
        L.oracle_combine_topk_swa_indices.restype = None
        L.oracle_combine_topk_swa_indices.argtypes = [
            _P, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P]
        L.oracle_top_k_per_row.restype = None
        L.oracle_top_k_per_row.argtypes = [_P, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _I64, _P]
        L.oracle_fp8_einsum.restype = None
        L.oracle_fp8_einsum.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P]
        _lib = L
    return _lib


def _threads(nthreads):
    if nthreads is None:
        return len(os.sched_getaffinity(0))
    return int(nthreads)


def _cpu(t, dtype=None):
    assert t.device.type == "cpu", "the oracle works on CPU tensors"
    if dtype is not None:
        assert t.dtype == dtype, f"expected {dtype}, got {t.dtype}"
    return t


def e4m3fn_codes(x: torch.Tensor) -> torch.Tensor:
    """uint8 e4m3fn codes of a float32 CPU tensor (RNE, no saturation)."""
    x = _cpu(x, torch.float32).contiguous()
    out = torch.empty(x.shape, dtype=torch.uint8)
    lib().oracle_e4m3fn_array(x.data_ptr(), out.data_ptr(), x.numel())
    return out


def bf16_bits(x: torch.Tensor) -> torch.Tensor:
    """bf16 bit patterns (as int16) of a float32 CPU tensor, RNE."""
    x = _cpu(x, torch.float32).contiguous()
    out = torch.empty(x.shape, dtype=torch.int16)
    lib().oracle_f32_to_bf16_array(x.data_ptr(), out.data_ptr(), x.numel())
    return out


def kv_ue8m0_exponent(amax: float) -> int:
    return lib().oracle_kv_ue8m0_exponent(amax)


def rms_factor(row: torch.Tensor, eps: float) -> float:
    row = _cpu(row, torch.bfloat16).contiguous()
    assert row.numel() == 512
    return lib().oracle_rms_factor(row.data_ptr(), eps)


def qnorm_rope_kv_insert(q, kv, k_cache, slot_mapping, position_ids, cos_sin_cache,
                         eps, cache_block_size, nthreads=None):
    """In-place CPU restatement of the main op on CPU tensors (same argument
    meaning as flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert).
    q and kv may be strided views with a unit last stride."""
    _cpu(q, torch.bfloat16), _cpu(kv, torch.bfloat16), _cpu(k_cache, torch.uint8)
    _cpu(slot_mapping, torch.int64), _cpu(position_ids, torch.int64)
    _cpu(cos_sin_cache, torch.float32)
    T, H, D = q.shape
    assert D == 512 and q.stride(2) == 1 and kv.stride(1) == 1
    assert cos_sin_cache.stride(1) == 1 and cos_sin_cache.shape[1] == 64
    slot_mapping = slot_mapping.contiguous()
    position_ids = position_ids.contiguous()
    lib().oracle_qnorm_rope_kv_insert(
        q.data_ptr(), q.stride(0), q.stride(1),
        kv.data_ptr(), kv.stride(0),
        k_cache.data_ptr(), k_cache.stride(0), k_cache.shape[0],
        slot_mapping.data_ptr(), slot_mapping.shape[0],
        position_ids.data_ptr(),
        cos_sin_cache.data_ptr(), cos_sin_cache.stride(0), cos_sin_cache.shape[0],
        T, H, float(eps), int(cache_block_size), _threads(nthreads),
    )


def inv_rope_fp8_quant(o, positions, cos_sin_cache, n_groups, heads_per_group,
                       eps=1e-10, tma_aligned_scales=False, nthreads=None, nope_dim=448, rope_dim=64,
                       quant_group_size=128):
    """CPU restatement of the sibling op.  Returns (fp8 codes as uint8 [T, G, d]
    with the reference's strides, scales [T, G, K] with the reference's
    token-fastest padded storage: float32, or int32 when packed).  Any
    geometry the reference's assertions accept (head_dim = nope_dim +
    rope_dim, quant_group_size | head_dim, rope in the last chunk); packed
    scales need four chunks per head or one head per group, as the
    reference's packed scale tensor only then holds every head's word."""
    _cpu(o, torch.bfloat16), _cpu(positions, torch.int64), _cpu(cos_sin_cache, torch.float32)
    T, H, D = o.shape
    G = quant_group_size
    assert D == nope_dim + rope_dim and D % G == 0 and nope_dim % G == G - rope_dim and rope_dim % 2 == 0
    assert o.stride(2) == 1 and H == n_groups * heads_per_group and cos_sin_cache.shape[1] == rope_dim
    chunks = D // G
    assert not tma_aligned_scales or chunks == 4 or (chunks < 4 and heads_per_group == 1)
    d = heads_per_group * D
    k_blocks = d // G
    tpad = (T + 3) // 4 * 4
    inner = (k_blocks + 3) // 4 if tma_aligned_scales else k_blocks
    fp8 = torch.empty((n_groups, T, d), dtype=torch.uint8)
    sdt = torch.int32 if tma_aligned_scales else torch.float32
    scale = torch.empty(n_groups * inner * tpad, dtype=sdt).as_strided(
        (n_groups, T, inner), (inner * tpad, 1, tpad))
    positions = positions.contiguous()
    lib().oracle_inv_rope_fp8_quant(
        o.data_ptr(), o.stride(0), o.stride(1),
        positions.data_ptr(), cos_sin_cache.data_ptr(), cos_sin_cache.stride(0),
        cos_sin_cache.shape[0], T, n_groups, heads_per_group, nope_dim, rope_dim, G,
        fp8.data_ptr(), fp8.stride(0), fp8.stride(1),
        scale.data_ptr(), scale.stride(0), scale.stride(2), tpad,
        float(eps), int(bool(tma_aligned_scales)), _threads(nthreads),
    )
    return fp8.transpose(0, 1), scale.transpose(0, 1)


def e4m3fn_decode(codes: torch.Tensor) -> torch.Tensor:
    """float32 values of uint8 e4m3fn codes."""
    codes = _cpu(codes, torch.uint8).contiguous()
    out = torch.empty(codes.shape, dtype=torch.float32)
    lib().oracle_e4m3fn_decode_array(codes.data_ptr(), out.data_ptr(), codes.numel())
    return out


def dequantize_and_gather_k_cache(out, k_cache, seq_lens, gather_lens, block_table, block_size,
                                  offset=0, rope_dim=64, nope_dim=None, scale_slots=None):
    """CPU restatement, in place on ``out`` (same arguments as
    flaggems_vllm.dequantize_and_gather_k_cache; int32 index tensors)."""
    _cpu(out, torch.bfloat16), _cpu(k_cache, torch.uint8)
    if nope_dim is None:
        nope_dim = out.shape[-1] - rope_dim
    if scale_slots is None:
        scale_slots = (nope_dim + 63) // 64 + (1 if nope_dim % 64 == 0 else 0)
    seq_lens = _cpu(seq_lens, torch.int32).contiguous()
    if gather_lens is not None:
        gather_lens = _cpu(gather_lens, torch.int32).contiguous()
    block_table = _cpu(block_table, torch.int32)
    assert out.stride(-1) == 1 and block_table.stride(-1) == 1
    lib().oracle_dequantize_and_gather_k_cache(
        out.data_ptr(), out.stride(0), out.stride(1), out.shape[1],
        k_cache.data_ptr(), k_cache.stride(0), k_cache.shape[0],
        seq_lens.data_ptr(), gather_lens.data_ptr() if gather_lens is not None else None,
        block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
        seq_lens.shape[0], int(block_size), int(offset), int(nope_dim), int(rope_dim),
        int(scale_slots),
    )


def fused_q_kv_rmsnorm(qr, kv, q_weight, kv_weight, eps, nthreads=None):
    """CPU restatement: returns (qr_out, kv_out) as contiguous bf16 tensors."""
    _cpu(qr, torch.bfloat16), _cpu(kv, torch.bfloat16)
    assert q_weight.dtype == kv_weight.dtype and q_weight.dtype in (torch.bfloat16, torch.float32)
    assert qr.stride(-1) == 1 and kv.stride(-1) == 1
    q_weight, kv_weight = q_weight.contiguous(), kv_weight.contiguous()
    qo = torch.empty(qr.shape, dtype=torch.bfloat16)
    ko = torch.empty(kv.shape, dtype=torch.bfloat16)
    lib().oracle_fused_q_kv_rmsnorm(
        qr.data_ptr(), qr.stride(0), qo.data_ptr(), qo.stride(0), q_weight.data_ptr(), qr.shape[1],
        kv.data_ptr(), kv.stride(0), ko.data_ptr(), ko.stride(0), kv_weight.data_ptr(), kv.shape[1],
        qr.shape[0], float(eps), int(q_weight.dtype == torch.float32), _threads(nthreads))
    return qo, ko


def e2m1_codes(x: torch.Tensor) -> torch.Tensor:
    """uint8 E2M1 nibbles (sign in bit 3) of a float32 CPU tensor."""
    x = _cpu(x, torch.float32).contiguous()
    out = torch.empty(x.shape, dtype=torch.uint8)
    lib().oracle_e2m1_array(x.data_ptr(), out.data_ptr(), x.numel())
    return out


def fused_indexer_q_rope_quant(positions, index_q, cos_sin, weights, softmax_scale, head_scale,
                               use_fp4=False):
    """CPU restatement.  Returns (q_fp8 codes uint8 [T, H, D], weights_out) or
    ((packed uint8 [T, H, D/2], scale bytes uint8 [T, H, D/32]), weights_out)."""
    _cpu(index_q, torch.bfloat16)
    T = positions.shape[0]
    _, H, D = index_q.shape
    positions = positions.to(torch.int64).contiguous()
    weights_out = torch.empty(weights.shape, dtype=torch.float32)
    if use_fp4:
        qo = torch.empty(T, H, D // 2, dtype=torch.uint8)
        so = torch.empty(T, H, D // 32, dtype=torch.uint8)
    else:
        qo = torch.empty(T, H, D, dtype=torch.uint8)
        so = torch.empty(1, 1, 1, dtype=torch.uint8)
    lib().oracle_fused_indexer_q_rope_quant(
        positions.data_ptr(), T, index_q.data_ptr(), index_q.stride(0), index_q.stride(1), H, D,
        cos_sin.data_ptr(), cos_sin.stride(0), cos_sin.shape[0], int(cos_sin.dtype == torch.bfloat16),
        weights.data_ptr(), weights.stride(0), int(weights.dtype == torch.float32),
        float(softmax_scale), float(head_scale), weights_out.data_ptr(), weights_out.stride(0),
        int(bool(use_fp4)), qo.data_ptr(), qo.stride(0), qo.stride(1),
        so.data_ptr(), so.stride(0), so.stride(1))
    if use_fp4:
        return (qo, so), weights_out
    return qo, weights_out


def compute_slot_mapping(num_tokens, max_num_tokens, query_start_loc, num_reqs, positions,
                         block_table, slot_mapping, block_size, cp_world_size=1, cp_rank=0,
                         cp_kv_cache_interleave_size=1, pad_id=-1):
    """CPU restatement, in place on ``slot_mapping`` (int64 CPU tensor)."""
    qsl = _cpu(query_start_loc, torch.int32).contiguous()
    positions = _cpu(positions).contiguous()
    bt = _cpu(block_table, torch.int32)
    _cpu(slot_mapping, torch.int64)
    lib().oracle_compute_slot_mapping(
        int(num_tokens), int(max_num_tokens), qsl.data_ptr(), int(num_reqs), positions.data_ptr(),
        int(positions.dtype == torch.int64), bt.data_ptr(), bt.stride(0), bt.shape[1],
        slot_mapping.data_ptr(), int(block_size), int(cp_world_size), int(cp_rank),
        int(cp_kv_cache_interleave_size), int(pad_id))


def model1_token_row(k_cache, token_id):
    """The dequantised 512-wide bf16 row of cache entry ``token_id`` of a
    [num_blocks, page, 1, 584] uint8 MODEL1 cache."""
    _cpu(k_cache, torch.uint8)
    row = torch.empty(512, dtype=torch.bfloat16)
    lib().oracle_model1_token_row(k_cache.data_ptr(), k_cache.stride(0), k_cache.shape[1],
                                  int(token_id), row.data_ptr())
    return row


def sparse_mla_decode_model1(q, k_cache, indices, topk_length=None, attn_sink=None,
                             extra_k_cache=None, extra_indices=None, extra_topk_length=None,
                             softmax_scale=None):
    """Exact (binary64) sparse MLA decode over MODEL1 caches.

    Returns ``(out, lse)`` as float64 tensors shaped [B, SQ, HQ, 512] and
    [B, HQ, SQ]; arguments as in flaggems_vllm.flash_mla_with_kvcache."""
    q = _cpu(q, torch.bfloat16).contiguous()
    B, SQ, HQ, D = q.shape
    assert D == 512
    if softmax_scale is None:
        softmax_scale = D ** -0.5

    def cache_args(cache, idx, length):
        if cache is None:
            return [None, 0, 1, 0, None, 0, None], []
        _cpu(cache, torch.uint8)
        idx = _cpu(idx, torch.int32).contiguous()
        keep = [idx]
        lp = None
        if length is not None:
            length = _cpu(length, torch.int32).contiguous()
            keep.append(length)
            lp = length.data_ptr()
        return [cache.data_ptr(), cache.shape[0], cache.shape[1], cache.stride(0), idx.data_ptr(),
                idx.shape[-1], lp], keep

    main, keep0 = cache_args(k_cache, indices, topk_length)
    extra, keep1 = cache_args(extra_k_cache, extra_indices, extra_topk_length)
    sink = None
    if attn_sink is not None:
        sink = _cpu(attn_sink, torch.float32).contiguous()
    out = torch.empty(B, SQ, HQ, D, dtype=torch.float64)
    lse = torch.empty(B, HQ, SQ, dtype=torch.float64)
    lib().oracle_sparse_mla_decode_model1(
        q.data_ptr(), B, SQ, HQ, *main, *extra,
        sink.data_ptr() if sink is not None else None, float(softmax_scale),
        out.data_ptr(), lse.data_ptr())
    del keep0, keep1
    return out, lse


def sparse_mla_prefill(q, kv, indices, sm_scale, attn_sink=None, topk_length=None):
    """Exact (binary64) sparse MLA prefill over bf16 rows.

    Returns ``(out, max_logits, lse)`` as float64 tensors shaped
    [s_q, h_q, 512], [s_q, h_q], [s_q, h_q]; arguments as in
    flaggems_vllm.flash_mla_sparse_fwd (kv [s_kv, 1, d_qk] or [s_kv, d_qk],
    indices [s_q, 1, topk] or [s_q, topk])."""
    q = _cpu(q, torch.bfloat16).contiguous()
    s_q, h_q, d_qk = q.shape
    kv = _cpu(kv, torch.bfloat16).reshape(kv.shape[0], -1).contiguous()
    assert kv.shape[1] == d_qk
    idx = _cpu(indices, torch.int32).reshape(s_q, -1).contiguous()
    sink = _cpu(attn_sink, torch.float32).contiguous() if attn_sink is not None else None
    tl = _cpu(topk_length, torch.int32).contiguous() if topk_length is not None else None
    out = torch.empty(s_q, h_q, 512, dtype=torch.float64)
    ml = torch.empty(s_q, h_q, dtype=torch.float64)
    lse = torch.empty(s_q, h_q, dtype=torch.float64)
    lib().oracle_sparse_mla_prefill(
        q.data_ptr(), kv.data_ptr(), kv.stride(0), kv.shape[0], idx.data_ptr(), idx.shape[1],
        tl.data_ptr() if tl is not None else None, sink.data_ptr() if sink is not None else None,
        float(sm_scale), s_q, h_q, d_qk, out.data_ptr(), ml.data_ptr(), lse.data_ptr())
    return out, ml, lse


def _cache_bytes(kv_cache):
    """(flat uint8 view, block stride bytes, num_blocks, block_size) of a
    [num_blocks, block_size, head_dim + 4 * head_dim / 128] uint8 cache."""
    _cpu(kv_cache, torch.uint8)
    assert kv_cache.dim() == 3 and kv_cache[0].is_contiguous()
    return kv_cache, kv_cache.stride(0), kv_cache.shape[0], kv_cache.shape[1]


def indexer_k_quant_and_cache(k, kv_cache, slot_mapping, quant_block_size, scale_fmt):
    """CPU restatement, in place on ``kv_cache`` (same arguments as
    flaggems_vllm.ops.indexer_k_quant_and_cache; k bf16 or fp16)."""
    _cpu(k)
    assert k.dtype in (torch.bfloat16, torch.float16) and k.stride(-1) == 1
    cache, bstride, nblk, bs = _cache_bytes(kv_cache)
    slots = _cpu(slot_mapping, torch.int64).contiguous()
    lib().oracle_indexer_k_quant_and_cache(
        k.data_ptr(), k.stride(0), int(k.dtype == torch.float16), slots.shape[0], k.shape[-1],
        int(quant_block_size), cache.data_ptr(), bstride, nblk, bs, slots.data_ptr(),
        int(scale_fmt == "ue8m0"))


def cp_gather_indexer_k_quant_cache(k_cache, k_fp8, k_fp8_scale, block_table, cu_seqlen):
    """CPU restatement, in place on ``k_fp8`` / ``k_fp8_scale`` (same arguments
    as flaggems_vllm.ops.cp_gather_indexer_k_quant_cache; k_fp8_scale holds
    4 * head_dim / quant_block_size bytes per row).  Positions whose table
    index or block is out of range are skipped."""
    cache, bstride, nblk, bs = _cache_bytes(k_cache)
    head_dim = k_fp8.shape[-1]
    qbs = head_dim * 4 // (k_fp8_scale.shape[1] * k_fp8_scale.element_size())
    kb = _cpu(k_fp8).view(torch.uint8)
    sb = _cpu(k_fp8_scale).view(torch.uint8)
    bt = _cpu(block_table, torch.int32)
    cu = _cpu(cu_seqlen, torch.int32).contiguous()
    assert kb.stride(-1) == 1 and sb.stride(-1) == 1 and bt.stride(-1) == 1
    assert cu.numel() >= bt.shape[0] + 1
    lib().oracle_cp_gather_indexer_k_quant_cache(
        cache.data_ptr(), bstride, nblk, bs, head_dim, qbs, kb.data_ptr(), kb.stride(0), sb.data_ptr(),
        sb.stride(0), bt.data_ptr(), bt.stride(0), bt.shape[1], cu.data_ptr(), bt.shape[0], kb.shape[0])


def _rows_arg(rows, total):
    rows = torch.arange(total, dtype=torch.int64) if rows is None else torch.as_tensor(rows, dtype=torch.int64)
    return rows.contiguous()


def mqa_logits(q, kv, weights, cu_seqlen_ks, cu_seqlen_ke, clean_logits=True, rows=None):
    """Binary64 logits and error bound ([len(rows), N] float64 each) of
    flaggems_vllm.fp8_fp4_mqa_logits for the listed query rows (all by
    default); CPU tensors, same argument forms as the product."""
    q_values, q_scale = q
    k_values, k_scales = kv
    M, H = q_values.shape[0], q_values.shape[1]
    D = q_values.shape[2] * (2 if q_scale is not None else 1)
    N = k_values.shape[0]
    qv = _cpu(q_values).view(torch.uint8)
    kb = _cpu(k_values).view(torch.uint8)
    assert qv.stride(-1) == 1 and kb.stride(-1) == 1
    ksc = _cpu(k_scales, torch.float32).reshape(N).contiguous()
    w = _cpu(weights, torch.float32)
    qs = _cpu(q_scale, torch.int32).reshape(M, H) if q_scale is not None else None
    ks = _cpu(cu_seqlen_ks).to(torch.int32).contiguous() if clean_logits else None
    ke = _cpu(cu_seqlen_ke).to(torch.int32).contiguous() if clean_logits else None
    r = _rows_arg(rows, M)
    out = torch.empty(r.numel(), N, dtype=torch.float64)
    bound = torch.empty_like(out)
    lib().oracle_mqa_logits(
        qv.data_ptr(), qv.stride(0), qv.stride(1), qs.data_ptr() if qs is not None else None,
        qs.stride(0) if qs is not None else 0, qs.stride(1) if qs is not None else 0,
        kb.data_ptr(), kb.stride(0), ksc.data_ptr(), w.data_ptr(), w.stride(0), w.stride(1),
        ks.data_ptr() if ks is not None else None, ke.data_ptr() if ke is not None else None,
        int(bool(clean_logits)), N, H, D, r.data_ptr(), r.numel(), out.data_ptr(), bound.data_ptr())
    return out, bound


def paged_mqa_logits(q, kv_cache, weights, context_lens, block_tables, max_model_len, clean_logits=False,
                     rows=None):
    """Binary64 logits and error bound ([len(rows), max_model_len] float64) of
    flaggems_vllm.fp8_fp4_paged_mqa_logits for the listed rows (all by
    default); CPU tensors, same argument forms as the product."""
    q_values, q_scale = q
    if q_values.dim() == 3:
        q_values = q_values.unsqueeze(1)
    B, next_n, H, last = q_values.shape
    nrows_total = B * next_n
    D = last * (2 if q_scale is not None else 1)
    qv = _cpu(q_values).view(torch.uint8).reshape(nrows_total, H, last)
    qs = _cpu(q_scale, torch.int32).reshape(nrows_total, H) if q_scale is not None else None
    kv = _cpu(kv_cache).view(torch.uint8)
    w = _cpu(weights, torch.float32)
    ctx = _cpu(context_lens).to(torch.int32)
    if ctx.dim() == 2:
        ctx, per_len = ctx.reshape(-1)[:nrows_total].contiguous(), 1
    else:
        ctx, per_len = ctx.contiguous(), next_n
    bt = _cpu(block_tables).to(torch.int32)
    if bt.dim() == 2 and bt.shape[0] == B:
        per_table = next_n
    else:
        bt, per_table = bt.reshape(nrows_total, -1), 1
    bt = bt.contiguous()
    r = _rows_arg(rows, nrows_total)
    out = torch.empty(r.numel(), max_model_len, dtype=torch.float64)
    bound = torch.empty_like(out)
    lib().oracle_paged_mqa_logits(
        qv.data_ptr(), qv.stride(0), qv.stride(1), qs.data_ptr() if qs is not None else None,
        qs.stride(0) if qs is not None else 0, qs.stride(1) if qs is not None else 0,
        kv.data_ptr(), kv.stride(0), kv.shape[0], kv.shape[1], w.data_ptr(), w.stride(0), w.stride(1),
        ctx.data_ptr(), per_len, bt.data_ptr(), bt.stride(0), bt.shape[1], per_table, H, D, int(max_model_len),
        float("-inf") if clean_logits else 0.0, r.data_ptr(), r.numel(), out.data_ptr(), bound.data_ptr())
    return out, bound


def compute_global_topk_indices_and_lens(topk_indices, token_to_req_indices, block_table, block_size,
                                         is_valid_token=None):
    """CPU restatement: (global_indices, lens) as int32 CPU tensors."""
    local = _cpu(topk_indices, torch.int32)
    req = _cpu(token_to_req_indices, torch.int32).contiguous()
    bt = _cpu(block_table, torch.int32)
    valid = _cpu(is_valid_token, torch.int32).contiguous() if is_valid_token is not None else None
    T, K = local.shape
    out = torch.empty((T, K), dtype=torch.int32)
    lens = torch.empty((T,), dtype=torch.int32)
    lib().oracle_compute_global_topk_indices(
        local.data_ptr(), local.stride(0), local.stride(1), T, K, req.data_ptr(), bt.data_ptr(), bt.stride(0),
        bt.shape[0], bt.shape[1], int(block_size), valid.data_ptr() if valid is not None else None,
        out.data_ptr(), out.stride(0), out.stride(1), lens.data_ptr())
    return out, lens


def combine_topk_swa_indices(topk_indices, query_start_loc, seq_lens, gather_lens, window_size, compress_ratio,
                             topk, M, N, fill=-7):
    """CPU restatement: (combined, lens); rows the op leaves unwritten keep
    ``fill`` (lens: ``fill`` too)."""
    t = _cpu(topk_indices, torch.int32)
    qsl = _cpu(query_start_loc, torch.int32).contiguous()
    seq = _cpu(seq_lens, torch.int32).contiguous()
    gat = _cpu(gather_lens, torch.int32).contiguous()
    width = (topk + window_size + 127) // 128 * 128
    out = torch.full((t.shape[0], width), fill, dtype=torch.int32)
    lens = torch.full((t.shape[0],), fill, dtype=torch.int32)
    lib().oracle_combine_topk_swa_indices(
        t.data_ptr(), t.stride(0), t.stride(1), t.shape[0], qsl.data_ptr(), seq.data_ptr(), gat.data_ptr(),
        seq.shape[0],
        int(window_size), int(compress_ratio), int(topk), int(M), int(N), out.data_ptr(), out.stride(0),
        out.stride(1), width, lens.data_ptr())
    return out, lens


def top_k_per_row(logits, k, row_starts=None, row_ends=None, seq_lens=None, next_n=1, rows=None):
    """CPU restatement: int32 [num_rows, k] (or [len(rows), k] for the given
    rows), each row's selected indices in ascending order (see
    oracle_top_k_per_row for the rows' ranges and the order of equal values)."""
    x = _cpu(logits, torch.float32)
    n = x.shape[0]
    st = _cpu(row_starts, torch.int32).contiguous() if row_starts is not None else None
    en = _cpu(row_ends, torch.int32).contiguous() if row_ends is not None else None
    sl = _cpu(seq_lens, torch.int32).contiguous() if seq_lens is not None else None
    if rows is not None:
        rows = torch.as_tensor(rows, dtype=torch.long)
        x = x[rows]
        if st is not None:
            st, en = st[rows].contiguous(), en[rows].contiguous()
        else:
            # each picked row keeps its decode range: give it its own seq_len entry
            r = rows
            sl = (sl[r // next_n] - next_n + r % next_n + 1).to(torch.int32).contiguous()
            next_n = 1
    out = torch.empty((x.shape[0], k), dtype=torch.int32)
    lib().oracle_top_k_per_row(x.data_ptr(), x.stride(0), x.stride(1), x.shape[0], x.shape[1],
                               st.data_ptr() if st is not None else None,
                               en.data_ptr() if en is not None else None,
                               sl.data_ptr() if sl is not None else None, int(next_n), int(k), out.data_ptr())
    return out


def fp8_einsum(x, xs, y, ys):
    """Binary64 'bhr,hdr->bhd' of flaggems_vllm.fp8_einsum and an error bound
    for a binary32 implementation before the output rounding ([B, H, D]
    float64 each); CPU or device tensors of any layout (e4m3fn or uint8
    codes, float32 scales)."""
    xb = _cpu(x).view(torch.uint8).contiguous()
    yb = _cpu(y).view(torch.uint8).contiguous()
    xsc = _cpu(xs, torch.float32).contiguous()
    ysc = _cpu(ys, torch.float32).contiguous()
    B, H, R = xb.shape
    D = yb.shape[1]
    out = torch.empty(B, H, D, dtype=torch.float64)
    bound = torch.empty_like(out)
    lib().oracle_fp8_einsum(xb.data_ptr(), xsc.data_ptr(), yb.data_ptr(), ysc.data_ptr(), B, H, R, D,
                            out.data_ptr(), bound.data_ptr())
    return out, bound
