"""The reference's PyTorch formulation of both ops, restated on CPU tensors.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  This follows the torch
oracle that the reference's own tests compare its Triton kernels against:

* main op: tests/test_fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py
  ``rmsnorm_no_weight_f32`` :143-148, ``apply_rope_gptj_last_k`` :93-140,
  ``_exact_pow2`` :154-163, ``torch_quantize_and_insert_k_cache`` :178-243,
  ``ref_impl`` :316-333 (q processed 2**19 rows at a time);
* sibling: tests/test_fused_inv_rope_fp8_quant.py
  ``native_fused_inv_rope_fp8_quant`` :150-198, ``_pack_ue8m0_scales`` :82-90;
* fused_q_kv_rmsnorm: tests/test_deepseek_v4_attention_fused_q_kv_rmsnorm.py
  ``_rmsnorm_ref`` :40-44;
* fused_indexer_q_rope_quant: tests/test_fused_indexer_q_rope_quant.py
  ``_rotate_tail_gptj`` :51-66, ``_reference_fp8`` :69-74, the E2M1 threshold
  table of ``_quantize_to_mxfp4`` :77-104;
* compute_slot_mapping_parallel: tests/test_slot_mapping.py ``_ref_slot_mapping``
  :53-66 (per-request loop), with the op's context-parallel arithmetic
  (runtime/backend/_ascend/ops/slot_mapping.py:88-105);
* dequantize_and_gather_k_cache: the reference kernel's per-row semantics
  (ops/deepseek_v4_attention_dequantize_and_gather_k_cache.py:61-120) in torch
  index arithmetic, with torch's float8 -> float cast and exp2 scale;
* sparse MLA decode over the MODEL1 cache: the portable kernel's chunked
  online softmax (ops/flash_mla_with_kvcache.py:489-688);
* sparse MLA prefill over bf16 rows: tests/test_flash_mla_sparse_fwd.py
  ``torch_flash_mla_sparse_fwd`` :93-150 (float32 gather, masked scores,
  logsumexp, the sink merged as a second logsumexp term);
* sparse-indexer logits: tests/test_fp8_fp4_mqa_logits.py
  ``reference_fp4_mqa_logits`` :40-66 (its per-row, per-head float32 loop,
  applied to FP8 q as well as MXFP4 q) and the paged test's per-row gather of
  the cache (tests/test_fp8_fp4_paged_mqa_logits.py:196-226);
* indexer key cache: tests/test_indexer_k_quant_and_cache.py ``torch_indexer``
  :99-142 and tests/test_cp_gather_indexer_k_quant_cache.py ``torch_gather``
  :83-114, with float8_e4m3fn codes.

Arithmetic is whatever torch's CPU kernels do in float32: the sum of squares
and rsqrt are torch's, which is why q is compared against this restatement
with a 1-bf16-ulp tolerance rather than bit for bit.  FP8 codes come from
torch's own float8_e4m3fn cast.

Unlike the reference oracle, ``kv`` is not modified (the op leaves it alone).
"""
import torch

HEAD_DIM, NOPE_DIM, ROPE_DIM, HALF_ROPE = 512, 448, 64, 32
KV_GROUP, KV_GROUPS = 64, 7
TOKEN_DATA_BYTES, SCALE_BYTES = 576, 8
FP8_MAX = 448.0
ROWS_PER_CHUNK = 1 << 19


def _pow2_exact(k: torch.Tensor) -> torch.Tensor:
    """2**k as float32 for integer-valued k, built from the exponent field."""
    field = (k.to(torch.int32) + 127).clamp(0, 255) << 23
    return field.view(torch.float32)


def _rotate_pairs(x_f32, cos, sin):
    """GPT-J rotation of interleaved (even, odd) pairs, separately rounded."""
    even, odd = x_f32[..., 0::2], x_f32[..., 1::2]
    new_even = even * cos - odd * sin
    new_odd = even * sin + odd * cos
    return torch.stack((new_even, new_odd), dim=-1).flatten(-2)


def qnorm_rope_kv_insert(q, kv, k_cache, slot_mapping, position_ids, cos_sin_cache,
                         eps, cache_block_size):
    """In place on q and k_cache (CPU tensors); kv is left untouched."""
    T, H, _ = q.shape
    tok_per_chunk = max(1, ROWS_PER_CHUNK // max(H, 1))
    for s in range(0, T, tok_per_chunk):
        qc = q[s:s + tok_per_chunk]
        cs = cos_sin_cache[position_ids[s:s + tok_per_chunk]].float()
        cos, sin = cs[:, None, :HALF_ROPE], cs[:, None, HALF_ROPE:]
        xf = qc.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
        qc[..., NOPE_DIM:] = _rotate_pairs(y[..., NOPE_DIM:], cos, sin).to(q.dtype)
        qc[..., :NOPE_DIM] = y[..., :NOPE_DIM].to(q.dtype)

    n_ins = slot_mapping.shape[0]
    tok = torch.arange(n_ins)
    slots = slot_mapping[:n_ins]
    keep = slots >= 0
    tok, slots = tok[keep], slots[keep]
    if tok.numel() == 0:
        return
    cs = cos_sin_cache[position_ids[tok]].float()
    rope = _rotate_pairs(kv[tok, NOPE_DIM:].float(), cs[:, :HALF_ROPE], cs[:, HALF_ROPE:])
    rope_bytes = rope.to(torch.bfloat16).contiguous().view(torch.uint8)  # [n, 128]

    groups = kv[tok, :NOPE_DIM].float().reshape(-1, KV_GROUPS, KV_GROUP)
    amax = groups.abs().amax(dim=-1).clamp(min=1e-4)
    expo = torch.ceil(torch.log2(amax / FP8_MAX))
    scaled = (groups / _pow2_exact(expo)[..., None]).clamp(-FP8_MAX, FP8_MAX)
    codes = scaled.to(torch.float8_e4m3fn).view(torch.uint8).reshape(-1, NOPE_DIM)
    scale_bytes = torch.zeros(tok.numel(), SCALE_BYTES, dtype=torch.uint8)
    scale_bytes[:, :KV_GROUPS] = (expo + 127.0).clamp(0.0, 255.0).to(torch.uint8)

    bs = cache_block_size
    blk, pib = slots // bs, slots % bs
    base = blk * k_cache.stride(0)
    flat = k_cache.as_strided((k_cache.shape[0] * k_cache.stride(0),), (1,))
    data_at = base + pib * TOKEN_DATA_BYTES
    scale_at = base + bs * TOKEN_DATA_BYTES + pib * SCALE_BYTES
    flat[data_at[:, None] + torch.arange(NOPE_DIM)] = codes
    flat[data_at[:, None] + NOPE_DIM + torch.arange(2 * ROPE_DIM)] = rope_bytes
    flat[scale_at[:, None] + torch.arange(SCALE_BYTES)] = scale_bytes


def inv_rope_fp8_quant(o, positions, cos_sin_cache, n_groups, heads_per_group,
                       eps=1e-10, tma_aligned_scales=False, nope_dim=NOPE_DIM, rope_dim=ROPE_DIM,
                       quant_group_size=128):
    """Returns (fp8 codes as uint8 [T, G, d], scales [T, G, K] float32 or
    packed int32 [T, G, hpg]) as plain contiguous tensors; any geometry the
    reference accepts (the test's oracle is written for nope_dim 448, rope_dim
    64, groups of 128: the same steps with those three as parameters)."""
    T, H, D = o.shape
    half = rope_dim // 2
    cs = cos_sin_cache[positions].float()
    cos, sin = cs[:, None, :half], cs[:, None, half:rope_dim]
    rf = o[..., nope_dim:].float()
    even, odd = rf[..., 0::2], rf[..., 1::2]
    inv = torch.stack((even * cos + odd * sin, odd * cos - even * sin), dim=-1).flatten(-2)
    x = torch.cat((o[..., :nope_dim], inv.to(o.dtype)), dim=-1).float()
    d = heads_per_group * D
    G = quant_group_size
    blocks = x.reshape(T, n_groups, d // G, G)
    scales = blocks.abs().amax(dim=-1).clamp(min=eps) * (1.0 / FP8_MAX)
    if tma_aligned_scales:
        scales = _pow2_exact(torch.ceil(torch.log2(scales.clamp(min=1e-10))))
    codes = (blocks / scales[..., None]).clamp(-FP8_MAX, FP8_MAX)
    codes = codes.to(torch.float8_e4m3fn).view(torch.uint8).reshape(T, n_groups, d)
    if not tma_aligned_scales:
        return codes, scales
    chunks = D // G
    byte = (scales.view(torch.int32) >> 23) & 0xFF
    byte = byte.reshape(T, n_groups, heads_per_group, chunks)
    packed = torch.zeros(T, n_groups, heads_per_group, dtype=torch.int32)
    for c in range(chunks):
        packed |= byte[..., c] << (8 * c)
    return codes, packed


def dequantize_and_gather_k_cache(out, k_cache, seq_lens, gather_lens, block_table, block_size,
                                  offset=0, rope_dim=64, nope_dim=None, scale_slots=None):
    """In place on ``out`` (CPU tensors)."""
    if nope_dim is None:
        nope_dim = out.shape[-1] - rope_dim
    if scale_slots is None:
        scale_slots = (nope_dim + 63) // 64 + (1 if nope_dim % 64 == 0 else 0)
    tb = nope_dim + 2 * rope_dim
    flat = k_cache.reshape(k_cache.shape[0], -1)
    for r in range(seq_lens.shape[0]):
        sl = int(seq_lens[r])
        gl = int(gather_lens[r]) if gather_lens is not None else sl
        n = max(0, min(gl, out.shape[1] - offset))
        if n == 0:
            continue
        pos = sl - gl + torch.arange(n)
        blk = block_table[r, pos // block_size].long()
        pib = pos % block_size
        rows = flat[blk]  # [n, block bytes]
        data_at = (pib * tb)[:, None] + torch.arange(tb)
        data = torch.gather(rows, 1, data_at)
        sc_at = (block_size * tb + pib * scale_slots)[:, None] + torch.arange(scale_slots)
        sbytes = torch.gather(rows, 1, sc_at)
        codes = data[:, :nope_dim].contiguous().view(torch.float8_e4m3fn).float()
        grp = torch.arange(nope_dim) // 64
        scale = torch.exp2(sbytes[:, grp].float() - 127.0)
        out[r, offset:offset + n, :nope_dim] = (codes * scale).to(torch.bfloat16)
        out[r, offset:offset + n, nope_dim:nope_dim + rope_dim] = (
            data[:, nope_dim:].contiguous().view(torch.bfloat16))


def rmsnorm(x, weight, eps):
    """Weighted RMSNorm in float32, result in x's dtype."""
    xf = x.float()
    y = xf * torch.rsqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + eps)
    return (y * weight.float()).to(x.dtype)


def fused_q_kv_rmsnorm(qr, kv, q_weight, kv_weight, eps):
    return rmsnorm(qr, q_weight, eps), rmsnorm(kv, kv_weight, eps)


def indexer_rotate(q, positions, cos_sin):
    """float32 copy of q with GPT-J RoPE on the last 64 dims, rounded to bf16."""
    nope = q.shape[-1] - ROPE_DIM
    cs = cos_sin[positions].float()
    cos, sin = cs[:, None, :HALF_ROPE], cs[:, None, HALF_ROPE:]
    x = q.float()
    even, odd = x[..., nope::2].clone(), x[..., nope + 1::2].clone()
    x[..., nope::2] = (even * cos - odd * sin).to(torch.bfloat16).float()
    x[..., nope + 1::2] = (odd * cos + even * sin).to(torch.bfloat16).float()
    return x


def e2m1_threshold_codes(xs):
    """E2M1 nibbles by the reference test's threshold table (ties to even)."""
    a = xs.abs()
    code = torch.zeros_like(a, dtype=torch.int32)
    for thr, c, inclusive in ((0.25, 1, False), (0.75, 2, True), (1.25, 3, False),
                              (1.75, 4, True), (2.5, 5, False), (3.5, 6, True), (5.0, 7, False)):
        code = torch.where(a >= thr if inclusive else a > thr, c, code)
    sign = ((xs.contiguous().view(torch.int32) >> 31) & 1).to(torch.uint8)
    return code.to(torch.uint8) | (sign << 3)


def fused_indexer_q_rope_quant(positions, index_q, cos_sin, weights, softmax_scale, head_scale,
                               use_fp4=False):
    x = indexer_rotate(index_q[:positions.shape[0]], positions, cos_sin)
    T, H, D = x.shape
    if not use_fp4:
        amax = x.abs().amax(dim=-1)
        q_scale = torch.exp2(torch.ceil(torch.log2(amax.clamp(min=1e-4) / FP8_MAX)))
        codes = (x / q_scale[..., None]).to(torch.float8_e4m3fn).view(torch.uint8)
        return codes, weights.float() * q_scale * softmax_scale * head_scale
    blocks = x.reshape(T, H, D // 32, 32)
    amax = blocks.abs().amax(dim=-1, keepdim=True).clamp(min=6 * (2 ** -126))
    k = (amax / 6.0).log2().ceil().clamp(-127.0, 127.0)
    xs = (blocks / k.exp2()).clamp(-6.0, 6.0)
    nib = e2m1_threshold_codes(xs).reshape(T, H, D)
    packed = (nib[..., 0::2] | (nib[..., 1::2] << 4)).contiguous()
    scales = (k + 127.0).to(torch.uint8).reshape(T, H, D // 32)
    return (packed, scales), weights.float() * softmax_scale * head_scale


def slot_mapping(num_tokens, qsl, positions, block_table, block_size, max_num_tokens=None,
                 cp_world_size=1, cp_rank=0, interleave=1, pad_id=-1):
    """int64 slot of every token, pad_id past num_tokens (Python loop)."""
    n = max_num_tokens if max_num_tokens is not None else len(positions)
    out = torch.full((n,), pad_id, dtype=torch.int64)
    vbs = block_size * cp_world_size
    for r in range(len(qsl) - 1):
        for t in range(int(qsl[r]), min(int(qsl[r + 1]), num_tokens, n)):
            pos = int(positions[t])
            voff = pos % vbs
            if (voff // interleave) % cp_world_size != cp_rank:
                continue
            blk = int(block_table[r][pos // vbs])
            out[t] = blk * block_size + voff // (cp_world_size * interleave) * interleave + voff % interleave
    return out


def model1_rows(k_cache):
    """Dequantise a whole [num_blocks, page, 1, 584] MODEL1 cache into
    [num_blocks * page, 512] bf16 rows (reference kernel
    ops/flash_mla_with_kvcache.py:508-559: f32 e4m3 value times the E8M0 scale
    bitcast from ``byte << 23``, rounded to bf16; RoPE copied)."""
    nb, page = k_cache.shape[0], k_cache.shape[1]
    flat = k_cache.reshape(nb, -1)
    data = flat[:, :page * 576].reshape(nb * page, 576)
    scl = flat[:, page * 576:page * 584].reshape(nb * page, 8)
    scale = (scl[:, :7].to(torch.int32) << 23).view(torch.float32)
    nope = data[:, :448].contiguous().view(torch.float8_e4m3fn).to(torch.float32)
    nope = (nope.view(-1, 7, 64) * scale[:, :, None]).reshape(-1, 448).to(torch.bfloat16)
    rope = data[:, 448:].contiguous().view(torch.bfloat16)
    return torch.cat([nope, rope], dim=1)


def sparse_mla_decode_model1(q, k_cache, indices, topk_length=None, attn_sink=None,
                             extra_k_cache=None, extra_indices=None, extra_topk_length=None,
                             softmax_scale=None, chunk=32):
    """The reference portable MODEL1 kernel's algorithm on CPU tensors
    (ops/flash_mla_with_kvcache.py:489-688): 32-token chunks, fp32 scores,
    online softmax with natural exp, probabilities rounded to bf16 before the
    PV product, fp32 accumulation, bf16 output.  A chunk whose tokens are all
    invalid before any valid one contributes nothing (the running max starts
    at -inf and is treated as 0 for the exponent, as the sm90 kernel's -1e30
    start does).  Returns (out bf16 [B,SQ,HQ,512], lse f32 [B,HQ,SQ])."""
    B, SQ, HQ, D = q.shape
    scale = D ** -0.5 if softmax_scale is None else softmax_scale
    lists = [(model1_rows(k_cache), k_cache.shape[0], k_cache.shape[1], indices, topk_length)]
    if extra_k_cache is not None:
        lists.append((model1_rows(extra_k_cache), extra_k_cache.shape[0], extra_k_cache.shape[1],
                      extra_indices, extra_topk_length))
    out = torch.zeros(B, SQ, HQ, D, dtype=torch.bfloat16)
    lse = torch.empty(B, HQ, SQ, dtype=torch.float32)
    for b in range(B):
        for s in range(SQ):
            qf = q[b, s].float()
            m = torch.full((HQ,), float("-inf"))
            lsum = torch.zeros(HQ)
            acc = torch.zeros(HQ, D)
            for rows, nb, page, idx, length in lists:
                topk = idx.shape[-1]
                n = topk if length is None else max(0, min(int(length[b]), topk))
                for c0 in range(0, n, chunk):
                    ids = idx[b, s, c0:min(c0 + chunk, n)].long()
                    valid = (ids >= 0) & (ids // page < nb)
                    kv = rows[torch.where(valid, ids, 0)].float() * valid[:, None]
                    qk = (qf @ kv.T) * scale
                    qk = torch.where(valid[None, :], qk, float("-inf"))
                    m_new = torch.maximum(m, qk.max(dim=1).values)
                    m_use = torch.where(torch.isinf(m_new) & (m_new < 0), 0.0, m_new)
                    p = torch.exp(qk - m_use[:, None])
                    alpha = torch.exp(m - m_use)
                    lsum = lsum * alpha + p.sum(dim=1)
                    acc = acc * alpha[:, None] + p.to(torch.bfloat16).float() @ kv
                    m = m_new
            empty = torch.isinf(m) & (m < 0)
            lse[b, :, s] = torch.where(empty, float("inf"), m + torch.log(lsum))
            if attn_sink is not None:
                denom = lsum + torch.exp(attn_sink.float() - m)
            else:
                denom = lsum
            o = acc / torch.where(empty, 1.0, denom)[:, None]
            out[b, s] = torch.where(empty[:, None], 0.0, o).to(torch.bfloat16)
    return out, lse


def flash_mla_sparse_fwd(q, kv, indices, sm_scale, attn_sink=None, topk_length=None):
    """(out bf16, max_logits, lse) as the reference test defines them, in
    float32 on CPU tensors (q [s_q, h_q, d_qk], kv [s_kv, 1, d_qk], indices
    [s_q, 1, topk])."""
    s_q, h_q, d_qk = q.shape
    s_kv, topk = kv.shape[0], indices.shape[-1]
    idx = indices.reshape(s_q, topk).clone()
    if topk_length is not None:
        idx[torch.arange(topk)[None, :] >= topk_length[:, None]] = -1
    invalid = (idx < 0) | (idx >= s_kv)
    idx[invalid] = 0
    rows = kv.reshape(s_kv, d_qk).index_select(0, idx.reshape(-1).long()).reshape(s_q, topk, d_qk).float()
    p = torch.bmm(q.float(), rows.transpose(1, 2).contiguous()) * sm_scale
    p[invalid[:, None, :].expand(p.shape)] = float("-inf")
    lse = torch.logsumexp(p, -1)
    max_logits = p.amax(-1)
    lse_o = lse if attn_sink is None else torch.logsumexp(torch.stack([lse, attn_sink.expand_as(lse)]), 0)
    lse_o = torch.where(lse_o == float("-inf"), float("inf"), lse_o)
    out = torch.bmm(torch.exp(p - lse_o[..., None]), rows[..., :512].contiguous())
    lse = torch.where(lse == float("-inf"), float("inf"), lse)
    return out.to(torch.bfloat16), max_logits, lse


def indexer_k_quant_and_cache(k, kv_cache, slot_mapping, quant_block_size, scale_fmt):
    """Per token and quant block, in place on the uint8 cache: scale =
    max(amax, 1e-4) / 448 (ue8m0: exp2(ceil(log2(scale)))), codes =
    float8_e4m3fn(k / scale), float32 scales after the block's codes.  The
    reference's per-token loop, batched over tokens (the same elementwise
    float32 operations); slots are assumed distinct, as vLLM assigns them."""
    num_blocks, block_size = kv_cache.shape[0], kv_cache.shape[1]
    head_dim = k.shape[-1]
    nqb = head_dim // quant_block_size
    flat = kv_cache.view(num_blocks, -1)
    values = flat[:, :block_size * head_dim]
    scales = flat[:, block_size * head_dim:].view(torch.float32)
    slots = slot_mapping.to(torch.int64)
    keep = torch.nonzero(slots >= 0).flatten()
    if keep.numel() == 0:
        return
    s = slots[keep]
    b, r = s // block_size, s % block_size
    v = k[keep].reshape(-1, nqb, quant_block_size)
    amax = v.abs().to(torch.float32).amax(dim=-1)
    scale = torch.maximum(amax, torch.tensor(1e-4, dtype=torch.float32)) / 448.0
    if scale_fmt == "ue8m0":
        scale = torch.exp2(torch.ceil(torch.log2(scale)))
    codes = (v.to(torch.float32) / scale[..., None]).to(torch.float8_e4m3fn).view(torch.uint8)
    codes = codes.reshape(-1, head_dim)
    cols = r[:, None] * head_dim + torch.arange(head_dim)
    values[b[:, None], cols] = codes
    scales[b[:, None], r[:, None] * nqb + torch.arange(nqb)] = scale


def cp_gather_indexer_k_quant_cache(k_cache, k_fp8, k_fp8_scale, block_table, cu_seqlen):
    """Token t of request b copies the codes and scales of position
    t - cu_seqlen[b] into row t of k_fp8 / k_fp8_scale (byte views)."""
    block_size = k_cache.shape[1]
    head_dim = k_fp8.shape[1]
    nqb = head_dim // (head_dim * 4 // k_fp8_scale.shape[1])
    flat = k_cache.view(k_cache.shape[0], -1)
    values = flat[:, :block_size * head_dim]
    scales = flat[:, block_size * head_dim:].view(torch.float32)
    kb, sf = k_fp8.view(torch.uint8), k_fp8_scale.view(torch.float32)
    for b in range(block_table.shape[0]):
        for t in range(int(cu_seqlen[b]), int(cu_seqlen[b + 1])):
            pos = t - int(cu_seqlen[b])
            blk, r = int(block_table[b, pos // block_size]), pos % block_size
            kb[t] = values[blk, r * head_dim:(r + 1) * head_dim]
            sf[t] = scales[blk, r * nqb:(r + 1) * nqb]


_E2M1_VALUES = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def mxfp4_values(packed, q_scale, head_dim):
    """float32 [..., head_dim] of packed E2M1 (even element in the low nibble)
    times 2^(byte - 127), byte b of the int32 scale covering 32 b..32 b + 31."""
    p = packed.view(torch.uint8).long()
    nib = torch.stack([p & 0xF, p >> 4], dim=-1).reshape(*packed.shape[:-1], head_dim)
    vals = _E2M1_VALUES[nib]
    sb = q_scale.reshape(*packed.shape[:-1]).long()
    blk = torch.arange(head_dim) // 32
    byte = ((sb[..., None] >> (8 * blk)) & 0xFF).float()
    return vals * torch.exp2(byte - 127.0)


def mqa_logits(q, kv, weights, cu_seqlen_ks, cu_seqlen_ke, clean_logits=True):
    """The reference test's float32 formulation: per row m and head h,
    ReLU(sum_d q k * k_scale) * w accumulated over heads."""
    q_values, q_scale = q
    k_values, k_scales = kv
    M, H = q_values.shape[:2]
    if q_scale is not None:
        qf = mxfp4_values(q_values, q_scale, q_values.shape[-1] * 2)
    else:
        qf = q_values.view(torch.float8_e4m3fn).float()
    kf = k_values.view(torch.float8_e4m3fn).float()
    ksc = k_scales.reshape(-1).float()
    logits = torch.zeros(M, kf.shape[0], dtype=torch.float32)
    for m in range(M):
        for h in range(H):
            dot = torch.sum(qf[m, h].unsqueeze(0) * kf, dim=1) * ksc
            logits[m] += dot.clamp_min(0.0) * weights[m, h]
    if clean_logits:
        for m in range(M):
            logits[m, :int(cu_seqlen_ks[m])] = float("-inf")
            logits[m, int(cu_seqlen_ke[m]):] = float("-inf")
    return logits


def paged_mqa_logits(q, kv_cache, weights, context_lens, block_tables, max_model_len, clean_logits=False):
    """Per row: gather the context's keys and scales from the paged cache as
    the reference test does, then the dense formulation above."""
    q_values, q_scale = q
    if q_values.dim() == 3:
        q_values = q_values.unsqueeze(1)
    B, next_n, H, last = q_values.shape
    rows = B * next_n
    nblk, bs = kv_cache.shape[0], kv_cache.shape[1]
    D = kv_cache.shape[3] - 4
    flat = kv_cache.reshape(nblk, -1)
    kdata = flat[:, :bs * D].reshape(nblk * bs, D)
    kscale = flat[:, bs * D:].contiguous().view(torch.float32).reshape(-1)
    ctx = context_lens.reshape(-1)[:rows] if context_lens.dim() == 2 else context_lens.repeat_interleave(next_n)
    out = torch.full((rows, max_model_len), float("-inf") if clean_logits else 0.0)
    qr = q_values.reshape(rows, H, last)
    qsr = q_scale.reshape(rows, H) if q_scale is not None else None
    for r in range(rows):
        c = int(ctx[r])
        if c == 0:
            continue
        pos = torch.arange(c)
        phys = block_tables[r // next_n, pos // bs].long()
        idx = phys * bs + pos % bs
        qq = (qr[r:r + 1], qsr[r:r + 1] if qsr is not None else None)
        out[r, :c] = mqa_logits(qq, (kdata[idx], kscale[idx]), weights[r:r + 1], None, None, False)[0]
    return out
