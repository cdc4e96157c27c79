"""Seeded workloads and byte accounting for the two ops.

The five main-op configurations are the ones the benchmark contract names
(c0 CPU plumbing, c1 decode, c2 prefill headline, c3 large prefill, c4 ragged
strided).  Everything is drawn on the CPU from a ``torch.Generator`` seeded
with the config index, so the same inputs reach the GPU kernel, the CPU oracle
and the CPU baseline; ``Workload.to(device)`` copies them over (keeping the
strided-view structure of c4).

Slot mappings follow vLLM's paged layout (reference
tests/test_slot_mapping.py:53-66): slot = block_table[seq][pos // bs] * bs
+ pos % bs, with block tables drawn from a random permutation of the cache's
blocks.
"""
import math
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field
from typing import Dict, Optional

import torch

HEAD_DIM = 512
NOPE_DIM = 448
ROPE_DIM = 64
TOKEN_DATA_BYTES = 576
SCALE_BYTES_PER_TOKEN = 8
HEAD_BYTES = TOKEN_DATA_BYTES + SCALE_BYTES_PER_TOKEN  # 584
BLOCK_SIZE = 64
EPS = 1e-6


def make_cos_sin_cache(max_pos: int, rope_dim: int = ROPE_DIM, base: float = 10000.0):
    """[max_pos, rope_dim] float32: cos(p * theta_j) | sin(p * theta_j),
    theta_j = base ** (-2j / rope_dim), computed in float32."""
    exps = torch.arange(0, rope_dim, 2, dtype=torch.float32) / rope_dim
    theta = 1.0 / (base ** exps)
    ang = torch.outer(torch.arange(max_pos, dtype=torch.float32), theta)
    return torch.cat((ang.cos(), ang.sin()), dim=-1).contiguous()


def yarn_correction_range(beta_fast: float, beta_slow: float, rope_dim: int, base: float,
                          max_pos: int):
    """YaRN's blend band (Peng et al. 2023, "YaRN: Efficient Context Window
    Extension of Large Language Models", eq. 17-18): the rotary dimension at
    which a frequency completes r turns over max_pos positions is
    d(r) = rope_dim * ln(max_pos / (2 pi r)) / (2 ln base); the band runs from
    floor(d(beta_fast)) to ceil(d(beta_slow)), clipped to [0, rope_dim - 1]."""
    def dim_of(turns):
        return rope_dim * math.log(max_pos / (turns * 2 * math.pi)) / (2 * math.log(base))

    return max(math.floor(dim_of(beta_fast)), 0), min(math.ceil(dim_of(beta_slow)), rope_dim - 1)


def make_yarn_cos_sin_cache(max_pos: int = 65536, rope_dim: int = ROPE_DIM, scaling_factor: float = 16,
                            base: float = 10000.0, beta_fast: float = 32, beta_slow: float = 1,
                            rows: int = None):
    """DeepSeek-V4's YaRN-scaled rotary table as the reference test builds it
    (tests/test_fused_inv_rope_fp8_quant.py:246-264): frequency j is
    theta_j = base^(-2j/rope_dim) below the blend band, theta_j / scaling_factor
    above it, and a linear blend inside it; row p holds cos(p theta) | sin(p
    theta) in float32.  The full table has max_pos * scaling_factor rows; `rows`
    keeps only its first rows (each row depends on p alone)."""
    half = rope_dim // 2
    extra = 1.0 / (base ** (torch.arange(0, rope_dim, 2, dtype=torch.float32) / rope_dim))
    interp = extra / scaling_factor
    lo, hi = yarn_correction_range(beta_fast, beta_slow, rope_dim, base, max_pos)
    if lo == hi:
        hi += 0.001
    ramp = ((torch.arange(half, dtype=torch.float32) - lo) / (hi - lo)).clamp(0, 1)
    keep = 1.0 - ramp  # 1: extrapolated frequency, 0: interpolated
    theta = interp * (1 - keep) + extra * keep
    n = int(max_pos * scaling_factor) if rows is None else rows
    ang = torch.outer(torch.arange(n, dtype=torch.float32), theta)
    return torch.cat((ang.cos(), ang.sin()), dim=-1).contiguous()


def randn_bf16(shape, gen: torch.Generator, chunk: int = 1 << 22) -> torch.Tensor:
    """N(0, 1) bf16 tensor.  One 62-bit seed is drawn from ``gen``; chunk i is
    then drawn from its own generator seeded with seed + i, on a thread pool,
    so large tensors are generated in parallel with bounded temporaries and
    the result does not depend on the number of threads."""
    out = torch.empty(shape, dtype=torch.bfloat16)
    flat = out.view(-1)
    base = int(torch.randint(0, 1 << 62, (1,), generator=gen))
    starts = range(0, flat.numel(), chunk)

    def fill(i_s):
        i, s = i_s
        n = min(chunk, flat.numel() - s)
        g = torch.Generator().manual_seed(base + i)
        flat[s:s + n] = torch.empty(n, dtype=torch.float32).normal_(generator=g)

    if len(starts) <= 1:
        for item in enumerate(starts):
            fill(item)
    else:
        workers = min(16, len(os.sched_getaffinity(0)), len(starts))
        with ThreadPoolExecutor(workers) as pool:
            list(pool.map(fill, enumerate(starts)))
    return out


def main_op_bytes(num_tokens: int, num_heads: int, num_inserted: int) -> int:
    """Algorithmic HBM bytes of one main-op call: q read + write, kv row read and
    584-byte cache write per inserted token, position + slot and the 256-byte
    cos/sin row per token."""
    return (4 * num_tokens * num_heads * HEAD_DIM + (1024 + HEAD_BYTES) * num_inserted
            + 16 * num_tokens + 256 * num_tokens)


def inv_rope_bytes(num_tokens: int, num_heads: int, tma_aligned_scales: bool) -> int:
    """Algorithmic HBM bytes of one sibling call: o read, fp8 write, scales,
    position and cos/sin row per token."""
    scale_bytes = 4 if tma_aligned_scales else 16
    return num_tokens * num_heads * (1024 + 512 + scale_bytes) + (8 + 256) * num_tokens


def gather_bytes(rows: int) -> int:
    """Algorithmic HBM bytes of gathering `rows` cached tokens: 584 cache bytes
    read, 1024 bf16 bytes written and a 4-byte block-table entry per row."""
    return rows * (HEAD_BYTES + 2 * HEAD_DIM + 4)


def rmsnorm_bytes(rows: int, q_size: int, kv_size: int) -> int:
    """Algorithmic HBM bytes of fused_q_kv_rmsnorm: each bf16 row read and
    written once, plus the two bf16 weight vectors."""
    return 4 * rows * (q_size + kv_size) + 2 * (q_size + kv_size)


def indexer_bytes(rows: int, heads: int, head_dim: int, fp4: bool) -> int:
    """Algorithmic HBM bytes of fused_indexer_q_rope_quant: bf16 q read, FP8
    codes (or E2M1 nibbles + one scale byte per 32) written, bf16 weight read
    and float32 weight written, position and cos/sin row per token."""
    per_head = 2 * head_dim + (head_dim // 2 + head_dim // 32 if fp4 else head_dim) + 2 + 4
    return rows * heads * per_head + rows * (8 + 256)


@dataclass
class Workload:
    name: str
    q: torch.Tensor
    kv: torch.Tensor
    k_cache: torch.Tensor
    slot_mapping: torch.Tensor
    position_ids: torch.Tensor
    cos_sin_cache: torch.Tensor
    eps: float = EPS
    block_size: int = BLOCK_SIZE
    rms_weight: Optional[torch.Tensor] = None  # drawn, not consumed by the op
    buffer: Optional[torch.Tensor] = None  # c4: the fused [T, H*D + D] buffer
    meta: Dict[str, object] = field(default_factory=dict)

    @property
    def num_tokens(self) -> int:
        return self.q.shape[0]

    @property
    def num_heads(self) -> int:
        return self.q.shape[1]

    @property
    def num_inserted(self) -> int:
        return int((self.slot_mapping >= 0).sum())

    def bytes_per_call(self) -> int:
        return main_op_bytes(self.num_tokens, self.num_heads, self.num_inserted)

    def args(self):
        return (self.q, self.kv, self.k_cache, self.slot_mapping, self.position_ids,
                self.cos_sin_cache, self.eps, self.block_size)

    def to(self, device) -> "Workload":
        """Copy every tensor to ``device``; c4's q/kv stay views of one buffer."""
        if self.buffer is not None:
            buf = self.buffer.to(device)
            hd = self.q.shape[1] * HEAD_DIM
            q = buf[:, :hd].view(self.q.shape)
            kv = buf[:, hd:]
        else:
            buf, q, kv = None, self.q.to(device), self.kv.to(device)
        return Workload(self.name, q, kv, self.k_cache.to(device), self.slot_mapping.to(device),
                        self.position_ids.to(device), self.cos_sin_cache.to(device), self.eps,
                        self.block_size, self.rms_weight, buf, dict(self.meta))

    def clone(self) -> "Workload":
        if self.buffer is not None:
            buf = self.buffer.clone()
            hd = self.q.shape[1] * HEAD_DIM
            q, kv = buf[:, :hd].view(self.q.shape), buf[:, hd:]
        else:
            buf, q, kv = None, self.q.clone(), self.kv.clone()
        return Workload(self.name, q, kv, self.k_cache.clone(), self.slot_mapping.clone(),
                        self.position_ids.clone(), self.cos_sin_cache.clone(), self.eps,
                        self.block_size, self.rms_weight, buf, dict(self.meta))


def _paged_slots(positions: torch.Tensor, seq_ids: torch.Tensor, tables, bs: int):
    blk_idx = positions // bs
    out = torch.empty_like(positions)
    for s, (table, first) in enumerate(tables):
        m = seq_ids == s
        out[m] = table[blk_idx[m] - first] * bs + positions[m] % bs
    return out


def _pad_some(slots: torch.Tensor, count: int, gen: torch.Generator) -> torch.Tensor:
    if count > 0:
        idx = torch.randperm(slots.numel(), generator=gen)[:count]
        slots[idx] = -1
    return slots


def _cache(num_blocks: int, bs: int = BLOCK_SIZE) -> torch.Tensor:
    return torch.zeros(num_blocks, bs * HEAD_BYTES, dtype=torch.uint8)


def make_workload(config: int, seed: Optional[int] = None, num_heads: Optional[int] = None,
                  num_tokens: Optional[int] = None) -> Workload:
    """Seeded CPU inputs of benchmark configuration ``config`` (0..4).

    ``num_tokens`` (c2, c3) and ``num_heads`` override the size for smaller
    parity runs with the same construction.  Draw order: q (or c4's fused
    buffer), kv, RMSNorm weight, positions, slots.
    """
    g = torch.Generator().manual_seed(config if seed is None else seed)
    bs = BLOCK_SIZE
    if config == 0:
        T, H, max_pos, nblk = 16, 8, 4096, 4
    elif config == 1:
        T, H, max_pos, nblk = 256, 64, 32768, 4096
    elif config == 2:
        T, H, max_pos, nblk = 8192, 64, 65536 + 2048, 16384
    elif config == 3:
        T, H, max_pos, nblk = 32768, 128, 32768, 65536
    elif config == 4:
        T, H, max_pos, nblk = None, 64, 131072, None
    else:
        raise ValueError(f"unknown config {config}")
    if num_heads is not None:
        H = num_heads
    if num_tokens is not None and config in (2, 3):
        T = num_tokens

    if config == 4:
        lens = torch.empty(64).log_normal_(mean=6.0, std=1.2, generator=g)
        lens = lens.round().clamp(1, 8192).to(torch.int64)
        T = int(lens.sum())
        buf = randn_bf16((T, H * HEAD_DIM + HEAD_DIM), g)
        q = buf[:, :H * HEAD_DIM].view(T, H, HEAD_DIM)
        kv = buf[:, H * HEAD_DIM:]
    else:
        buf = None
        q = randn_bf16((T, H, HEAD_DIM), g)
        kv = randn_bf16((T, HEAD_DIM), g)
    weight = 1.0 + 0.1 * torch.randn(HEAD_DIM, generator=g)

    if config in (0, 1):
        positions = torch.randint(0, max_pos, (T,), generator=g, dtype=torch.int64)
        slots = torch.randperm(nblk * bs, generator=g)[:T].to(torch.int64)
        slots = _pad_some(slots, 2 if config == 0 else round(0.05 * T), g)
    elif config == 2:
        nseq, per = 4, T // 4
        starts = torch.randint(0, 65536, (nseq,), generator=g, dtype=torch.int64)
        positions = torch.cat([s + torch.arange(per) for s in starts.tolist()])
        seq_ids = torch.arange(nseq).repeat_interleave(per)
        perm = torch.randperm(nblk, generator=g)
        need = (65536 + per) // bs + 1
        tables = [(perm[s * need:(s + 1) * need], 0) for s in range(nseq)]
        slots = _paged_slots(positions, seq_ids, tables, bs)
        seq_lens, new_lens = starts + per, torch.full((nseq,), per)
    elif config == 3:
        positions = torch.arange(T, dtype=torch.int64)
        perm = torch.randperm(nblk, generator=g)
        tables = [(perm[:(T + bs - 1) // bs], 0)]
        slots = _paged_slots(positions, torch.zeros(T, dtype=torch.int64), tables, bs)
        seq_lens, new_lens = torch.tensor([T]), torch.tensor([T])
    else:  # config 4
        starts = (torch.rand(64, generator=g, dtype=torch.float64) *
                  (max_pos - lens).to(torch.float64)).to(torch.int64)
        positions = torch.cat([s + torch.arange(n) for s, n in zip(starts.tolist(), lens.tolist())])
        seq_ids = torch.arange(64).repeat_interleave(lens)
        firsts = starts // bs
        counts = (starts + lens - 1) // bs - firsts + 1
        nblk = int(counts.sum()) + 64
        perm = torch.randperm(nblk, generator=g)
        tables, at = [], 0
        for f, c in zip(firsts.tolist(), counts.tolist()):
            tables.append((perm[at:at + c], f))
            at += c
        slots = _paged_slots(positions, seq_ids, tables, bs)
        slots = _pad_some(slots, round(0.10 * T), g)
        seq_lens, new_lens = starts + lens, lens

    meta = {"config": config, "max_pos": max_pos, "num_blocks": nblk}
    if config >= 2:
        # per-sequence block tables (int32, [num_seqs, max_blocks]; entries before a
        # sequence's first touched block are 0 and never read), the sequence
        # lengths after this chunk and the number of tokens it added
        width = max(f + len(t) for t, f in tables)
        bt = torch.zeros(len(tables), width, dtype=torch.int32)
        for i, (t, f) in enumerate(tables):
            bt[i, f:f + len(t)] = t.to(torch.int32)
        meta.update(block_table=bt, seq_lens=seq_lens.to(torch.int32),
                    new_lens=new_lens.to(torch.int32))
    cos_sin = make_cos_sin_cache(max_pos)
    return Workload(f"c{config}", q, kv, _cache(nblk, bs), slots.contiguous(),
                    positions.contiguous(), cos_sin, EPS, bs, weight, buf, meta)


@dataclass
class InvRopeWorkload:
    o: torch.Tensor
    positions: torch.Tensor
    cos_sin_cache: torch.Tensor
    n_groups: int
    heads_per_group: int

    def to(self, device):
        return InvRopeWorkload(self.o.to(device), self.positions.to(device),
                               self.cos_sin_cache.to(device), self.n_groups, self.heads_per_group)


def make_inv_rope_workload(num_tokens: int = 8192, num_heads: int = 64, n_groups: int = 8,
                           seed: int = 0, scale: float = 1.0, max_pos: int = 65536, head_dim: int = HEAD_DIM,
                           rope_dim: int = ROPE_DIM) -> InvRopeWorkload:
    """Seeded CPU inputs for the sibling op (default: T=8192, H=64, G=8,
    DeepSeek-V4's head_dim 512 with 64 rope dims)."""
    g = torch.Generator().manual_seed(seed)
    o = randn_bf16((num_tokens, num_heads, head_dim), g)
    if scale != 1.0:
        o = (o.float() * scale).to(torch.bfloat16)
    positions = torch.randint(0, max_pos, (num_tokens,), generator=g, dtype=torch.int64)
    return InvRopeWorkload(o, positions, make_cos_sin_cache(max_pos, rope_dim=rope_dim), n_groups,
                           num_heads // n_groups)


# ------------------------------------------------------------ sparse MLA ----

def make_model1_cache(num_pages: int, page: int, gen: torch.Generator, std: float = 0.1) -> torch.Tensor:
    """A [num_pages, page, 1, 584] uint8 MODEL1 cache filled like the
    reference's test generator (tests/test_flash_mla_with_kvcache.py:94-140):
    NoPE = std * randn quantised per 64-group with a power-of-two scale
    2^ceil(log2(max(amax, 1e-4) / 448)) (E8M0 byte = exponent + 127), RoPE =
    std * randn in bf16; token data first in each page, then 8 scale bytes per
    token (the 8th zero)."""
    n = num_pages * page
    nope = (torch.randn(n, NOPE_DIM, generator=gen) * std).to(torch.bfloat16).float()
    groups = nope.view(n, 7, 64)
    amax = groups.abs().amax(dim=-1).clamp_min(1e-4)
    expo = torch.ceil(torch.log2(amax / 448.0))
    codes = (groups / torch.exp2(expo)[:, :, None]).clamp(-448.0, 448.0).reshape(n, NOPE_DIM)
    codes = codes.to(torch.float8_e4m3fn).view(torch.uint8)
    rope = (torch.randn(n, ROPE_DIM, generator=gen) * std).to(torch.bfloat16)
    data = torch.cat([codes, rope.view(torch.uint8).view(n, 2 * ROPE_DIM)], dim=1)
    scales = torch.zeros(n, SCALE_BYTES_PER_TOKEN, dtype=torch.uint8)
    scales[:, :7] = (expo + 127).clamp(0, 255).to(torch.uint8)
    cache = torch.empty(num_pages, page * HEAD_BYTES, dtype=torch.uint8)
    cache[:, :page * TOKEN_DATA_BYTES] = data.view(num_pages, page * TOKEN_DATA_BYTES)
    cache[:, page * TOKEN_DATA_BYTES:] = scales.view(num_pages, page * SCALE_BYTES_PER_TOKEN)
    return cache.view(num_pages, page, 1, HEAD_BYTES)


@dataclass
class MlaWorkload:
    """Inputs of one flash_mla_with_kvcache sparse MODEL1 call (CPU tensors
    until ``to``)."""
    name: str
    q: torch.Tensor
    k_cache: torch.Tensor
    indices: torch.Tensor
    topk_length: Optional[torch.Tensor] = None
    attn_sink: Optional[torch.Tensor] = None
    extra_k_cache: Optional[torch.Tensor] = None
    extra_indices: Optional[torch.Tensor] = None
    extra_topk_length: Optional[torch.Tensor] = None

    def kwargs(self):
        return dict(topk_length=self.topk_length, attn_sink=self.attn_sink,
                    extra_k_cache=self.extra_k_cache,
                    extra_indices_in_kvcache=self.extra_indices,
                    extra_topk_length=self.extra_topk_length)

    def oracle_kwargs(self):
        return dict(topk_length=self.topk_length, attn_sink=self.attn_sink,
                    extra_k_cache=self.extra_k_cache, extra_indices=self.extra_indices,
                    extra_topk_length=self.extra_topk_length)

    def to(self, device):
        mv = lambda t: None if t is None else t.to(device)
        return MlaWorkload(self.name, mv(self.q), mv(self.k_cache), mv(self.indices),
                           mv(self.topk_length), mv(self.attn_sink), mv(self.extra_k_cache),
                           mv(self.extra_indices), mv(self.extra_topk_length))

    def used_tokens(self) -> int:
        """Selected entries the kernel attends (within the top-k lengths and
        pointing inside their cache), summed over batch rows and query
        positions."""
        total = 0
        for cache, idx, length in ((self.k_cache, self.indices, self.topk_length),
                                   (self.extra_k_cache, self.extra_indices, self.extra_topk_length)):
            if cache is None:
                continue
            limit = cache.shape[0] * cache.shape[1]
            topk = idx.shape[-1]
            n = torch.full((idx.shape[0],), topk) if length is None else length.cpu().long().clamp(0, topk)
            pos = torch.arange(topk)
            inside = (pos[None, None, :] < n[:, None, None]) & (idx.cpu() >= 0) & (idx.cpu() < limit)
            total += int(inside.sum())
        return total


# The reference benchmark's MODEL1 cases (benchmark/test_flash_mla_with_kvcache.py:230-270):
# batch 512, seq_q 1, 64 heads, top-k 128 over 512 pages of 64, attention sink, top-k lengths;
# plus an extra cache of top-k 512 (64-token pages) or 8192 (2-token pages).
MLA_CASES = {
    "decode": dict(batch=512, topk=128, num_pages=512),
    "extra512": dict(batch=512, topk=128, num_pages=512, extra_topk=512, extra_page=64,
                     extra_pages=512),
    "extra8192": dict(batch=512, topk=128, num_pages=512, extra_topk=8192, extra_page=2,
                      extra_pages=512),
}


def make_mla_workload(batch: int = 8, topk: int = 128, num_pages: int = 16, page: int = 64,
                      heads: int = 64, seq_q: int = 1, extra_topk: int = 0, extra_page: int = 64,
                      extra_pages: int = 0, topk_length: bool = True, sink: bool = True,
                      seed: int = 43, name: str = "mla", q_scale: float = 1.0) -> MlaWorkload:
    """Seeded inputs shaped like the reference's MODEL1 tests and benchmark:
    q ~ randn (times q_scale), indices uniform over the cache, top-k lengths
    uniform in [1, topk], sink ~ randn."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, seq_q, heads, HEAD_DIM, generator=g)
    q = (q * q_scale).to(torch.bfloat16)
    cache = make_model1_cache(num_pages, page, g)
    idx = torch.randint(0, num_pages * page, (batch, seq_q, topk), generator=g, dtype=torch.int32)
    lens = torch.randint(1, topk + 1, (batch,), generator=g, dtype=torch.int32) if topk_length else None
    sink_t = torch.randn(heads, generator=g) if sink else None
    w = MlaWorkload(name, q, cache, idx, lens, sink_t)
    if extra_topk:
        pages = extra_pages or (extra_topk + extra_page - 1) // extra_page + 4
        w.extra_k_cache = make_model1_cache(pages, extra_page, g)
        w.extra_indices = torch.randint(0, pages * extra_page, (batch, seq_q, extra_topk),
                                        generator=g, dtype=torch.int32)
        if topk_length:
            w.extra_topk_length = torch.randint(1, extra_topk + 1, (batch,), generator=g,
                                                dtype=torch.int32)
    return w


def make_mla_case(case: str, seed: int = 0) -> MlaWorkload:
    """One of the MLA_CASES (bench workloads), q scaled by 1/10 as the
    reference benchmark draws it."""
    return make_mla_workload(seed=seed, name=case, q_scale=0.1, **MLA_CASES[case])


def mla_bytes(w: MlaWorkload) -> int:
    """Algorithmic bytes of one sparse MODEL1 decode call: q read and output
    written (bf16, 512 per head), the LSE, and per attended cache entry its
    4-byte index and 584 cache bytes, once per 64-head block."""
    B, SQ, HQ, D = w.q.shape
    head_blocks = HQ // 64
    return (4 * B * SQ * HQ * D + 4 * B * HQ * SQ
            + head_blocks * w.used_tokens() * (4 + HEAD_BYTES))


def mla_flops(w: MlaWorkload) -> int:
    """MFMA work of one call: QK^T and PV, 2 * 512 multiply-adds each per
    (head, attended entry)."""
    HQ = w.q.shape[2]
    return 4 * HEAD_DIM * HQ * w.used_tokens()


# ---------------------------------------------------------------------------
# Sparse MLA prefill over bf16 rows (flash_mla_sparse_fwd).  Inputs drawn as
# the reference's FlashMLA-style cases draw them
# (tests/test_flash_mla_sparse_fwd.py:232-370): q, kv ~ randn / 10 plus a
# per-call offset, clamped to [-10, 10]; index rows a random permutation of
# [0, s_kv) (as much of it as fits), padded with invalid values; sink ~ randn
# with about a third set to -inf and a third to +inf; top-k lengths uniform in
# [0, max(topk + 1, 64)) clamped to topk.
# ---------------------------------------------------------------------------

MLA_SPARSE_INVALID = (-2147483648, -123456, -1, None, 114514, 1919810, 2147480000, 2147483647)  # None: s_kv

# Reference benchmark cases (benchmark/test_flash_mla_sparse_fwd.py:105-121):
# s_q 4096 with the attention sink, name -> (s_kv, topk, h_q, d_qk).
MLA_SPARSE_CASES = {
    **{f"v32_{s // 1024}k": (s, 2048, 128, 576) for s in (8192, 32768, 65536, 98304, 131072)},
    **{f"h64_{s // 1024}k": (s, 512, 64, 512) for s in (8192, 32768, 49152, 65536)},
    **{f"h128_{s // 1024}k": (s, 1024, 128, 512) for s in (8192, 32768, 49152, 65536)},
}


@dataclass
class MlaSparseInputs:
    q: torch.Tensor            # [s_q, h_q, d_qk] bf16
    kv: torch.Tensor           # [s_kv, 1, d_qk] bf16
    indices: torch.Tensor      # [s_q, 1, topk] int32
    attn_sink: Optional[torch.Tensor]
    topk_length: Optional[torch.Tensor]
    sm_scale: float

    def to(self, device) -> "MlaSparseInputs":
        mv = lambda t: t.to(device) if t is not None else None
        return MlaSparseInputs(mv(self.q), mv(self.kv), mv(self.indices), mv(self.attn_sink),
                               mv(self.topk_length), self.sm_scale)

    def args(self):
        return (self.q, self.kv, self.indices, self.sm_scale, 512, self.attn_sink, self.topk_length)


def _index_rows(s_q: int, s_kv: int, topk: int, g: torch.Generator, affine: bool) -> torch.Tensor:
    """[s_q, topk] int32: row t is distinct ids of [0, s_kv) (min(s_kv, topk)
    of them) then invalid padding.  affine: the ids are an arithmetic
    progression mod s_kv with a step coprime to s_kv (O(topk) per row, for the
    benchmark's sizes); otherwise a uniformly random permutation prefix."""
    n = min(s_kv, topk)
    rows = torch.empty(s_q, topk, dtype=torch.int32)
    if n:
        if affine:
            pos = torch.arange(n, dtype=torch.int64)
            off = torch.randint(0, s_kv, (s_q,), generator=g)
            step = torch.randint(1, max(2, s_kv), (s_q,), generator=g).tolist()
            for t in range(s_q):
                while s_kv > 1 and math.gcd(step[t], s_kv) != 1:
                    step[t] = step[t] % (s_kv - 1) + 1
            rows[:, :n] = ((off[:, None] + torch.tensor(step)[:, None] * pos) % s_kv).to(torch.int32)
        else:
            rows[:, :n] = torch.rand(s_q, s_kv, generator=g).argsort(-1)[:, :n].to(torch.int32)
    if n < topk:
        cands = torch.tensor([s_kv if c is None else c for c in MLA_SPARSE_INVALID], dtype=torch.int64)
        pick = torch.randint(0, len(cands), (s_q, topk - n), generator=g)
        rows[:, n:] = cands[pick].to(torch.int32)
    return rows


def make_mla_sparse_inputs(s_q: int, s_kv: int, topk: int, h_q: int = 128, d_qk: int = 512,
                           have_attn_sink: bool = False, have_topk_length: bool = False,
                           all_invalid_rows: bool = False, seed: int = 0, sm_scale: float = 0.5,
                           affine: Optional[bool] = None) -> MlaSparseInputs:
    """Seeded CPU inputs for flash_mla_sparse_fwd (see the section comment)."""
    g = torch.Generator().manual_seed(seed)
    off_q, off_kv = (torch.rand(2, generator=g) - 0.5) / 10
    q = (randn_bf16((s_q, h_q, d_qk), g).float() / 10 + off_q).clamp_(-10, 10).to(torch.bfloat16)
    kv = (randn_bf16((s_kv, 1, d_qk), g).float() / 10 + off_kv).clamp_(-10, 10).to(torch.bfloat16)
    if affine is None:
        affine = s_q * s_kv > (1 << 26)
    idx = _index_rows(s_q, s_kv, topk, g, affine)
    if all_invalid_rows:
        dead = torch.randn(s_q, generator=g) < -1
        idx[dead] = -1
    sink = None
    if have_attn_sink:
        sink = torch.randn(h_q, generator=g)
        m = torch.randn(h_q, generator=g)
        sink[m < -0.5] = float("-inf")
        sink[m > 0.5] = float("inf")
    lens = None
    if have_topk_length:
        lens = torch.randint(0, max(topk + 1, 64), (s_q,), generator=g).clamp_max(topk).to(torch.int32)
    return MlaSparseInputs(q, kv, idx.view(s_q, 1, topk), sink, lens, sm_scale)


def mla_sparse_used(w: MlaSparseInputs) -> int:
    """(token, entry) pairs attended: entries inside the length with an id in [0, s_kv)."""
    s_q, _, topk = w.indices.shape
    idx = w.indices.reshape(s_q, topk).cpu().long()
    ok = (idx >= 0) & (idx < w.kv.shape[0])
    if w.topk_length is not None:
        ok &= torch.arange(topk)[None, :] < w.topk_length.cpu().long().clamp(0, topk)[:, None]
    return int(ok.sum())


def mla_sparse_flops(w: MlaSparseInputs) -> int:
    """MFMA work: per (head, attended entry) d_qk multiply-adds for QK and 512 for PV."""
    h_q, d_qk = w.q.shape[1], w.q.shape[2]
    return 2 * (d_qk + HEAD_DIM) * h_q * mla_sparse_used(w)


def mla_sparse_bytes(w: MlaSparseInputs) -> int:
    """Algorithmic bytes: q read, out written (bf16), max_logits and lse
    (float32), the index rows, and each attended row (2 d_qk bytes) once per
    64-head block."""
    s_q, h_q, d_qk = w.q.shape
    return (2 * s_q * h_q * (d_qk + HEAD_DIM) + 8 * s_q * h_q + 4 * w.indices.numel()
            + (h_q // 64) * mla_sparse_used(w) * 2 * d_qk)


# ---------------------------------------------------------------------------
# Sparse-indexer key cache (indexer_k_quant_and_cache / its gather).  Shapes of
# the reference's tests (tests/test_indexer_k_quant_and_cache.py:177-185,
# tests/test_cp_gather_indexer_k_quant_cache.py:168-175) and benchmarks
# (benchmark/test_indexer_k_quant_and_cache.py:97-102,
# benchmark/test_cp_gather_indexer_k_quant_cache.py:125-131).
# ---------------------------------------------------------------------------

INDEXER_QUANT_BLOCK = 128
INDEXER_K_INSERT_CASES = [  # num_tokens, num_blocks, block_size, head_dim (reference benchmark)
    (128, 16, 16, 128), (512, 64, 16, 128), (1024, 128, 16, 512), (2048, 256, 16, 512)]
INDEXER_K_GATHER_CASES = [  # batch, seq_len, block_size, head_dim (reference benchmark)
    (4, 256, 16, 128), (8, 512, 16, 128), (16, 1024, 16, 512), (32, 1024, 16, 512)]


def indexer_k_row_bytes(head_dim: int) -> int:
    """Cache bytes per token: head_dim e4m3fn codes + a float32 scale per 128."""
    return head_dim + 4 * (head_dim // INDEXER_QUANT_BLOCK)


def make_indexer_k_cache(num_blocks: int, block_size: int, head_dim: int, gen: torch.Generator) -> torch.Tensor:
    """uint8 [num_blocks, block_size, row bytes] filled as the reference's tests
    fill it: codes of N(0, 1) samples, scales uniform in [0.01, 1.01)."""
    nqb = head_dim // INDEXER_QUANT_BLOCK
    cache = torch.empty(num_blocks, block_size, indexer_k_row_bytes(head_dim), dtype=torch.uint8)
    flat = cache.view(num_blocks, -1)
    codes = torch.randn(num_blocks, block_size * head_dim, generator=gen).to(torch.float8_e4m3fn)
    flat[:, :block_size * head_dim] = codes.view(torch.uint8)
    flat[:, block_size * head_dim:].view(torch.float32)[:] = (
        torch.rand(num_blocks, block_size * nqb, generator=gen) + 0.01)
    return cache


def make_indexer_k_insert(num_tokens: int, num_blocks: int, block_size: int, head_dim: int,
                          dtype=torch.bfloat16, seed: int = 0):
    """(k, kv_cache, slot_mapping): N(0, 1) keys, distinct random slots with the
    last one -1, as the reference's test draws them."""
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(num_tokens, head_dim, generator=g).to(dtype)
    slots = torch.randperm(num_blocks * block_size, generator=g)[:num_tokens].to(torch.int64)
    if num_tokens:
        slots[-1] = -1
    return k, make_indexer_k_cache(num_blocks, block_size, head_dim, g), slots


def make_indexer_k_gather(seq_lens, block_size: int, head_dim: int, extra_tokens: int = 0, seed: int = 1,
                          sentinel: int = 0x7B):
    """(k_cache, k_fp8, k_fp8_scale, block_table, cu_seqlen) with the reference
    test's metadata: consecutive blocks per request, -1 past each request's
    blocks, outputs pre-filled with a sentinel byte, extra_tokens rows past
    the last request."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.tensor(seq_lens, dtype=torch.int32)
    cu = torch.zeros(len(seq_lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    per = [(n + block_size - 1) // block_size for n in seq_lens]
    table = torch.full((len(seq_lens), max(1, max(per))), -1, dtype=torch.int32)
    nxt = 0
    for b, n in enumerate(per):
        table[b, :n] = torch.arange(nxt, nxt + n, dtype=torch.int32)
        nxt += n
    cache = make_indexer_k_cache(max(1, nxt), block_size, head_dim, g)
    rows = int(cu[-1]) + extra_tokens
    k_fp8 = torch.full((rows, head_dim), sentinel, dtype=torch.uint8).view(torch.float8_e4m3fn)
    k_scale = torch.full((rows, 4 * (head_dim // INDEXER_QUANT_BLOCK)), sentinel, dtype=torch.uint8)
    return cache, k_fp8, k_scale, table, cu


def indexer_k_insert_bytes(num_tokens: int, head_dim: int, key_bytes: int = 2) -> int:
    """Algorithmic HBM bytes of one insert: key row read, slot read, codes and
    scales written."""
    return num_tokens * (key_bytes * head_dim + 8 + indexer_k_row_bytes(head_dim))


def indexer_k_gather_bytes(num_tokens: int, head_dim: int) -> int:
    """Algorithmic HBM bytes of one gather: per token the cached row read and
    written out, and its 4-byte block-table entry."""
    return num_tokens * (2 * indexer_k_row_bytes(head_dim) + 4)


# ---------------------------------------------------------------------------
# Sparse-indexer logits (fp8_fp4_mqa_logits / fp8_fp4_paged_mqa_logits):
# inputs drawn as the reference's tests draw them
# (tests/test_fp8_fp4_mqa_logits.py:168-186, tests/test_fp8_fp4_paged_mqa_logits.py:29-114).
# ---------------------------------------------------------------------------

MQA_HEADS = 64
MQA_DECODE_SHAPES = [(1, 1024), (1, 2048), (1, 4096), (4, 2048), (4, 4096)]
MQA_PREFILL_SHAPES = [(64, 4096), (256, 4096), (1024, 4096), (2048, 4096), (1024, 8192)]
PAGED_MQA_SHAPES = [(4, 1, 512), (4, 1, 1024), (4, 1, 2048), (8, 1, 1024), (8, 2, 1024), (16, 1, 2048),
                    (32, 1, 4096), (64, 1, 4096), (128, 1, 2048)]
PAGED_MQA_BENCH_SHAPES = [(256, 1, 1024), (256, 1, 2048), (256, 1, 4096), (256, 1, 8192), (256, 2, 8192),
                          (128, 1, 16384), (64, 1, 32768), (32, 1, 65536)]
PAGED_MAX_MODEL_LEN = 111 * 1024
_E2M1_MAGS = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def quantize_mxfp4(x: torch.Tensor):
    """(packed uint8 [..., D/2] (even element in the low nibble), int32 [...]
    of the D/32 UE8M0 bytes) for float x with D = 128: per 32 elements
    scale 2^ceil(log2(amax / 6)), elements rounded to the nearest E2M1 value,
    ties to the even code."""
    D = x.shape[-1]
    xb = x.float().reshape(*x.shape[:-1], D // 32, 32)
    amax = xb.abs().amax(-1, keepdim=True).clamp_min(6.0 * 2.0 ** -126)
    e = torch.ceil(torch.log2(amax / 6.0))
    y = (xb / torch.exp2(e)).clamp(-6.0, 6.0)
    dist = (y.abs()[..., None] - _E2M1_MAGS).abs() + (torch.arange(8) % 2) * 1e-6
    code = dist.argmin(-1) | ((y < 0).long() << 3)
    code = code.reshape(*x.shape[:-1], D)
    packed = (code[..., 0::2] | (code[..., 1::2] << 4)).to(torch.uint8)
    byte = (e.squeeze(-1) + 127).long()
    scale = torch.zeros(x.shape[:-1], dtype=torch.int64)
    for b in range(D // 32):
        scale |= byte[..., b] << (8 * b)
    return packed, scale.to(torch.int32)


def fp8_per_token(x: torch.Tensor):
    """(e4m3fn codes, float32 scale per row) with scale = max(amax, 1e-4) / 448."""
    sf = x.float().abs().amax(-1).clamp_min(1e-4) / 448.0
    return (x.float() / sf[..., None]).to(torch.float8_e4m3fn), sf


def make_mqa_logits_inputs(M: int, N: int, H: int = MQA_HEADS, fp4: bool = False, seed: int = 42):
    """(q, kv, weights, ks, ke) on the CPU: q ~ N(0, 1) cast to e4m3fn (or
    MXFP4), k ~ N(0, 1) per-token FP8 with float32 scales, weights |N(0, 1)|,
    ks = 0 and ke = N as the reference test builds them."""
    g = torch.Generator().manual_seed(seed)
    qf = torch.randn(M, H, 128, generator=g).to(torch.bfloat16)
    kf = torch.randn(N, 128, generator=g).to(torch.bfloat16)
    w = torch.randn(M, H, generator=g).abs()
    q = quantize_mxfp4(qf) if fp4 else (qf.to(torch.float8_e4m3fn), None)
    k, ks = fp8_per_token(kf)
    return q, (k, ks), w, torch.zeros(M, dtype=torch.int32), torch.full((M,), N, dtype=torch.int32)


def make_paged_cache(num_blocks: int, block_size: int, gen: torch.Generator) -> torch.Tensor:
    """uint8 [num_blocks, block_size, 1, 132] as the reference test fills it:
    N(0, 1) keys, per-token scale max(amax, 1e-4) / 448, codes then scales."""
    x = torch.randn(num_blocks, block_size, 128, generator=gen).to(torch.bfloat16)
    codes, sf = fp8_per_token(x)
    cache = torch.empty(num_blocks, block_size * 132, dtype=torch.uint8)
    cache[:, :block_size * 128] = codes.view(torch.uint8).reshape(num_blocks, -1)
    cache[:, block_size * 128:] = sf.reshape(num_blocks, block_size).contiguous().view(torch.uint8)
    return cache.view(num_blocks, block_size, 1, 132)


def make_paged_mqa_inputs(batch: int, next_n: int, avg_ctx: int, fp4: bool = False, block_size: int = 64,
                          num_blocks: int = None, seed: int = 0):
    """(q, kv_cache, weights, context_lens [B, next_n], block_tables) as the
    reference test draws them: lengths uniform in [0.7, 1.3] x avg_ctx,
    distinct random blocks per sequence."""
    g = torch.Generator().manual_seed(seed)
    qf = torch.randn(batch, next_n, MQA_HEADS, 128, generator=g).to(torch.bfloat16)
    w = torch.randn(batch * next_n, MQA_HEADS, generator=g)
    base = torch.randint(max(1, int(0.7 * avg_ctx)), int(1.3 * avg_ctx) + 1, (batch,), generator=g,
                         dtype=torch.int32)
    per = (base + block_size - 1) // block_size
    need = int(per.sum())
    num_blocks = num_blocks or max(need + 16, 64)
    cache = make_paged_cache(num_blocks, block_size, g)
    table = torch.zeros(batch, int(per.max()), dtype=torch.int32)
    pool = torch.randperm(num_blocks, generator=g).to(torch.int32)
    off = 0
    for b in range(batch):
        n = int(per[b])
        if off + n > num_blocks:
            pool, off = torch.randperm(num_blocks, generator=g).to(torch.int32), 0
        table[b, :n] = pool[off:off + n]
        off += n
    q = quantize_mxfp4(qf) if fp4 else (qf.to(torch.float8_e4m3fn), None)
    if fp4:
        q = (q[0], q[1])
    ctx = base[:, None].expand(batch, next_n).contiguous()
    return q, cache, w, ctx, table


def mqa_logits_flops(M: int, N: int, H: int = MQA_HEADS) -> int:
    return 2 * M * N * H * 128


def paged_mqa_logits_bytes(ctx: torch.Tensor, rows: int, H: int, max_model_len: int, fp4: bool) -> int:
    """Algorithmic HBM bytes of one paged call: each row's context keys (132 B
    with the scale) and a 4-byte block-table entry per 64 positions, q and
    weights per row, and the whole float32 output row."""
    q_bytes = H * (64 + 4 if fp4 else 128) + 4 * H
    return int(ctx.sum()) * 132 + int(ctx.sum()) // 16 + rows * (q_bytes + 4 * max_model_len)
