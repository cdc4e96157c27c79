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
                           seed: int = 0, scale: float = 1.0, max_pos: int = 65536) -> InvRopeWorkload:
    """Seeded CPU inputs for the sibling op (default: T=8192, H=64, G=8)."""
    g = torch.Generator().manual_seed(seed)
    o = randn_bf16((num_tokens, num_heads, HEAD_DIM), g)
    if scale != 1.0:
        o = (o.float() * scale).to(torch.bfloat16)
    positions = torch.randint(0, max_pos, (num_tokens,), generator=g, dtype=torch.int64)
    return InvRopeWorkload(o, positions, make_cos_sin_cache(max_pos), n_groups,
                           num_heads // n_groups)
