"""Shared helpers for the parity tests (comparison metrics, sub-sampling)."""
import torch

import oracle
from flaggems_vllm import testing as W


def bf16_ulp_distance(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|a - b| in bf16 ulps (monotone integer order of the bit patterns;
    +0 and -0 are the same point)."""
    def order(x):
        bits = x.contiguous().view(torch.int16).to(torch.int32)
        mag = bits & 0x7FFF
        return torch.where(bits < 0, -mag, mag)

    return (order(a) - order(b)).abs()


def rope_cancellation_bound(y_ref_f32: torch.Tensor, cos_sin: torch.Tensor) -> torch.Tensor:
    """Allowed difference for each rope output when the RMS factor r of two
    implementations differs by a few float32 ulps: the rotated value
    e*c - o*s (or e*s + o*c) moves by at most (|e*c| + |o*s|) * 2^-20 before
    the final bf16 rounding.  y_ref_f32: [..., 64] the normalised rope inputs;
    cos_sin: [..., 64] broadcastable (cos | sin)."""
    c, s = cos_sin[..., :32], cos_sin[..., 32:]
    e, o = y_ref_f32[..., 0::2], y_ref_f32[..., 1::2]
    be = (e * c).abs() + (o * s).abs()
    bo = (e * s).abs() + (o * c).abs()
    return torch.stack((be, bo), dim=-1).flatten(-2) * 2.0 ** -20


def bf16_ulp_size(x: torch.Tensor) -> torch.Tensor:
    """Size of one bf16 ulp at |x| (float32)."""
    xf = x.float().abs().clamp(min=2.0 ** -126)
    e = torch.floor(torch.log2(xf))
    return torch.exp2(e - 7)


def sub_workload(w: W.Workload, tokens: torch.Tensor) -> W.Workload:
    """The main-op workload restricted to ``tokens`` (sorted, all < T), with
    each kept token's slot (or -1 if it is past slot_mapping's end)."""
    n_ins = w.slot_mapping.shape[0]
    slots = torch.full((tokens.numel(),), -1, dtype=torch.int64)
    inside = tokens < n_ins
    slots[inside] = w.slot_mapping[tokens[inside]]
    return W.Workload(w.name + "-sub", w.q[tokens].clone(), w.kv[tokens].clone(),
                      torch.zeros_like(w.k_cache), slots, w.position_ids[tokens].clone(),
                      w.cos_sin_cache, w.eps, w.block_size)


def slot_byte_index(slots: torch.Tensor, block_size: int, block_stride: int):
    """Flat byte offsets [n, 584] of each slot's token data and scale bytes."""
    blk, p = slots // block_size, slots % block_size
    base = blk * block_stride
    data = base[:, None] + p[:, None] * 576 + torch.arange(576, device=slots.device)
    scale = base[:, None] + block_size * 576 + p[:, None] * 8 + torch.arange(8, device=slots.device)
    return torch.cat((data, scale), dim=1)


def split_cache(cache: torch.Tensor, block_size: int):
    """(token data [num_blocks * bs, 576], scale bytes [num_blocks * bs, 8]) of
    a paged cache, indexed by slot."""
    nblk = cache.shape[0]
    rows = cache.view(nblk, -1)
    data = rows[:, :block_size * 576].reshape(nblk * block_size, 576)
    scales = rows[:, block_size * 576:block_size * 584].reshape(nblk * block_size, 8)
    return data, scales


def oracle_main(w: W.Workload) -> W.Workload:
    r = w.clone()
    oracle.qnorm_rope_kv_insert(*r.args())
    return r
