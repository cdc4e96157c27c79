"""The FP8 quantisers of the main op and the sibling over their whole exponent
range, on inputs built so that every exponent the quantiser can produce
occurs, with every bf16 magnitude at or below each group's maximum.

Main op (reference ops/fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:115-145,
280-286; exact-byte bar at tests/test_fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:246-289):
per 64-element group k = ceil(log2(max(amax, 1e-4) / 448)), codes
e4m3fn(clamp(x * 2^-k, +-448)), scale byte k + 127.  For bf16 input k runs
from -22 (the 1e-4 floor) to 120 (the bf16 maximum), so the scale bytes run
105..247.  Every k is hit twice: with amax = 448 * 2^k exactly (the largest
amax giving k; its mantissa is the closed form's 0x600000 boundary) and with
the next bf16 above 448 * 2^(k-1) (the smallest).  The other 63 slots of
each group take every bf16 magnitude at or below amax (both signs; +-0), so
every code, subnormals included, and every rounding tie the kernel's
v_cvt_pk_fp8_f32 can meet occurs at every k.  All-zero groups and groups
below the floor complete it.

Sibling (reference ops/fused_inv_rope_fp8_quant.py:61-154): per 128-element
chunk s = max(amax, eps) * fl32(1/448), then either x / s (fp32 scales) or
x * 2^-ceil(log2(max(s, 1e-10))) (packed UE8M0); both clamp to +-448 first.
amax spans 1e-12 (below eps) to the bf16 maximum: four mantissas in every
binade, each chunk filled with the magnitudes within 2^-22 of amax (every
value that can give a nonzero code) and a few below.  Rows whose amax is at
most 2^100 are rotated at random positions, the others at position 0
(cos 1, sin 0), so that the rotation cannot overflow binary32.

CPU tests pin the inputs (every exponent and every finite code occurs; the C
oracle equals the torch restatement of the reference on them); GPU tests
compare the kernels' bytes with the C oracle bit for bit.
"""
import pytest
import torch

import oracle
from flaggems_vllm import testing as W
from oracle import torch_ref

DEV = torch.device("cuda:0")
BF16_MAX_BITS = 0x7F7F


def _bf16(bits):
    return torch.as_tensor(bits, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


def _positive_bf16_upto(limit_bits, floor_bits=1):
    """Every positive finite bf16 value with bits in [floor_bits, limit_bits]
    (bf16 bit order equals value order for positive numbers)."""
    return _bf16(torch.arange(max(1, floor_bits), limit_bits + 1)).float()


def _groups(amax_bits, per_group, floor_bits=1):
    """Groups of per_group + 1 values: amax first (sign alternating by group),
    then every magnitude in [floor_bits, amax_bits] once with each sign, and
    +0 / -0, padded with zeros."""
    mag = _positive_bf16_upto(amax_bits, floor_bits)
    vals = torch.cat([mag, -mag, torch.tensor([0.0, -0.0])])
    n = (vals.numel() + per_group - 1) // per_group
    body = torch.zeros(n * per_group)
    body[:vals.numel()] = vals
    top = _bf16(amax_bits).float().repeat(n)
    top[1::2] = -top[1::2]
    return torch.cat([top[:, None], body.view(n, per_group)], dim=1)


def _kv_bits_for_exponent(k):
    """(largest, smallest) bf16 bits whose KV group exponent is k."""
    top = min(((k + 8 + 127) << 7) | 0x60, BF16_MAX_BITS)   # 448 * 2^k = 1.75 * 2^(k+8)
    low = (((k + 7 + 127) << 7) | 0x60) + 1                   # just above 448 * 2^(k-1)
    return top, low


def main_op_sweep_rows():
    """kv rows [n, 512] bf16: 7 quant groups per row from the groups above,
    dims 448..511 (the RoPE slice, not quantised) seeded N(0, 1)."""
    groups = []
    for k in range(-22, 121):
        top, low = _kv_bits_for_exponent(k)
        groups.append(_groups(top, 63))
        # the smallest amax of k: its window of magnitudes that can give a
        # nonzero code (x >= amax * 2^-22) and every code at the low edge
        groups.append(_groups(low, 63, floor_bits=max(1, low - 22 * 128)))
    # the 1e-4 floor: all-zero groups (+0 and -0), groups whose amax is below
    # or at the floor
    groups.append(torch.zeros(2, 64))
    groups.append(torch.full((2, 64), -0.0))
    for amax in (5e-5, 9.98e-5, 1.0e-4, 1.0014e-4):
        bits = int(torch.tensor(amax).to(torch.bfloat16).view(torch.int16))
        groups.append(_groups(bits, 63))
    g = torch.cat(groups)
    rows = (g.shape[0] + 6) // 7
    nope = torch.zeros(rows * 7, 64)
    nope[:g.shape[0]] = g
    gen = torch.Generator().manual_seed(21)
    rope = torch.randn(rows, 64, generator=gen)
    return torch.cat([nope.view(rows, 448), rope], dim=1).to(torch.bfloat16)


def main_op_sweep_workload():
    kv = main_op_sweep_rows()
    T = kv.shape[0]
    gen = torch.Generator().manual_seed(22)
    bs = 64
    nblk = (T + bs - 1) // bs + 1
    slots = torch.randperm(nblk * bs, generator=gen)[:T].to(torch.int64)
    slots[::97] = -1
    return W.Workload("kv quant sweep", W.randn_bf16((T, 1, 512), gen), kv,
                      torch.zeros(nblk, bs * W.HEAD_BYTES, dtype=torch.uint8), slots,
                      torch.randint(0, 4096, (T,), generator=gen, dtype=torch.int64),
                      W.make_cos_sin_cache(4096), 1e-6, bs)


def sibling_sweep_inputs():
    """(o [T, 1, 512] bf16, positions [T]) for G = 1, heads_per_group = 1."""
    chunks, big = [], []
    amaxes = []
    for e in range(-40, 128):
        for mant in (0x00, 0x30, 0x60, 0x7F):
            bits = ((e + 127) << 7) | mant
            if bits <= BF16_MAX_BITS:
                amaxes.append(bits)
    for a in (1e-12, 5e-11, 9.99e-11, 1e-10, 1.01e-10):
        amaxes.append(int(torch.tensor(a).to(torch.bfloat16).view(torch.int16)))
    for bits in amaxes:
        c = _groups(bits, 127, floor_bits=max(1, bits - 22 * 128))
        # a few magnitudes far below the window (they give code 0)
        c[0, 1:4] = _bf16([max(1, bits - 40 * 128), 1, 0x0080]).float()
        chunks.append(c)
        big.extend([bits > ((100 + 127) << 7)] * c.shape[0])
    x = torch.cat(chunks)
    big = torch.tensor(big)
    rows = (x.shape[0] + 3) // 4
    o = torch.zeros(rows * 4, 128)
    o[:x.shape[0]] = x
    big_row = torch.zeros(rows * 4, dtype=torch.bool)
    big_row[:x.shape[0]] = big
    big_row = big_row.view(rows, 4).any(1)
    gen = torch.Generator().manual_seed(23)
    pos = torch.randint(0, 4096, (rows,), generator=gen, dtype=torch.int64)
    pos[big_row] = 0
    return o.view(rows, 1, 512).to(torch.bfloat16), pos


# ------------------------------------------------------------------- CPU ----

def test_main_sweep_covers_every_exponent_and_code():
    """The oracle, run on the sweep, writes every scale byte 105..247 and,
    across all groups, all 254 finite e4m3 codes; the torch restatement of
    the reference's oracle writes the same cache bytes."""
    w = main_op_sweep_workload()
    a = w.clone()
    oracle.qnorm_rope_kv_insert(*a.args())
    b = w.clone()
    torch_ref.qnorm_rope_kv_insert(*b.args())
    assert torch.equal(a.k_cache, b.k_cache)
    keep = w.slot_mapping >= 0
    from tests._helpers import slot_byte_index
    idx = slot_byte_index(w.slot_mapping[keep], w.block_size, w.k_cache.stride(0))
    got = a.k_cache.view(-1)[idx]
    scale_bytes = set(got[:, 576:583].flatten().tolist())
    assert scale_bytes == set(range(105, 248))
    codes = set(got[:, :448].flatten().tolist())
    assert codes == set(range(256)) - {0x7F, 0xFF}
    assert int(got[:, 583].abs().sum()) == 0


@pytest.mark.parametrize("tma", [False, True])
def test_sibling_sweep_oracles_agree(tma):
    """The C oracle and the torch restatement of the reference's oracle give
    the same codes and scales over the whole sweep; the packed mode's scale
    bytes span the range the eps floor and the bf16 maximum allow."""
    o, pos = sibling_sweep_inputs()
    cs = W.make_cos_sin_cache(4096)
    c8, cs_ = oracle.inv_rope_fp8_quant(o, pos, cs, 1, 1, tma_aligned_scales=tma)
    t8, ts = torch_ref.inv_rope_fp8_quant(o, pos, cs, 1, 1, tma_aligned_scales=tma)
    assert torch.equal(c8, t8)
    assert torch.equal(cs_.contiguous(), ts)
    codes = set(c8.flatten().tolist())
    assert codes == set(range(256)) - {0x7F, 0xFF}
    if tma:
        b = ((cs_.contiguous() >> 0) & 0xFF).flatten()
        assert int(b.min()) <= 94 and int(b.max()) >= 247   # 2^-33 (eps floor) .. 2^120


# ------------------------------------------------------------------- GPU ----

@pytest.mark.gpu
def test_gpu_main_op_kv_quant_every_exponent():
    """The main op on the sweep: the whole cache, q and kv bit for bit against
    the C oracle."""
    import flaggems_vllm

    w = main_op_sweep_workload()
    print(f"\n[case] main op kv quant sweep T={w.num_tokens}", flush=True)
    ref = w.clone()
    oracle.qnorm_rope_kv_insert(*ref.args())
    g = w.to(DEV)
    flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(*g.args())
    torch.cuda.synchronize()
    gc = g.k_cache.cpu()
    if not torch.equal(gc, ref.k_cache):
        diff = torch.nonzero(gc.view(-1) != ref.k_cache.view(-1)).flatten()
        raise AssertionError(f"{diff.numel()} cache bytes differ; first at byte {int(diff[0])}: "
                             f"gpu {int(gc.view(-1)[diff[0]])} oracle {int(ref.k_cache.view(-1)[diff[0]])}")
    assert torch.equal(g.q.cpu().view(torch.int16), ref.q.view(torch.int16))
    assert torch.equal(g.kv.cpu(), w.kv)


@pytest.mark.gpu
@pytest.mark.parametrize("tma", [False, True])
def test_gpu_sibling_quant_every_exponent(tma):
    """The sibling on the sweep, fp32 and packed UE8M0 scales: codes and
    scales bit for bit against the C oracle."""
    import flaggems_vllm

    o, pos = sibling_sweep_inputs()
    print(f"\n[case] sibling quant sweep T={o.shape[0]} tma={tma}", flush=True)
    cs = W.make_cos_sin_cache(4096)
    r8, rs = oracle.inv_rope_fp8_quant(o, pos, cs, 1, 1, tma_aligned_scales=tma)
    g8, gs = flaggems_vllm.fused_inv_rope_fp8_quant(o.to(DEV), pos.to(DEV), cs.to(DEV), 1, 1,
                                                    tma_aligned_scales=tma)
    torch.cuda.synchronize()
    g8 = g8.cpu().view(torch.uint8)
    if not torch.equal(g8, r8):
        d = torch.nonzero(g8 != r8)
        t, _, i = d[0].tolist()
        raise AssertionError(f"{d.shape[0]} codes differ; first token {t} dim {i}: "
                             f"gpu {int(g8[t, 0, i])} oracle {int(r8[t, 0, i])}")
    assert torch.equal(gs.cpu().view(torch.int32), rs.view(torch.int32))
