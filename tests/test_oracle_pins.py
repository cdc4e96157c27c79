"""CPU pins of the oracle: every function of oracle/ is checked against a
library routine, exact arithmetic or a closed form that a plausible mistake
(dropped term, wrong sign, transposed operand, off-by-one exponent) fails.

* e4m3fn encoder   vs torch's CPU cast, exhaustively over every bf16 value at
                   every power-of-two scale that can reach the encoder, plus
                   random binary32 patterns and the tie / overflow points
* bf16 rounding    vs torch's CPU cast on random binary32 patterns
* UE8M0 exponent   vs exact rational arithmetic for every positive bf16 amax
* RMS factor       vs exact rational arithmetic + high-precision sqrt
* RoPE             closed-form rotations (identity, quarter turn, inverse)
* cache placement  brute force over a small, padded, sentinel-filled cache
* whole ops        C oracle vs the torch restatement (two implementations)
"""
import decimal
import math
import struct
from fractions import Fraction

import pytest
import torch

import oracle
from flaggems_vllm import testing as W
from oracle import torch_ref

from ._helpers import bf16_ulp_distance, split_cache


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def ulp32(x: float) -> float:
    return 2.0 ** (math.floor(math.log2(abs(x))) - 23)


def all_bf16_finite() -> torch.Tensor:
    bits = torch.arange(-(1 << 15), 1 << 15, dtype=torch.int32).to(torch.int16)
    v = bits.view(torch.bfloat16).float()
    return v[torch.isfinite(v)]


# ---------------------------------------------------------------- e4m3fn ----

def test_e4m3_encoder_exhaustive_over_bf16_times_pow2():
    """What reaches the encoder is bf16 * 2^-k (k = -22..120) clamped to +-448:
    every value with an 8-bit significand.  Check all bf16 magnitudes scaled by
    2^j over the whole range that can land in [2^-12, 480]."""
    v = all_bf16_finite()
    v = v[v.abs() <= 480.0]
    for j in range(-4, 12):
        x = (v * 2.0 ** -j).float()
        x = x[x.abs() <= 480.0]
        got = oracle.e4m3fn_codes(x)
        want = x.to(torch.float8_e4m3fn).view(torch.uint8)
        assert torch.equal(got, want), f"scale 2^-{j}: {int((got != want).sum())} codes differ"


def test_e4m3_encoder_random_and_special():
    g = torch.Generator().manual_seed(5)
    bits = torch.randint(-(1 << 31), 1 << 31, (4_000_000,), generator=g, dtype=torch.int64)
    x = bits.to(torch.int32).view(torch.float32)
    x = x[torch.isfinite(x)]
    x = torch.cat([x, x.clamp(-500, 500), torch.rand(1_000_000, generator=g) * 960 - 480])
    specials = torch.tensor([0.0, -0.0, 448.0, -448.0, 464.0, 464.0001, 465.0, 479.9, 480.0,
                             2.0 ** -6, 2.0 ** -7, 2.0 ** -9, 2.0 ** -10, 2.0 ** -10 * 1.0001,
                             3 * 2.0 ** -11, 2.0 ** -11, 1.0625, 1.1875, -1.0625, 1e-30,
                             -1e-30, float("inf"), float("-inf")])
    x = torch.cat([x, specials])
    got = oracle.e4m3fn_codes(x)
    want = x.to(torch.float8_e4m3fn).view(torch.uint8)
    assert torch.equal(got, want), f"{int((got != want).sum())} codes differ"
    # the facts the kernel relies on: 448 is the top finite code, -0 keeps its sign
    assert oracle.lib().oracle_e4m3fn(448.0) == 0x7E
    assert oracle.lib().oracle_e4m3fn(-0.0) == 0x80
    assert oracle.lib().oracle_e4m3fn(464.0) == 0x7E  # tie to even
    assert oracle.lib().oracle_e4m3fn(480.0) == 0x7F  # NaN, no infinity


# ------------------------------------------------------------------ bf16 ----

def test_bf16_rounding_vs_torch():
    g = torch.Generator().manual_seed(6)
    bits = torch.randint(-(1 << 31), 1 << 31, (4_000_000,), generator=g, dtype=torch.int64)
    x = bits.to(torch.int32).view(torch.float32)
    x = x[~torch.isnan(x)]
    # ties: low 16 bits exactly 0x8000 with both parities of bit 16
    ties = (torch.arange(0, 1 << 16, 7, dtype=torch.int32) << 16 | 0x8000).view(torch.float32)
    x = torch.cat([x, ties[~torch.isnan(ties)]])
    got = oracle.bf16_bits(x)
    want = x.to(torch.bfloat16).view(torch.int16)
    assert torch.equal(got, want)


# ----------------------------------------------------------------- UE8M0 ----

def _exact_ceil_log2_ratio(a: Fraction, denom: int) -> int:
    """Smallest integer k with 2^k >= a / denom, in exact arithmetic."""
    r = a / denom
    k = math.floor(math.log2(r)) - 2
    while Fraction(2) ** k < r:
        k += 1
    return k


def test_kv_ue8m0_exponent_exact_all_bf16():
    v = all_bf16_finite()
    v = v[v > 0]
    floor = Fraction(f32(1e-4))
    for a in v.tolist() + [f32(1e-4), 0.0]:
        exact = _exact_ceil_log2_ratio(max(Fraction(a), floor), 448)
        assert oracle.kv_ue8m0_exponent(a) == exact, a
    # the encoded byte stays inside [0, 255] without the clamp for any bf16 amax
    assert 127 + oracle.kv_ue8m0_exponent(float(v.max())) == 247
    assert 127 + oracle.kv_ue8m0_exponent(0.0) == 105


# ------------------------------------------------------------ RMS factor ----

def test_rms_factor_is_correctly_rounded():
    """r = fl32(1/sqrt(fl32(fl32(sum x^2 / 512) + eps))) with the sum exact."""
    decimal.getcontext().prec = 60
    g = torch.Generator().manual_seed(7)
    rows = W.randn_bf16((64, 512), g)
    rows[1] *= 1e-3
    rows[2] = 0
    rows[3, :5] = 300.0
    for eps in (1e-6, 1e-5):
        for row in rows:
            xs = [Fraction(float(x)) for x in row.float().tolist()]
            var = sum(x * x for x in xs) / 512
            w = f32(f32(float(var)) + f32(eps))
            r_exact = 1 / decimal.Decimal(w).sqrt()
            want = f32(float(r_exact))
            got = oracle.rms_factor(row, eps)
            assert got == want, (got, want)
            # and within 2 fp32 ulps of the reference's torch formulation
            ref = torch.rsqrt(row.float().pow(2).mean() + eps).item()
            assert abs(got - ref) <= 2 * ulp32(ref)


# ------------------------------------------------------------------ RoPE ----

def _tiny(T=6, H=3, seed=11, cs=None):
    g = torch.Generator().manual_seed(seed)
    q = W.randn_bf16((T, H, 512), g)
    kv = W.randn_bf16((T, 512), g)
    cache = torch.zeros(2, 8 * 584, dtype=torch.uint8)
    slots = torch.arange(T, dtype=torch.int64)
    pos = torch.randint(0, 16, (T,), generator=g)
    if cs is None:
        cs = W.make_cos_sin_cache(16)
    return W.Workload("tiny", q, kv, cache, slots, pos, cs, 1e-6, 8)


def test_rope_identity_and_quarter_turn():
    ident = torch.zeros(16, 64)
    ident[:, :32] = 1.0
    w = _tiny(cs=ident)
    r = w.clone()
    oracle.qnorm_rope_kv_insert(*r.args())
    x = w.q.float()
    rr = torch.tensor([oracle.rms_factor(row, 1e-6) for row in w.q.reshape(-1, 512)]).view(6, 3, 1)
    assert torch.equal(r.q, (x * rr).to(torch.bfloat16)), "cos=1, sin=0 must leave rope = x*r"
    rope_bytes = split_cache(r.k_cache, 8)[0][:6, 448:576].contiguous()
    assert torch.equal(rope_bytes, w.kv[:, 448:].contiguous().view(torch.uint8)), "kv rope identity"

    quarter = torch.zeros(16, 64)
    quarter[:, 32:] = 1.0  # cos=0, sin=1: (e, o) -> (-o, e)
    w = _tiny(cs=quarter)
    r = w.clone()
    oracle.qnorm_rope_kv_insert(*r.args())
    rope = split_cache(r.k_cache, 8)[0][:6, 448:576].contiguous().view(torch.bfloat16).float()
    src = w.kv[:, 448:].float()
    assert torch.equal(rope[:, 0::2], -src[:, 1::2]) and torch.equal(rope[:, 1::2], src[:, 0::2])


def test_inverse_rope_undoes_forward_rope():
    """Sibling's inverse rotation after the main op's forward rotation returns
    the input within two bf16 roundings."""
    w = _tiny(T=8, H=1, seed=12)
    r = w.clone()
    oracle.qnorm_rope_kv_insert(*r.args())
    fwd = split_cache(r.k_cache, 8)[0][:8, 448:576].contiguous().view(torch.bfloat16)  # [8, 64]
    o = torch.zeros(8, 1, 512, dtype=torch.bfloat16)
    o[:, 0, 448:] = fwd
    o[:, 0, :448] = 1.0
    codes, scales = oracle.inv_rope_fp8_quant(o, w.position_ids, w.cos_sin_cache, 1, 1)
    back = codes.contiguous().view(torch.float8_e4m3fn).float()[:, 0, 448:] * scales[:, 0, 3:4]
    x = w.kv[:, 448:].float()
    amax = x.abs().amax(-1, keepdim=True)
    assert bool(((back - x).abs() <= 2.0 ** -4 * x.abs() + 2.0 ** -8 * amax).all())


# ------------------------------------------------------- cache placement ----

@pytest.mark.parametrize("bs,extra", [(4, 0), (4, 24), (3, 8), (16, 0)])
def test_cache_placement_bruteforce(bs, extra):
    g = torch.Generator().manual_seed(13)
    nblk, T, n_ins = 5, 14, 11
    stride = bs * 584 + extra
    w = _tiny(T=T, H=2, seed=14)
    slots = torch.randperm(nblk * bs, generator=g)[:n_ins].to(torch.int64)
    slots[torch.tensor([1, 6])] = -1
    cache = torch.full((nblk, stride), 0xA5, dtype=torch.uint8)
    w = W.Workload("bf", w.q, w.kv, cache, slots, w.position_ids, w.cos_sin_cache, 1e-6, bs)
    a, b = w.clone(), w.clone()
    oracle.qnorm_rope_kv_insert(*a.args())
    torch_ref.qnorm_rope_kv_insert(*b.args())
    assert torch.equal(a.k_cache, b.k_cache)
    touched = torch.zeros(nblk * stride, dtype=torch.bool)
    flat = a.k_cache.view(-1)
    for t in range(n_ins):
        s = int(slots[t])
        if s < 0:
            continue
        blk, p = s // bs, s % bs
        d0 = blk * stride + p * 576
        s0 = blk * stride + bs * 576 + p * 8
        touched[d0:d0 + 576] = True
        touched[s0:s0 + 8] = True
        assert int(flat[s0 + 7]) == 0, "pad byte"
        rope = flat[d0 + 448:d0 + 576].contiguous().view(torch.bfloat16)
        assert rope.numel() == 64
    assert bool((flat[~touched] == 0xA5).all()), "bytes outside inserted slots changed"
    assert int(touched.sum()) == 584 * int((slots >= 0).sum())
    assert torch.equal(a.kv, w.kv)


def test_dequant_round_trip_and_known_answers():
    """Decoding the cache (codes * 2^(byte-127)) recovers kv's nope values to
    e4m3 precision; a constant-1.0 group encodes as byte 119 (2^-8) and code
    0x78 (256); a group whose amax is 448 uses scale 1 (byte 127)."""
    w = _tiny(T=4, H=1, seed=15)
    w.kv[0, :64] = 1.0
    w.kv[1, :64] = torch.linspace(-448, 448, 64).to(torch.bfloat16)
    r = w.clone()
    oracle.qnorm_rope_kv_insert(*r.args())
    data, scl = split_cache(r.k_cache, 8)
    data, scl = data[:4], scl[:4]
    assert int(scl[0, 0]) == 119 and bool((data[0, :64] == 0x78).all())
    assert int(scl[1, 0]) == 127
    assert torch.equal(data[1, :64], w.kv[1, :64].float().to(torch.float8_e4m3fn).view(torch.uint8))
    codes = data[:, :448].contiguous().view(torch.float8_e4m3fn).float().view(4, 7, 64)
    deq = codes * torch.exp2(scl[:, :7].float() - 127)[..., None]
    x = w.kv[:, :448].float().view(4, 7, 64)
    tol = torch.maximum(x.abs() * 2.0 ** -4, torch.exp2(scl[:, :7].float() - 127 - 10)[..., None])
    assert bool(((deq - x).abs() <= tol).all())


# --------------------------------------------- C oracle vs torch restatement --

@pytest.mark.parametrize("config", [0, 1])
def test_main_op_c_oracle_vs_torch_ref(config):
    w = W.make_workload(config)
    a, b = w.clone(), w.clone()
    oracle.qnorm_rope_kv_insert(*a.args())
    torch_ref.qnorm_rope_kv_insert(*b.args())
    assert torch.equal(a.k_cache, b.k_cache)
    d = bf16_ulp_distance(a.q, b.q)
    assert int(d[..., :448].max()) <= 1 and int(d.max()) <= 2
    assert torch.equal(a.kv, w.kv) and torch.equal(b.kv, w.kv)


def test_main_op_strided_and_dp_padding():
    """c4-style strided views and slot_mapping shorter than q."""
    g = torch.Generator().manual_seed(16)
    T, H = 40, 4
    buf = W.randn_bf16((T, H * 512 + 512), g)
    q, kv = buf[:, :H * 512].view(T, H, 512), buf[:, H * 512:]
    slots = torch.randperm(3 * 64, generator=g)[:33].to(torch.int64)
    slots[::5] = -1
    w = W.Workload("strided", q, kv, torch.zeros(3, 64 * 584, dtype=torch.uint8), slots,
                   torch.randint(0, 4096, (T,), generator=g), W.make_cos_sin_cache(4096), 1e-6, 64,
                   buffer=buf)
    a = w.clone()
    oracle.qnorm_rope_kv_insert(*a.args())
    qc = W.Workload("contig", q.contiguous(), kv.contiguous(), w.k_cache.clone(), slots,
                    w.position_ids, w.cos_sin_cache, 1e-6, 64)
    oracle.qnorm_rope_kv_insert(*qc.args())
    assert torch.equal(a.q, qc.q) and torch.equal(a.k_cache, qc.k_cache)
    b = w.clone()
    torch_ref.qnorm_rope_kv_insert(*b.args())
    assert torch.equal(a.k_cache, b.k_cache)


@pytest.mark.parametrize("tma", [False, True])
@pytest.mark.parametrize("T,H,G,scale", [(7, 64, 8, 1.0), (32, 128, 8, 1.0), (16, 32, 4, 1000.0),
                                         (9, 64, 8, 1e-12)])
def test_sibling_c_oracle_vs_torch_ref(T, H, G, scale, tma):
    w = W.make_inv_rope_workload(T, H, G, seed=3, scale=scale, max_pos=4096)
    c8, cs = oracle.inv_rope_fp8_quant(w.o, w.positions, w.cos_sin_cache, G, H // G,
                                       tma_aligned_scales=tma)
    t8, ts = torch_ref.inv_rope_fp8_quant(w.o, w.positions, w.cos_sin_cache, G, H // G,
                                          tma_aligned_scales=tma)
    assert torch.equal(c8, t8)
    assert torch.equal(cs.contiguous(), ts)
    assert c8.stride() == (H // G * 512, T * H // G * 512, 1)


# Sibling geometries the reference's assertions accept besides DeepSeek-V4's
# (head_dim = nope + rope, quant_group_size | head_dim, the rope dims inside
# the last chunk: nope % group == group - rope), as (nope, rope, group).
SIBLING_GEOMETRIES = [(448, 64, 128), (192, 64, 128), (64, 64, 128), (448, 64, 64), (480, 32, 128),
                      (224, 32, 64), (384, 128, 256), (448, 64, 512), (56, 8, 32), (62, 2, 64), (124, 4, 32)]


def _packed_ok(nope, rope, group, hpg):
    chunks = (nope + rope) // group
    return chunks == 4 or (chunks < 4 and hpg == 1)


@pytest.mark.parametrize("tma", [False, True])
@pytest.mark.parametrize("nope,rope,group", SIBLING_GEOMETRIES)
def test_sibling_geometries_c_oracle_vs_torch_ref(nope, rope, group, tma):
    """The C oracle and the torch restatement agree bit for bit (codes and
    scales) on every geometry, packed scales where the reference's packed
    tensor holds every head's word."""
    for H, G in ((8, 2), (4, 4)):
        hpg = H // G
        if tma and not _packed_ok(nope, rope, group, hpg):
            continue
        w = W.make_inv_rope_workload(9, H, G, seed=nope + rope + group, max_pos=512, head_dim=nope + rope,
                                     rope_dim=rope)
        kw = dict(tma_aligned_scales=tma, nope_dim=nope, rope_dim=rope, quant_group_size=group)
        c8, cs = oracle.inv_rope_fp8_quant(w.o, w.positions, w.cos_sin_cache, G, hpg, **kw)
        t8, ts = torch_ref.inv_rope_fp8_quant(w.o, w.positions, w.cos_sin_cache, G, hpg, **kw)
        assert torch.equal(c8, t8)
        assert torch.equal(cs.contiguous(), ts)
        d = hpg * (nope + rope)
        assert c8.stride() == (d, 9 * d, 1)


@pytest.mark.parametrize("nope,rope,group", SIBLING_GEOMETRIES)
def test_sibling_geometries_closed_forms(nope, rope, group):
    """Position 0 (cos 1, sin 0) leaves every dim as it is, so each chunk's
    codes are the plain quantisation of o; a chunk holding one non-zero
    value v gets scale |v| / 448 and code 0x7E (+448) or 0xFE there, zeros
    elsewhere."""
    D = nope + rope
    T, H = 3, 2
    g = torch.Generator().manual_seed(D + group)
    o = torch.zeros(T, H, D, dtype=torch.bfloat16)
    where = torch.randint(0, group, (T, H, D // group), generator=g)
    vals = (torch.rand(T, H, D // group, generator=g) * 8 + 0.5) * torch.where(
        torch.rand(T, H, D // group, generator=g) < 0.5, -1.0, 1.0)
    for t in range(T):
        for h in range(H):
            for c in range(D // group):
                o[t, h, c * group + int(where[t, h, c])] = vals[t, h, c]
    pos = torch.zeros(T, dtype=torch.int64)
    cs = W.make_cos_sin_cache(16, rope_dim=rope)
    codes, scales = oracle.inv_rope_fp8_quant(o, pos, cs, 1, H, nope_dim=nope, rope_dim=rope,
                                              quant_group_size=group)
    codes = codes.contiguous().view(T, H, D // group, group)
    scales = scales.contiguous().view(T, H, D // group)
    v = o.float().view(T, H, D // group, group).gather(-1, where[..., None])[..., 0]
    assert torch.equal(scales, v.abs() * torch.tensor(1.0 / 448.0, dtype=torch.float32))
    hit = codes.gather(-1, where[..., None])[..., 0]
    assert torch.equal(hit, torch.where(v > 0, 0x7E, 0xFE).to(torch.uint8))
    assert int(codes.sum()) == int(hit.long().sum())
