"""fused_indexer_q_rope_quant: CPU pins of its oracle and GPU parity.

Reference: src/flaggems_vllm/ops/fused_indexer_q_rope_quant.py:64-410 and
tests/test_fused_indexer_q_rope_quant.py:51-110 (HEAD_DIM 128, ROPE 64, 8 heads,
T in {1, 7, 32}, fp32/bf16 cos-sin, exact codes, scales and weights).
"""
import math
from fractions import Fraction

import pytest
import torch

import oracle
from flaggems_vllm import testing as W
from oracle import torch_ref

DEV = torch.device("cuda:0")
E2M1_GRID = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def _all_bf16_finite():
    bits = torch.arange(-(1 << 15), 1 << 15, dtype=torch.int32).to(torch.int16)
    v = bits.view(torch.bfloat16).float()
    return v[torch.isfinite(v)]


def _case(T, H=8, D=128, cache_dtype=torch.float32, seed=0, max_pos=4096):
    g = torch.Generator().manual_seed(seed)
    q = W.randn_bf16((T, H, D), g)
    pos = torch.randint(0, max_pos, (T,), generator=g, dtype=torch.int64)
    cs = W.make_cos_sin_cache(max_pos).to(cache_dtype)
    w = W.randn_bf16((T, H), g)
    return pos, q, cs, w, D ** -0.5, H ** -0.5


# ------------------------------------------------------------------- CPU ----

def test_e2m1_encoder_vs_threshold_table_and_nearest_even():
    v = _all_bf16_finite()
    xs = torch.cat([v[v.abs() <= 8.0], torch.tensor([-0.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.5])])
    got = oracle.e2m1_codes(xs)
    assert torch.equal(got, torch_ref.e2m1_threshold_codes(xs.clamp(-6.0, 6.0)))
    for x, c in zip(xs[::37].tolist(), got[::37].tolist()):
        a = min(abs(x), 6.0)
        best = min(range(8), key=lambda i: (abs(E2M1_GRID[i] - a), i % 2))  # nearest, ties to even
        assert c & 7 == best and (c >> 3) == (1 if math.copysign(1.0, x) < 0 else 0)


def test_block_exponent_closed_forms_all_bf16():
    """The kernel's integer exponents equal exact ceil(log2(a / d)) for every
    positive bf16 a: d = 448 with floor 1e-4 (FP8) and d = 6 with floor
    6*2^-126 (MXFP4)."""
    v = _all_bf16_finite()
    v = v[v > 0]
    bits = v.view(torch.int32)
    for d, floor_bits, shift_e, mant_cut in ((448, 0x38D1B717, 8, 0x600000), (6, 0x01C00000, 2, 0x400000)):
        floor = torch.tensor([floor_bits], dtype=torch.int32).view(torch.float32).item()
        a_bits = torch.maximum(bits, torch.tensor(floor_bits, dtype=torch.int32))
        closed = (a_bits >> 23) - 127 - shift_e + ((a_bits & 0x7FFFFF) > mant_cut).to(torch.int32)
        for a, k in zip(v.tolist()[::7] + [0.0], closed.tolist()[::7] + [None]):
            r = max(Fraction(a), Fraction(floor)) / d
            exact = math.floor(math.log2(r)) - 2
            while Fraction(2) ** exact < r:
                exact += 1
            if k is not None:
                assert k == exact, (a, d)


@pytest.mark.parametrize("T", [1, 7, 32])
@pytest.mark.parametrize("cache_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("use_fp4", [False, True])
def test_oracle_vs_torch_ref(T, cache_dtype, use_fp4):
    args = _case(T, cache_dtype=cache_dtype)
    (oq, ow), (tq, tw) = (oracle.fused_indexer_q_rope_quant(*args, use_fp4=use_fp4),
                          torch_ref.fused_indexer_q_rope_quant(*args, use_fp4=use_fp4))
    if use_fp4:
        assert torch.equal(oq[0], tq[0]) and torch.equal(oq[1], tq[1])
    else:
        assert torch.equal(oq, tq)
    assert torch.equal(ow, tw)


def test_oracle_extreme_rows():
    """zeros, tiny, huge and mixed-sign rows (amax floors, sign of zero)."""
    pos, q, cs, w, sm, hs = _case(4, H=4)
    q[0] = 0.0
    q[1] = (q[1].float() * 1e-30).to(torch.bfloat16)
    q[2] = (q[2].float() * 1e30).to(torch.bfloat16)
    q[3, 0] = -0.0
    for fp4 in (False, True):
        (oq, ow), (tq, tw) = (oracle.fused_indexer_q_rope_quant(pos, q, cs, w, sm, hs, use_fp4=fp4),
                              torch_ref.fused_indexer_q_rope_quant(pos, q, cs, w, sm, hs, use_fp4=fp4))
        if fp4:
            assert torch.equal(oq[0], tq[0]) and torch.equal(oq[1], tq[1])
        else:
            assert torch.equal(oq, tq)
        assert torch.equal(ow, tw)


# ------------------------------------------------------------------- GPU ----

def _gpu(pos, q, cs, w, sm, hs, use_fp4):
    import flaggems_vllm

    out, wo = flaggems_vllm.fused_indexer_q_rope_quant(pos.to(DEV), q.to(DEV), cs.to(DEV), w.to(DEV),
                                                       sm, hs, use_fp4=use_fp4)
    torch.cuda.synchronize()
    if use_fp4:
        return (out[0].cpu(), out[1].cpu()), wo.cpu()
    return out.cpu().view(torch.uint8), wo.cpu()


def _check(args, use_fp4):
    (gq, gw) = _gpu(*args, use_fp4)
    (oq, ow) = oracle.fused_indexer_q_rope_quant(*args, use_fp4=use_fp4)
    if use_fp4:
        T, H = oq[1].shape[:2]
        assert torch.equal(gq[0], oq[0])
        assert torch.equal(gq[1], oq[1].contiguous().view(torch.int32).reshape(T, H, -1).squeeze(-1))
    else:
        assert torch.equal(gq, oq)
    assert gw.dtype == torch.float32 and torch.equal(gw, ow)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 7, 32, 4096])
@pytest.mark.parametrize("cache_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("use_fp4", [False, True])
def test_gpu_matches_oracle(T, cache_dtype, use_fp4):
    print(f"\n[case] indexer T={T} cs={cache_dtype} fp4={use_fp4}", flush=True)
    H = 64 if T == 4096 else 8
    _check(_case(T, H=H, cache_dtype=cache_dtype, seed=T), use_fp4)


@pytest.mark.gpu
@pytest.mark.parametrize("D", [256, 512])
@pytest.mark.parametrize("use_fp4", [False, True])
def test_gpu_wider_heads(D, use_fp4):
    print(f"\n[case] indexer D={D} fp4={use_fp4}", flush=True)
    _check(_case(16, H=4, D=D, seed=5), use_fp4)


def _exhaustive_rows(limit):
    """Rows of 128 whose every 32-element block holds `limit` (so the block
    and row scales are 1) followed by successive bf16 values |v| <= limit."""
    v = _all_bf16_finite()
    v = v[v.abs() <= limit]
    per = 31
    nblk = (v.numel() + per - 1) // per
    vals = torch.zeros(nblk * per)
    vals[:v.numel()] = v
    blocks = torch.cat([torch.full((nblk, 1), limit), vals.view(nblk, per)], dim=1)
    nrow = (nblk + 3) // 4
    rows = torch.zeros(nrow * 4, 32)
    rows[:nblk] = blocks
    rows[nblk:, 0] = limit
    return rows.view(nrow, 1, 128).to(torch.bfloat16)


def _exhaustive_rows_at(limit, k):
    """Like _exhaustive_rows at block exponent k: every bf16 value with
    |v| <= limit * 2^k, 31 per 32-element block after one entry of exactly
    limit * 2^k, so the row (FP8) or block (MXFP4) exponent is k."""
    v = _all_bf16_finite()
    top = limit * 2.0 ** k
    v = v[v.abs() <= top]
    per = 31
    nblk = (v.numel() + per - 1) // per
    vals = torch.zeros(nblk * per, dtype=torch.float64)
    vals[:v.numel()] = v.double()
    blocks = torch.cat([torch.full((nblk, 1), top, dtype=torch.float64), vals.view(nblk, per)], dim=1)
    nrow = (nblk + 3) // 4
    rows = torch.zeros(nrow * 4, 32, dtype=torch.float64)
    rows[:nblk] = blocks
    rows[nblk:, 0] = top
    return rows.view(nrow, 1, 128).to(torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("use_fp4,limit,k", [(False, 448.0, 0), (True, 6.0, 0),
                                             (False, 448.0, -22), (False, 448.0, -7), (False, 448.0, 9),
                                             (False, 448.0, 100), (True, 6.0, -124), (True, 6.0, -60),
                                             (True, 6.0, 13), (True, 6.0, 125)])
def test_gpu_converter_exhaustive(use_fp4, limit, k):
    """Every bf16 value within range of block exponent k goes through the
    hardware's scaled e4m3 / E2M1 conversion (position 0: cos 1, sin 0, so
    RoPE is the identity); codes must equal the oracle's software encoders of
    x * 2^-k, at the ends of the exponent ranges the quantisers produce
    (FP8 -22..120, MXFP4 -124..125) and between."""
    print(f"\n[case] indexer converter exhaustive fp4={use_fp4} k={k}", flush=True)
    q = _exhaustive_rows(limit) if k == 0 else _exhaustive_rows_at(limit, k)
    T = q.shape[0]
    pos = torch.zeros(T, dtype=torch.int64)
    cs = W.make_cos_sin_cache(16)
    w = torch.ones(T, 1, dtype=torch.bfloat16)
    _check((pos, q, cs, w, 1.0, 1.0), use_fp4)


@pytest.mark.gpu
@pytest.mark.parametrize("D,H", [(128, 64), (128, 128), (256, 32), (512, 16)])
@pytest.mark.parametrize("use_fp4", [False, True])
@pytest.mark.parametrize("w_f32", [False, True])
def test_gpu_one_token_blocks(D, H, use_fp4, w_f32):
    """Head counts that fill whole blocks with one token's rows, so the kernel
    with per-block token and 32-bit row offsets runs (including two blocks per
    token at H=128), on a strided q view (head stride D + 64) with bf16 or fp32
    weights."""
    import flaggems_vllm

    print(f"\n[case] indexer one-token D={D} H={H} fp4={use_fp4} w_f32={w_f32}", flush=True)
    T = 37
    pos, q, cs, w, sm, hs = _case(T, H=H, D=D, seed=11)
    if w_f32:
        w = (w.float() * 1.0009765625).contiguous()  # not representable in bf16
    wide = torch.zeros(T, H, D + 64, dtype=torch.bfloat16, device=DEV)
    wide[..., :D] = q.to(DEV)
    qv = wide[..., :D]
    assert qv.stride() == (H * (D + 64), D + 64, 1)
    out, wo = flaggems_vllm.fused_indexer_q_rope_quant(pos.to(DEV), qv, cs.to(DEV), w.to(DEV), sm, hs,
                                                       use_fp4=use_fp4)
    torch.cuda.synchronize()
    (oq, ow) = oracle.fused_indexer_q_rope_quant(pos, q, cs, w, sm, hs, use_fp4=use_fp4)
    if use_fp4:
        assert torch.equal(out[0].cpu(), oq[0])
        assert torch.equal(out[1].cpu(), oq[1].contiguous().view(torch.int32).reshape(T, H, -1).squeeze(-1))
    else:
        assert torch.equal(out.cpu().view(torch.uint8), oq)
    assert torch.equal(wo.cpu(), ow)
