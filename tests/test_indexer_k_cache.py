"""Sparse-indexer key cache: indexer_k_quant_and_cache and
cp_gather_indexer_k_quant_cache.

Reference ops: src/flaggems_vllm/ops/indexer_k_quant_and_cache.py:44-132,
src/flaggems_vllm/ops/cp_gather_indexer_k_quant_cache.py:23-176.  Reference
tests: tests/test_indexer_k_quant_and_cache.py:177-222 (three shapes, UE8M0,
whole-cache equality against ``torch_indexer`` :99-142) and
tests/test_cp_gather_indexer_k_quant_cache.py:168-249 (two shapes, sentinel
rows past the last request, equality against ``torch_gather`` :83-114).

CPU: the C oracle against closed forms (known codes and scales at fixed
amax, the cache layout by byte offset), against the torch restatement of the
reference's oracles on the reference's shapes and on whole-exponent sweeps,
the UE8M0 closed form the kernel uses against exp2(ceil(log2())) over every
bf16 and fp16 amax, and the wrappers' and C ABI's argument checks.  GPU: the
kernels' bytes against the C oracle, bit for bit, on the same cases, on the
sweeps, on edge cases and at the reference benchmark's largest shapes.
"""
import ctypes
import inspect
import struct

import pytest
import torch

import flaggems_vllm
import oracle
from flaggems_vllm import _native
from flaggems_vllm import testing as W
from oracle import torch_ref

from .test_quant_sweep import _groups, _kv_bits_for_exponent

DEV = torch.device("cuda:0")
QB = W.INDEXER_QUANT_BLOCK
FP8 = torch.float8_e4m3fn

# dtype, num_tokens, num_blocks, block_size, head_dim (reference test :177-185)
REF_INSERT = [(torch.bfloat16, 19, 4, 16, 128), (torch.float16, 23, 5, 16, 512),
              (torch.bfloat16, 17, 4, 64, 512)]
# seq_lens, block_size, head_dim, extra_tokens (reference test :168-175)
REF_GATHER = [([13, 7, 16], 8, 128, 0), ([17, 1, 33, 9], 16, 512, 5)]
SENTINEL = 0x7B


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _insert_oracle(k, cache, slots, fmt):
    out = cache.clone()
    oracle.indexer_k_quant_and_cache(k, out, slots, QB, fmt)
    return out


def _gather_oracle(cache, k_fp8, k_scale, bt, cu):
    k2, s2 = k_fp8.clone(), k_scale.clone()
    oracle.cp_gather_indexer_k_quant_cache(cache, k2, s2, bt, cu)
    return k2, s2


def _first_diff(got, want, what):
    g, w = got.reshape(-1), want.reshape(-1)
    if torch.equal(g, w):
        return
    d = torch.nonzero(g != w).flatten()
    raise AssertionError(f"{what}: {d.numel()} bytes differ; first at {int(d[0])}: "
                         f"gpu {int(g[d[0]])} oracle {int(w[d[0]])}")


def _sweep_keys(dtype, ue8m0):
    """[n, 512] keys whose 128-element blocks cover every scale the quantiser
    can produce for dtype: UE8M0 exponents -22..120 (bf16) / -22..8 (fp16),
    each at its largest and smallest amax; fp32 scales at four mantissas per
    binade (fp16: every third of a binade, plus 448 * 2^k and the value above
    it).  Each block holds its amax and the magnitudes within 2^-22 of it
    (every value that can give a nonzero code), both signs."""
    if dtype == torch.bfloat16:
        groups = []
        if ue8m0:
            for e in range(-22, 121):
                top, low = _kv_bits_for_exponent(e)
                groups.append(_groups(top, QB - 1, floor_bits=max(1, top - 22 * 128)))
                groups.append(_groups(low, QB - 1, floor_bits=max(1, low - 22 * 128)))
        else:
            for e in range(-40, 128):
                for mant in (0x00, 0x30, 0x60, 0x7F):
                    bits = ((e + 127) << 7) | mant
                    if bits <= 0x7F7F:
                        groups.append(_groups(bits, QB - 1, floor_bits=max(1, bits - 22 * 128)))
        for amax in (0.0, 5e-5, 9.98e-5, 1.0e-4, 1.0014e-4):
            bits = int(torch.tensor(amax).to(torch.bfloat16).view(torch.int16))
            groups.append(_groups(max(bits, 1), QB - 1) if amax else torch.zeros(2, QB))
        g = torch.cat(groups)
    else:
        mags = torch.arange(1, 0x7C00, dtype=torch.int32).to(torch.int16).view(torch.float16).float()
        blocks = []
        tops = list(range(0x0400, 0x7C00, 0x0155)) + [0x7BFF, 0x3C00, 0x0001, 0x03FF]
        # 448 * 2^k exactly (1.75 * 2^(k + 8): the largest amax of exponent k)
        # and the next value above it (the smallest amax of exponent k + 1)
        tops += [(e << 10) | 0x300 for e in range(1, 31)] + [((e << 10) | 0x300) + 1 for e in range(1, 30)]
        for top in tops:
            amax = float(mags[top - 1])
            window = mags[(mags >= amax * 2.0 ** -22) & (mags <= amax)]
            vals = torch.cat([window, -window])
            n = (vals.numel() + QB - 2) // (QB - 1)
            body = torch.zeros(n * (QB - 1))
            body[:vals.numel()] = vals
            head = torch.full((n, 1), amax)
            head[1::2] = -amax
            blocks.append(torch.cat([head, body.view(n, QB - 1)], dim=1))
        g = torch.cat(blocks)
    rows = (g.shape[0] + 3) // 4
    out = torch.zeros(rows * 4, QB)
    out[:g.shape[0]] = g
    return out.view(rows, 4 * QB).to(dtype)


def _sweep_case(dtype, ue8m0, seed=31):
    k = _sweep_keys(dtype, ue8m0)
    T = k.shape[0]
    gen = torch.Generator().manual_seed(seed)
    bs = 64
    nblk = (T + bs - 1) // bs + 2
    slots = torch.randperm(nblk * bs, generator=gen)[:T].to(torch.int64)
    slots[::101] = -1
    return k, W.make_indexer_k_cache(nblk, bs, 512, gen), slots


# ------------------------------------------------------------------- CPU ----

def test_signatures_match_reference():
    p = inspect.signature(flaggems_vllm.indexer_k_quant_and_cache).parameters
    assert list(p) == ["k", "kv_cache", "slot_mapping", "quant_block_size", "scale_fmt"]
    p = inspect.signature(flaggems_vllm.cp_gather_indexer_k_quant_cache).parameters
    assert list(p) == ["k_cache", "k_fp8", "k_fp8_scale", "block_table", "cu_seqlen"]
    assert flaggems_vllm.ops.indexer_k_quant_and_cache is flaggems_vllm.indexer_k_quant_and_cache


@pytest.mark.parametrize("fmt", ["ue8m0", None])
def test_oracle_known_answers(fmt):
    """Fixed keys with hand-derived results: a block of +-448 gives scale 1
    and codes 0x7E / 0xFE; a block of 1.0 with one 3.0 gives UE8M0 scale
    2^-7 (3/448 = 2^-7.22) and codes e4m3(128) = 0x70, e4m3(384) = 0x7C, or
    fp32 scale fl(3/448) with codes e4m3(149.33) = e4m3(144) = 0x71 and
    e4m3(448) = 0x7E;
    a zero block gives 2^-22 (UE8M0: 1e-4/448 = 2^-22.09) or fl(1e-4/448)
    and code 0.  Slot 1 * 16 + 3 puts the token at block 1, row 3: codes at
    byte 3 * 256, scales at 16 * 256 + (3 * 2 + j) * 4."""
    k = torch.zeros(1, 256, dtype=torch.bfloat16)
    k[0, :128] = 448.0
    k[0, 1:128:2] = -448.0
    k[0, 128:] = 0.0
    k2 = torch.ones(1, 256, dtype=torch.bfloat16)
    k2[0, 5] = 3.0
    k2[0, 128:] = 0.0
    cache = torch.zeros(3, 16, 256 + 8, dtype=torch.uint8)
    a = _insert_oracle(k, cache, torch.tensor([16 + 3]), fmt)
    b = _insert_oracle(k2, cache, torch.tensor([16 + 3]), fmt)
    blk_a, blk_b = a[1].view(-1), b[1].view(-1)
    assert int(a[0].sum()) == 0 and int(a[2].sum()) == 0

    def scale(blk, j):
        return struct.unpack("<f", bytes(blk[16 * 256 + (3 * 2 + j) * 4:][:4].tolist()))[0]

    codes_a = blk_a[3 * 256:3 * 256 + 256]
    assert codes_a[:128:2].eq(0x7E).all() and codes_a[1:128:2].eq(0xFE).all()
    assert codes_a[128:].eq(0).all()
    assert scale(blk_a, 0) == 1.0
    codes_b = blk_b[3 * 256:3 * 256 + 256]
    zero_scale = 2.0 ** -22 if fmt == "ue8m0" else float(torch.tensor(1e-4) / 448.0)
    assert scale(blk_b, 1) == zero_scale and codes_b[128:].eq(0).all()
    if fmt == "ue8m0":
        assert scale(blk_b, 0) == 2.0 ** -7
        assert int(codes_b[5]) == 0x7C and int(codes_b[0]) == 0x70
    else:
        assert scale(blk_b, 0) == float(torch.tensor(3.0) / 448.0)
        assert int(codes_b[5]) == 0x7E and int(codes_b[0]) == 0x71
    # only the one row's codes and scales changed
    changed = torch.nonzero(b.view(-1) != cache.view(-1)).flatten()
    base = 1 * 16 * 264
    assert bool(((changed >= base + 3 * 256) & (changed < base + 4 * 256)
                 | (changed >= base + 16 * 256 + 24) & (changed < base + 16 * 256 + 32)).all())


@pytest.mark.parametrize("fmt", ["ue8m0", None])
@pytest.mark.parametrize("case", REF_INSERT)
def test_insert_oracle_matches_reference_formulation(case, fmt):
    dtype, T, nblk, bs, hd = case
    k, cache, slots = W.make_indexer_k_insert(T, nblk, bs, hd, dtype, seed=0)
    a = _insert_oracle(k, cache, slots, fmt)
    b = cache.clone()
    torch_ref.indexer_k_quant_and_cache(k, b, slots, QB, fmt)
    assert torch.equal(a, b)
    assert not torch.equal(a, cache)


@pytest.mark.parametrize("dtype,ue8m0", [(torch.bfloat16, True), (torch.bfloat16, False),
                                         (torch.float16, True), (torch.float16, False)])
def test_insert_sweep_oracles_agree(dtype, ue8m0):
    """The C oracle equals the reference's torch formulation over the whole
    exponent sweep; all 254 finite codes occur."""
    fmt = "ue8m0" if ue8m0 else None
    k, cache, slots = _sweep_case(dtype, ue8m0)
    a = _insert_oracle(k, cache, slots, fmt)
    b = cache.clone()
    torch_ref.indexer_k_quant_and_cache(k, b, slots, QB, fmt)
    assert torch.equal(a, b)
    keep = slots >= 0
    blk, row = slots[keep] // 64, slots[keep] % 64
    codes = a.view(a.shape[0], -1)[blk[:, None], row[:, None] * 512 + torch.arange(512)]
    assert set(codes.flatten().tolist()) == set(range(256)) - {0x7F, 0xFF}
    if ue8m0:
        sc = a.view(a.shape[0], -1)[:, 64 * 512:].contiguous().view(torch.float32)
        sc = sc[blk[:, None], row[:, None] * 4 + torch.arange(4)]
        exps = set(torch.log2(sc).flatten().tolist())
        hi = 120 if dtype == torch.bfloat16 else 8
        assert set(range(-22, hi + 1)) <= exps


def _ue8m0_closed_form(scale: torch.Tensor) -> torch.Tensor:
    bits = scale.view(torch.int32)
    e = (bits >> 23) - 127 + ((bits & 0x7FFFFF) != 0).to(torch.int32)
    return ((e + 127) << 23).view(torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_ue8m0_closed_form_every_amax(dtype):
    """The kernel's UE8M0 scale (binary32 exponent, plus one when any
    mantissa bit is set) equals exp2(ceil(log2(max(amax, 1e-4) / 448))) for
    every finite amax of the input type, zero included."""
    lim = 0x7F80 if dtype == torch.bfloat16 else 0x7C00
    amax = torch.arange(0, lim, dtype=torch.int32).to(torch.int16).view(dtype).float()
    scale = torch.maximum(amax, torch.tensor(1e-4)) / 448.0
    want = torch.exp2(torch.ceil(torch.log2(scale)))
    assert torch.equal(_ue8m0_closed_form(scale).view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("case", REF_GATHER)
def test_gather_oracle_matches_reference_formulation(case):
    lens, bs, hd, extra = case
    cache, kf, ks, bt, cu = W.make_indexer_k_gather(lens, bs, hd, extra)
    k1, s1 = _gather_oracle(cache, kf, ks, bt, cu)
    k2, s2 = kf.clone(), ks.clone()
    torch_ref.cp_gather_indexer_k_quant_cache(cache, k2, s2, bt, cu)
    assert torch.equal(k1.view(torch.uint8), k2.view(torch.uint8)) and torch.equal(s1, s2)
    n = int(cu[-1])
    assert bool((k1.view(torch.uint8)[n:] == SENTINEL).all()) and bool((s1[n:] == SENTINEL).all())
    assert not bool((k1.view(torch.uint8)[:n] == SENTINEL).all())


def test_gather_oracle_round_trip():
    """Insert tokens of three requests at the slots their block tables give,
    then gather: row t holds exactly the bytes the insert wrote for token t
    (checked against the insert's output read back by slot)."""
    gen = torch.Generator().manual_seed(3)
    lens, bs, hd = [40, 0, 77, 5], 16, 256
    per = [(n + bs - 1) // bs for n in lens]
    nblk = sum(per) + 3
    perm = torch.randperm(nblk, generator=gen).to(torch.int32)
    bt = torch.full((len(lens), max(per)), -1, dtype=torch.int32)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    slots, used = [], 0
    for b, n in enumerate(lens):
        bt[b, :per[b]] = perm[used:used + per[b]]
        used += per[b]
        cu[b + 1] = cu[b] + n
        slots += [int(bt[b, p // bs]) * bs + p % bs for p in range(n)]
    T = int(cu[-1])
    k = torch.randn(T, hd, generator=gen).to(torch.bfloat16)
    cache = _insert_oracle(k, W.make_indexer_k_cache(nblk, bs, hd, gen), torch.tensor(slots), "ue8m0")
    kf = torch.zeros(T, hd, dtype=torch.uint8)
    ks = torch.zeros(T, 8, dtype=torch.uint8)
    g_k, g_s = _gather_oracle(cache, kf, ks, bt, cu)
    flat = cache.view(nblk, -1)
    for t, s in enumerate(slots):
        blk, row = s // bs, s % bs
        assert torch.equal(g_k[t], flat[blk, row * hd:(row + 1) * hd])
        assert torch.equal(g_s[t], flat[blk, bs * hd + row * 8:bs * hd + row * 8 + 8])
    # and the codes decode back to within half an e4m3 step of k / scale
    sc = g_s.view(torch.float32)
    dec = g_k.view(FP8).float().view(T, 2, 128) * sc[:, :, None]
    err = (dec - k.float().view(T, 2, 128)).abs()
    assert bool((err <= k.float().view(T, 2, 128).abs() * 2.0 ** -4 + sc[:, :, None] * 2.0 ** -9).all())


@pytest.mark.parametrize("hd,qbs", [(192, 128), (128, 96)])
def test_wrappers_raise_value_error_like_reference(hd, qbs):
    k = torch.zeros(4, hd, dtype=torch.bfloat16)
    cache = torch.zeros(2, 16, hd + 8, dtype=torch.uint8)
    with pytest.raises(ValueError):
        flaggems_vllm.indexer_k_quant_and_cache(k, cache, torch.zeros(4, dtype=torch.int64), qbs, "ue8m0")
    kf = torch.zeros(4, hd, dtype=torch.uint8)
    ks = torch.zeros(4, hd * 4 // qbs, dtype=torch.uint8)
    with pytest.raises(ValueError):
        flaggems_vllm.cp_gather_indexer_k_quant_cache(cache, kf, ks, torch.zeros(1, 4, dtype=torch.int32),
                                                      torch.tensor([0, 4], dtype=torch.int32))


def test_wrappers_refuse_cpu_tensors():
    k, cache, slots = W.make_indexer_k_insert(4, 2, 16, 128)
    with pytest.raises(AssertionError):
        flaggems_vllm.indexer_k_quant_and_cache(k, cache, slots, 128, "ue8m0")


def _call_insert(**kw):
    a = dict(k=256, kst=128, fp16=0, T=4, hd=128, qbs=128, cache=256, cst=16 * 132, nblk=4, bs=16,
             slots=256, ue=1)
    a.update(kw)
    return _native.lib().fgv_indexer_k_quant_and_cache(
        a["k"], a["kst"], a["fp16"], a["T"], a["hd"], a["qbs"], a["cache"], a["cst"], a["nblk"], a["bs"],
        a["slots"], a["ue"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(qbs=64), -2), (dict(hd=192), -2), (dict(hd=4096), -2), (dict(T=-1), -2), (dict(bs=0), -2),
    (dict(k=None), -1), (dict(slots=None), -1), (dict(k=264), -3), (dict(kst=132), -3),
    (dict(cache=258), -3), (dict(cst=16 * 132 - 8), -4), (dict(cst=16 * 132 + 2), -3),
])
def test_insert_c_abi_rejects_bad_arguments(kw, code):
    assert _call_insert(**kw) == code
    assert _native.lib().fgv_last_error()


def test_insert_c_abi_empty_call_is_a_no_op():
    assert _call_insert(T=0, k=None, slots=None) == 0


def _call_gather(**kw):
    a = dict(cache=256, cst=16 * 132, nblk=4, bs=16, hd=128, qbs=128, ko=256, kst=128, so=256, sst=4,
             bt=256, btst=4, maxb=4, cu=256, B=2, T=8)
    a.update(kw)
    return _native.lib().fgv_cp_gather_indexer_k_quant_cache(
        a["cache"], a["cst"], a["nblk"], a["bs"], a["hd"], a["qbs"], a["ko"], a["kst"], a["so"], a["sst"],
        a["bt"], a["btst"], a["maxb"], a["cu"], a["B"], a["T"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(qbs=256), -2), (dict(hd=100), -2), (dict(B=-1), -2), (dict(bs=0), -2), (dict(cu=None), -1),
    (dict(ko=None), -1), (dict(cst=100), -4), (dict(ko=258), -3), (dict(kst=130), -3), (dict(sst=6), -3),
    (dict(so=258), -3),
])
def test_gather_c_abi_rejects_bad_arguments(kw, code):
    assert _call_gather(**kw) == code
    assert _native.lib().fgv_last_error()


def test_gather_c_abi_empty_call_is_a_no_op():
    assert _call_gather(T=0, cache=None) == 0
    assert _call_gather(B=0, bt=None) == 0


# ------------------------------------------------------------------- GPU ----

@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["ue8m0", None])
@pytest.mark.parametrize("case", REF_INSERT)
def test_gpu_insert_reference_cases(case, fmt):
    """The reference test's shapes: the whole cache bit for bit."""
    dtype, T, nblk, bs, hd = case
    _say(f"indexer k insert {dtype} T={T} blocks={nblk} bs={bs} hd={hd} fmt={fmt}")
    k, cache, slots = W.make_indexer_k_insert(T, nblk, bs, hd, dtype, seed=0)
    want = _insert_oracle(k, cache, slots, fmt)
    g = cache.to(DEV)
    flaggems_vllm.indexer_k_quant_and_cache(k.to(DEV), g, slots.to(DEV), QB, fmt)
    torch.cuda.synchronize()
    _first_diff(g.cpu(), want, "cache")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,ue8m0", [(torch.bfloat16, True), (torch.bfloat16, False),
                                         (torch.float16, True), (torch.float16, False)])
def test_gpu_insert_every_exponent(dtype, ue8m0):
    fmt = "ue8m0" if ue8m0 else None
    k, cache, slots = _sweep_case(dtype, ue8m0)
    _say(f"indexer k insert sweep {dtype} fmt={fmt} T={k.shape[0]}")
    want = _insert_oracle(k, cache, slots, fmt)
    g = cache.to(DEV)
    flaggems_vllm.indexer_k_quant_and_cache(k.to(DEV), g, slots.to(DEV), QB, fmt)
    torch.cuda.synchronize()
    _first_diff(g.cpu(), want, "cache")


@pytest.mark.gpu
def test_gpu_insert_edge_cases():
    """A strided key view with more rows than slots, slots past the cache and
    -1 (skipped), head_dim 2048 (the largest), an all-padding call and an
    empty call (no-ops)."""
    _say("indexer k insert edge cases")
    gen = torch.Generator().manual_seed(9)
    wide = torch.randn(40, 640, generator=gen).to(torch.bfloat16)
    k = wide[:, 64:576]  # row stride 640
    cache = W.make_indexer_k_cache(3, 16, 512, gen)
    slots = torch.randperm(48, generator=gen)[:30].to(torch.int64)
    slots[3], slots[7], slots[11] = -1, 48, 1000  # padding and two past the cache's 3 blocks
    want = cache.clone()
    ok = (slots >= 0) & (slots < 48)
    oracle.indexer_k_quant_and_cache(k[:30][ok], want, slots[ok], QB, "ue8m0")
    g = cache.to(DEV)
    flaggems_vllm.indexer_k_quant_and_cache(wide.to(DEV)[:, 64:576], g, slots.to(DEV), QB, "ue8m0")
    torch.cuda.synchronize()
    _first_diff(g.cpu(), want, "strided / out-of-range cache")

    k, cache, slots = W.make_indexer_k_insert(37, 5, 16, 2048, torch.bfloat16, seed=4)
    want = _insert_oracle(k, cache, slots, "ue8m0")
    g = cache.to(DEV)
    flaggems_vllm.indexer_k_quant_and_cache(k.to(DEV), g, slots.to(DEV), QB, "ue8m0")
    torch.cuda.synchronize()
    _first_diff(g.cpu(), want, "head_dim 2048")

    before = g.clone()
    flaggems_vllm.indexer_k_quant_and_cache(k.to(DEV), g, torch.full((37,), -1, dtype=torch.int64, device=DEV),
                                            QB, "ue8m0")
    flaggems_vllm.indexer_k_quant_and_cache(k.to(DEV), g, torch.empty(0, dtype=torch.int64, device=DEV),
                                            QB, "ue8m0")
    torch.cuda.synchronize()
    assert torch.equal(g, before)


@pytest.mark.gpu
@pytest.mark.parametrize("case", REF_GATHER)
def test_gpu_gather_reference_cases(case):
    lens, bs, hd, extra = case
    _say(f"indexer k gather lens={lens} bs={bs} hd={hd} extra={extra}")
    cache, kf, ks, bt, cu = W.make_indexer_k_gather(lens, bs, hd, extra)
    wk, ws = _gather_oracle(cache, kf, ks, bt, cu)
    gk, gs = kf.to(DEV), ks.to(DEV)
    flaggems_vllm.cp_gather_indexer_k_quant_cache(cache.to(DEV), gk, gs, bt.to(DEV), cu.to(DEV))
    torch.cuda.synchronize()
    _first_diff(gk.cpu().view(torch.uint8), wk.view(torch.uint8), "k_fp8")
    _first_diff(gs.cpu(), ws, "k_fp8_scale")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(6))
def test_gpu_gather_fuzz(seed):
    """Random ragged batches (1..300 requests, empty ones included; more than
    16 takes the reference's binary-search path), random block tables with
    some -1 and out-of-range entries (rows left as they were), a float32
    scale view and row-strided outputs."""
    gen = torch.Generator().manual_seed(100 + seed)
    B = [1, 5, 16, 17, 64, 300][seed]
    bs = [16, 64, 8, 16, 32, 64][seed]
    hd = [128, 512, 256, 128, 1024, 128][seed]
    lens = torch.randint(0, 90, (B,), generator=gen)
    lens[torch.randint(0, B, (max(1, B // 5),), generator=gen)] = 0
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    maxb = (int(lens.max()) + bs - 1) // bs + 1
    nblk = max(4, B * maxb // 2)
    bt = torch.randint(0, nblk, (B, maxb), generator=gen, dtype=torch.int32)
    bad = torch.rand(B, maxb, generator=gen) < 0.05
    bt[bad] = torch.where(torch.rand(int(bad.sum()), generator=gen) < 0.5, -1, nblk + 3).to(torch.int32)
    cache = W.make_indexer_k_cache(nblk, bs, hd, gen)
    T = int(cu[-1]) + 7
    kw = torch.full((T, hd + 64), SENTINEL, dtype=torch.uint8)
    sw = torch.full((T, hd // 128 + 2), float(SENTINEL), dtype=torch.float32)
    kf, ks = kw[:, :hd], sw[:, :hd // 128]
    _say(f"indexer k gather fuzz seed={seed} B={B} bs={bs} hd={hd} T={T}")
    wk, ws = kw.clone(), sw.clone()
    oracle.cp_gather_indexer_k_quant_cache(cache, wk[:, :hd], ws[:, :hd // 128], bt, cu)
    gkw, gsw = kw.to(DEV), sw.to(DEV)
    flaggems_vllm.cp_gather_indexer_k_quant_cache(cache.to(DEV), gkw[:, :hd], gsw[:, :hd // 128], bt.to(DEV),
                                                  cu.to(DEV))
    torch.cuda.synchronize()
    _first_diff(gkw.cpu(), wk, "k_fp8 (with the untouched stride padding)")
    _first_diff(gsw.cpu().view(torch.int32), ws.view(torch.int32), "scales")


def _gather_case(lens, bs, hd, gen, nblk=None):
    """Random block tables (distinct blocks per request) for the given lengths."""
    B = len(lens)
    cu = torch.zeros(B + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int64), 0).to(torch.int32)
    maxb = max(1, (max(lens) + bs - 1) // bs)
    nblk = nblk or max(4, B * maxb)
    bt = torch.randint(0, nblk, (B, maxb), generator=gen, dtype=torch.int32)
    return W.make_indexer_k_cache(nblk, bs, hd, gen), bt, cu


def _run_gather_pair(cache, bt, cu, T, hd, k_offset=0):
    """GPU gather into sentinel-filled outputs (k_fp8 starting k_offset bytes
    into its buffer) against the oracle on the same outputs."""
    nqb = hd // 128
    kbuf = torch.full((T * hd + k_offset,), SENTINEL, dtype=torch.uint8)
    ks = torch.full((T, 4 * nqb), SENTINEL, dtype=torch.uint8)
    wk, ws = kbuf.clone(), ks.clone()
    oracle.cp_gather_indexer_k_quant_cache(cache, wk[k_offset:].view(T, hd), ws, bt, cu)
    gk, gs = kbuf.to(DEV), ks.to(DEV)
    flaggems_vllm.cp_gather_indexer_k_quant_cache(cache.to(DEV), gk[k_offset:].view(T, hd), gs, bt.to(DEV),
                                                  cu.to(DEV))
    torch.cuda.synchronize()
    _first_diff(gk.cpu(), wk, "k_fp8 buffer")
    _first_diff(gs.cpu(), ws, "k_fp8_scale")


@pytest.mark.gpu
@pytest.mark.parametrize("hd,k_offset", [(384, 0), (2048, 0), (512, 8), (256, 8), (1024, 0)])
def test_gpu_gather_chunk_variants(hd, k_offset):
    """Every chunk layout of the gather: 16-byte chunks at head_dim 256-2048,
    8-byte chunks where head_dim is not a power-of-two multiple of 256 (384)
    or where k_fp8 is only 8-byte aligned."""
    gen = torch.Generator().manual_seed(hd + k_offset)
    lens = torch.randint(1, 70, (9,), generator=gen).tolist()
    cache, bt, cu = _gather_case(lens, 16, hd, gen)
    T = int(cu[-1]) + 3
    _say(f"indexer k gather chunks hd={hd} k_offset={k_offset} T={T}")
    _run_gather_pair(cache, bt, cu, T, hd, k_offset)


@pytest.mark.gpu
@pytest.mark.parametrize("bs", [1, 2, 3, 6])
def test_gpu_odd_block_sizes(bs):
    """Block sizes whose packed blocks are only 4- or 8-byte aligned (132 *
    block_size bytes at head_dim 128): the insert's narrower code stores and
    the gather's narrower chunks, bit for bit against the oracle."""
    for hd in (128, 512):
        _say(f"indexer k odd block size bs={bs} hd={hd}")
        T = 29
        k, cache, slots = W.make_indexer_k_insert(T, (T + bs - 1) // bs + 2, bs, hd, torch.bfloat16, seed=bs)
        want = _insert_oracle(k, cache, slots, "ue8m0")
        g = cache.to(DEV)
        flaggems_vllm.indexer_k_quant_and_cache(k.to(DEV), g, slots.to(DEV), QB, "ue8m0")
        torch.cuda.synchronize()
        _first_diff(g.cpu(), want, "cache")
        gen = torch.Generator().manual_seed(bs)
        lens = torch.randint(0, 20, (5,), generator=gen).tolist()
        gcache, bt, cu = _gather_case(lens, bs, hd, gen)
        _run_gather_pair(gcache, bt, cu, int(cu[-1]) + 2, hd)


@pytest.mark.gpu
@pytest.mark.parametrize("B", [70, 5000])
def test_gpu_gather_many_short_requests(B):
    """Thousands of requests of 0-2 tokens: more than 64 request starts inside
    one wave's tokens (the per-token fallback search) and a request search
    over more than 4096 boundaries (three ballot levels)."""
    gen = torch.Generator().manual_seed(B)
    lens = torch.tensor([0, 0, 0, 1, 2])[torch.randint(0, 5, (B,), generator=gen)].tolist()
    lens[0] = 0
    cache, bt, cu = _gather_case(lens, 16, 128, gen, nblk=64)
    T = int(cu[-1]) + 5
    _say(f"indexer k gather many requests B={B} T={T}")
    _run_gather_pair(cache, bt, cu, T, 128)


@pytest.mark.gpu
@pytest.mark.parametrize("bench_case", range(4))
def test_gpu_reference_benchmark_shapes(bench_case):
    """The reference benchmarks' shapes: every insert case in both input
    types and every gather case, bit for bit against the oracle; the largest
    gather (32 x 1024 tokens, head_dim 512) is the bench workload."""
    T, nblk, bs, hd = W.INDEXER_K_INSERT_CASES[bench_case]
    for dtype in (torch.float16, torch.bfloat16):
        _say(f"indexer k insert bench shape T={T} blocks={nblk} bs={bs} hd={hd} {dtype}")
        k, cache, slots = W.make_indexer_k_insert(T, nblk, bs, hd, dtype, seed=bench_case)
        want = _insert_oracle(k, cache, slots, "ue8m0")
        g = cache.to(DEV)
        flaggems_vllm.indexer_k_quant_and_cache(k.to(DEV), g, slots.to(DEV), QB, "ue8m0")
        torch.cuda.synchronize()
        _first_diff(g.cpu(), want, "cache")
    B, L, bs, hd = W.INDEXER_K_GATHER_CASES[bench_case]
    _say(f"indexer k gather bench shape B={B} L={L} bs={bs} hd={hd}")
    cache, kf, ks, bt, cu = W.make_indexer_k_gather([L] * B, bs, hd, seed=bench_case)
    wk, ws = _gather_oracle(cache, kf, ks, bt, cu)
    gk, gs = kf.to(DEV), ks.to(DEV)
    flaggems_vllm.cp_gather_indexer_k_quant_cache(cache.to(DEV), gk, gs, bt.to(DEV), cu.to(DEV))
    torch.cuda.synchronize()
    _first_diff(gk.cpu().view(torch.uint8), wk.view(torch.uint8), "k_fp8")
    _first_diff(gs.cpu(), ws, "k_fp8_scale")


@pytest.mark.gpu
def test_gpu_round_trip_large():
    """65536 tokens of 4 requests inserted at their block tables' slots and
    gathered back: the gathered rows equal the oracle's, and each equals the
    cache row its slot names (a size-independent check)."""
    _say("indexer k insert + gather round trip T=65536")
    gen = torch.Generator().manual_seed(12)
    bs, hd, lens = 64, 128, [16384] * 4
    nblk = sum(n // bs for n in lens) + 16
    perm = torch.randperm(nblk, generator=gen).to(torch.int32)
    bt = perm[:sum(n // bs for n in lens)].view(4, -1).contiguous()
    cu = torch.tensor([0, 16384, 32768, 49152, 65536], dtype=torch.int32)
    pos = torch.arange(65536) % 16384
    req = torch.arange(65536) // 16384
    slots = (bt[req, pos // bs].to(torch.int64) * bs + pos % bs)
    k = W.randn_bf16((65536, hd), gen)
    cache = W.make_indexer_k_cache(nblk, bs, hd, gen)
    want_cache = _insert_oracle(k, cache, slots, "ue8m0")
    kf = torch.empty(65536, hd, dtype=torch.uint8)
    ks = torch.empty(65536, 4, dtype=torch.uint8)
    wk, ws = _gather_oracle(want_cache, kf, ks, bt, cu)
    g = cache.to(DEV)
    flaggems_vllm.indexer_k_quant_and_cache(k.to(DEV), g, slots.to(DEV), QB, "ue8m0")
    gk, gs = torch.empty_like(kf, device=DEV), torch.empty_like(ks, device=DEV)
    flaggems_vllm.cp_gather_indexer_k_quant_cache(g, gk, gs, bt.to(DEV), cu.to(DEV))
    torch.cuda.synchronize()
    _first_diff(g.cpu(), want_cache, "cache")
    _first_diff(gk.cpu(), wk, "k_fp8")
    _first_diff(gs.cpu(), ws, "k_fp8_scale")
    flat = want_cache.view(nblk, -1)
    idx = slots // bs, slots % bs
    assert torch.equal(wk, flat[idx[0][:, None], idx[1][:, None] * hd + torch.arange(hd)])


@pytest.mark.gpu
def test_gpu_graph_capture_replays():
    """Insert + gather captured in one HIP graph; three replays, each after a
    new key batch is copied into the captured input and with eager work and
    synchronisation between them, each checked against the oracle."""
    _say("indexer k insert + gather graph replays")
    gen = torch.Generator().manual_seed(13)
    bs, hd, T = 16, 512, 300
    nblk = T // bs + 2
    bt = torch.arange(nblk - 1, dtype=torch.int32)[None, :].contiguous()
    cu = torch.tensor([0, T], dtype=torch.int32)
    slots = torch.arange(T, dtype=torch.int64)
    cache0 = W.make_indexer_k_cache(nblk, bs, hd, gen)
    k_d = torch.empty(T, hd, dtype=torch.bfloat16, device=DEV)
    cache_d, slots_d, bt_d, cu_d = cache0.to(DEV), slots.to(DEV), bt.to(DEV), cu.to(DEV)
    kf = torch.zeros(T, hd, dtype=torch.uint8, device=DEV)
    ks = torch.zeros(T, 16, dtype=torch.uint8, device=DEV)
    k_d.copy_(W.randn_bf16((T, hd), gen).to(DEV))

    def run():
        flaggems_vllm.indexer_k_quant_and_cache(k_d, cache_d, slots_d, QB, "ue8m0")
        flaggems_vllm.cp_gather_indexer_k_quant_cache(cache_d, kf, ks, bt_d, cu_d)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for rep in range(3):
        k = W.randn_bf16((T, hd), gen) * (10.0 ** (rep - 1))
        k_d.copy_(k.to(DEV))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = _insert_oracle(k.to(torch.bfloat16), cache_d.cpu(), slots, "ue8m0")
        wk, ws = _gather_oracle(want, torch.zeros(T, hd, dtype=torch.uint8), torch.zeros(T, 16, dtype=torch.uint8),
                                bt, cu)
        _first_diff(cache_d.cpu(), want, f"replay {rep} cache")
        _first_diff(kf.cpu(), wk, f"replay {rep} k_fp8")
        _first_diff(ks.cpu(), ws, f"replay {rep} scales")
        _ = (k_d.float() * 2).sum().item()  # eager work between replays


@pytest.mark.gpu
def test_gpu_torch_ops_match_functions():
    _say("torch.ops indexer k insert / gather")
    k, cache, slots = W.make_indexer_k_insert(23, 5, 16, 512, torch.float16, seed=2)
    a, b = cache.to(DEV), cache.to(DEV)
    flaggems_vllm.indexer_k_quant_and_cache(k.to(DEV), a, slots.to(DEV), QB, "ue8m0")
    torch.ops.flaggems_vllm.indexer_k_quant_and_cache(k.to(DEV), b, slots.to(DEV), QB, "ue8m0")
    cache, kf, ks, bt, cu = W.make_indexer_k_gather([17, 1, 33, 9], 16, 512, 5)
    k1, s1, k2, s2 = kf.to(DEV), ks.to(DEV), kf.to(DEV), ks.to(DEV)
    flaggems_vllm.cp_gather_indexer_k_quant_cache(cache.to(DEV), k1, s1, bt.to(DEV), cu.to(DEV))
    torch.ops.flaggems_vllm.cp_gather_indexer_k_quant_cache(cache.to(DEV), k2, s2, bt.to(DEV), cu.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(k1.view(torch.uint8), k2.view(torch.uint8)) and torch.equal(s1, s2)
