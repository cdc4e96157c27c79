"""GPU parity of the main op against the CPU oracle (bit for bit) and against
the reference's torch formulation.

Reference tests mirrored: tests/test_fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py
  test_q_path_matches_reference :358-402, test_kv_path_matches_reference :419-462,
  test_kv_path_with_dp_padding :468-515, test_combined_q_and_kv :521-573.
"""
import pytest
import torch

import flaggems_vllm
import oracle
from flaggems_vllm import testing as W
from oracle import torch_ref

from ._helpers import (bf16_ulp_distance, bf16_ulp_size, oracle_main, rope_cancellation_bound,
                       slot_byte_index, sub_workload)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
OP = flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def run_gpu(w: W.Workload):
    g = w.to(DEV)
    OP(*g.args())
    torch.cuda.synchronize()
    return g


def assert_q_exact(q_gpu_cpu, q_ref, what):
    d = bf16_ulp_distance(q_gpu_cpu, q_ref)
    n_bad = int((d > 0).sum())
    assert n_bad == 0, f"{what}: {n_bad} q elements differ from the oracle (max {int(d.max())} ulp)"


# Rope elements of q allowed beyond 1 bf16 ulp of the reference's torch
# formulation: this fraction of all rope elements, plus one (a shape of a few
# hundred thousand rope elements is too small for the rate to mean anything).
# The torch path's float32 RMS factor differs from the correctly rounded one
# by a few float32 ulps; where the rotation e*c - o*s (or e*s + o*c) cancels,
# that moves the result by more than one of its own ulps.  Measured (the GPU
# equals the C oracle bit for bit): c2 13 of 33,554,432 (max 16 ulps), c3's
# 2048 sampled tokens 9 of 16,777,216, c4's 7 of 8,388,608, the reference's
# T=1000 H=128 shape 4 of 8,192,000, T=64 H=64 1 of 262,144; none at c0, c1.
ROPE_BEYOND_1ULP_CEILING = 1e-6


def assert_q_within_torch_ref(q_gpu_cpu, w_in: W.Workload, what):
    """North-star bar against the reference's torch formulation: every nope
    element within 1 bf16 ulp; rope elements within 1 ulp except at most
    ROPE_BEYOND_1ULP_CEILING of them plus one, and each of those within 1 ulp plus the
    cancellation term of rope_cancellation_bound.  Prints the counts and the
    largest distances."""
    r = w_in.clone()
    torch_ref.qnorm_rope_kv_insert(*r.args())
    d = bf16_ulp_distance(q_gpu_cpu, r.q)
    nope_d, rope_d = d[..., :448], d[..., 448:]
    beyond = rope_d > 1
    n_beyond = int(beyond.sum())
    print(f"[q vs torch ref] {what}: nope elements at 1 ulp {int((nope_d == 1).sum())} of "
          f"{nope_d.numel()} (max {int(nope_d.max())} ulp); rope elements beyond 1 ulp {n_beyond} of "
          f"{rope_d.numel()} (max {int(rope_d.max())} ulp)", flush=True)
    assert int(nope_d.max()) <= 1, f"{what}: nope beyond 1 ulp"
    assert n_beyond <= ROPE_BEYOND_1ULP_CEILING * rope_d.numel() + 1, (
        f"{what}: {n_beyond} rope elements beyond 1 ulp, above the ceiling")
    if n_beyond:
        tok = torch.nonzero(beyond.flatten(1).any(1)).flatten()  # only tokens with an exceedance
        xf = w_in.q[tok].float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + w_in.eps)
        cs = w_in.cos_sin_cache[w_in.position_ids[tok]][:, None, :]
        bound = rope_cancellation_bound(y[..., 448:], cs) + bf16_ulp_size(r.q[tok][..., 448:])
        diff = (q_gpu_cpu[tok][..., 448:].float() - r.q[tok][..., 448:].float()).abs()
        assert bool((diff <= bound).all()), f"{what}: rope beyond the cancellation bound"


@pytest.mark.parametrize("config", [0, 1, 2])
def test_benchmark_configs_full(config):
    """c0-c2 at full size: q and the whole cache bit-exact vs the oracle."""
    _say(f"main op c{config} full size")
    w = W.make_workload(config)
    g = run_gpu(w)
    ref = oracle_main(w)
    assert_q_exact(g.q.cpu(), ref.q, f"c{config}")
    assert torch.equal(g.k_cache.cpu(), ref.k_cache), f"c{config}: k_cache differs"
    assert torch.equal(g.kv.cpu(), w.kv), f"c{config}: kv modified"
    assert_q_within_torch_ref(g.q.cpu(), w, f"c{config}")


@pytest.mark.parametrize("config", [3, 4])
def test_benchmark_configs_sampled(config):
    """c3 (T=32768, H=128, 2^31 q elements: int64 addressing) and c4 (ragged,
    strided q/kv views of one buffer, 10% padding) at full size; 2048 sampled
    tokens compared bit for bit with the oracle, and size-independent checks on
    everything: cache bytes outside inserted slots untouched, every inserted
    token's dequantised nope within e4m3 error of kv, kv unchanged."""
    _say(f"main op c{config} full size, sampled oracle")
    w = W.make_workload(config)
    g = run_gpu(w)
    gen = torch.Generator().manual_seed(100 + config)
    toks = torch.randperm(w.num_tokens, generator=gen)[:2048].sort().values
    sub = sub_workload(w, toks)
    ref = oracle_main(sub)
    q_sampled = g.q[toks.to(DEV)].cpu()
    assert_q_exact(q_sampled, ref.q, f"c{config} sampled q")
    assert_q_within_torch_ref(q_sampled, sub, f"c{config} sampled")
    keep = sub.slot_mapping >= 0
    idx = slot_byte_index(sub.slot_mapping[keep], w.block_size, w.k_cache.stride(0))
    flat_g = g.k_cache.view(-1)
    assert torch.equal(flat_g[idx.to(DEV)].cpu(), ref.k_cache.view(-1)[idx]), f"c{config}: slots differ"

    # every inserted slot, on the GPU: outside bytes zero, nope round trip
    slots = g.slot_mapping[g.slot_mapping >= 0]
    tok_ids = torch.nonzero(g.slot_mapping >= 0).flatten()
    all_idx = slot_byte_index(slots, w.block_size, w.k_cache.stride(0))
    bytes_ = flat_g[all_idx]
    rest = g.k_cache.clone().view(-1)
    rest[all_idx] = 0
    assert int(torch.count_nonzero(rest)) == 0, f"c{config}: bytes outside slots written"
    codes = bytes_[:, :448].contiguous().view(torch.float8_e4m3fn).float().view(-1, 7, 64)
    expo = bytes_[:, 576:583].to(torch.float32) - 127.0
    deq = codes * torch.exp2(expo)[..., None]
    x = g.kv[tok_ids, :448].float().view(-1, 7, 64)
    tol = torch.maximum(x.abs() * 2.0 ** -4, torch.exp2(expo - 10.0)[..., None])
    assert bool(((deq - x).abs() <= tol).all()), f"c{config}: dequantised kv out of e4m3 error"
    assert int(bytes_[:, 583].abs().sum()) == 0, "pad byte not zero"
    assert torch.equal(g.kv.cpu(), w.kv), f"c{config}: kv modified"
    # q rows are RMS-normalised: mean square within bf16 rounding of 1
    ms = g.q.float().pow(2).mean(-1)
    assert float((ms - 1).abs().max()) < 2e-2


def _ref_style(T, H, bs, *, kv_random, q_random, slots, seed, pad=0):
    """Inputs built like the reference tests (positions = arange, cos/sin
    base chosen by max_pos as in tests/...insert.py:68-90)."""
    g = torch.Generator().manual_seed(seed)
    total = T + pad
    max_pos = max(4096, total)
    base = 10000.0 if max_pos <= 8192 else 20000.0 if max_pos <= 32768 else 40000.0 \
        if max_pos <= 65536 else 60000.0 if max_pos <= 98304 else 100000.0
    q = W.randn_bf16((total, H, 512), g) if q_random else torch.zeros(total, H, 512, dtype=torch.bfloat16)
    kv = W.randn_bf16((total, 512), g) if kv_random else torch.zeros(total, 512, dtype=torch.bfloat16)
    nblk = (T + bs - 1) // bs + 1
    cache = torch.zeros(nblk, bs * W.HEAD_BYTES, dtype=torch.uint8)
    return W.Workload(f"ref T{T} H{H} bs{bs}", q, kv, cache, slots,
                      torch.arange(total, dtype=torch.int64), W.make_cos_sin_cache(max_pos, base=base),
                      1e-6, bs)


def _check_ref_case(w):
    g = run_gpu(w)
    ref = oracle_main(w)
    assert_q_exact(g.q.cpu(), ref.q, w.name)
    assert torch.equal(g.k_cache.cpu(), ref.k_cache), f"{w.name}: cache differs"
    t = w.clone()
    torch_ref.qnorm_rope_kv_insert(*t.args())
    # the reference's own assertions: q at 1e-2, fp8 codes and scales exact,
    # and under DP padding the whole cache exact
    torch.testing.assert_close(g.q.cpu(), t.q, rtol=1e-2, atol=1e-2)
    assert torch.equal(g.k_cache.cpu(), t.k_cache), f"{w.name}: cache differs from torch ref"
    assert_q_within_torch_ref(g.q.cpu(), w, w.name)


@pytest.mark.parametrize("T", [1, 4, 17, 64])
@pytest.mark.parametrize("H", [8, 64])
def test_q_path(T, H):
    _say(f"q path T={T} H={H}")
    _check_ref_case(_ref_style(T, H, 16, kv_random=False, q_random=True,
                               slots=torch.full((T,), -1, dtype=torch.int64), seed=0))


@pytest.mark.parametrize("T", [1, 4, 17, 64])
@pytest.mark.parametrize("bs", [16, 64])
def test_kv_path(T, bs):
    _say(f"kv path T={T} bs={bs}")
    _check_ref_case(_ref_style(T, 1, bs, kv_random=True, q_random=False,
                               slots=torch.arange(T, dtype=torch.int64), seed=1))


@pytest.mark.parametrize("T", [4, 17])
@pytest.mark.parametrize("pad", [1, 5])
@pytest.mark.parametrize("bs", [16, 64])
def test_kv_path_dp_padding(T, pad, bs):
    _say(f"dp padding T={T} pad={pad} bs={bs}")
    _check_ref_case(_ref_style(T, 1, bs, kv_random=True, q_random=False,
                               slots=torch.arange(T, dtype=torch.int64), seed=3, pad=pad))


@pytest.mark.parametrize("T", [1, 4, 17, 64, 1000, 8192])
@pytest.mark.parametrize("H", [64, 128])
@pytest.mark.parametrize("bs", [16, 64])
def test_combined(T, H, bs):
    _say(f"combined T={T} H={H} bs={bs}")
    w = _ref_style(T, H, bs, kv_random=True, q_random=True,
                   slots=torch.arange(T, dtype=torch.int64), seed=2)
    if T * H > (1 << 20):
        g = run_gpu(w)
        ref = oracle_main(w)
        assert_q_exact(g.q.cpu(), ref.q, w.name)
        assert torch.equal(g.k_cache.cpu(), ref.k_cache)
    else:
        _check_ref_case(w)


# (T, H, gap units between tokens, 1 KiB units from the 16 KiB boundary below q).
# These place q so that its rows do not tile 16 KiB-aligned chunks, which the
# kernel then walks chunk by chunk of address space: gaps smaller and larger
# than a chunk, q starting mid-chunk, head counts below / not a multiple of 16,
# one token, and the contiguous-but-misaligned case.
LAYOUTS = [
    (37, 64, 1, 0),    # c4: q = buf[:, :H*512] of a [T, H*512 + 512] buffer
    (37, 64, 1, 3),
    (50, 7, 0, 5),     # contiguous rows, misaligned start
    (20, 16, 0, 1),
    (9, 3, 40, 2),     # gap wider than a chunk: whole chunks hold no q row
    (1, 64, 0, 9),
    (33, 128, 5, 15),
    (200, 1, 2, 7),
    (64, 64, 0, 0),    # aligned and contiguous: the row-order mapping
    (100, 64, 1, 3),   # a grid of 414 workgroups: chunk mapping in XCD-contiguous order
]


@pytest.mark.parametrize("T,H,gap,lead", LAYOUTS)
def test_q_layouts(T, H, gap, lead):
    """q as a strided view at a chosen address: every q element bit-exact vs the
    oracle, the cache exact, and every element of the buffer outside q (pitch
    gaps, before and after) left as it was."""
    _say(f"q layout T={T} H={H} gap={gap} lead={lead}")
    w = _ref_style(T, H, 16, kv_random=True, q_random=True,
                   slots=torch.arange(T, dtype=torch.int64), seed=4)
    ref = oracle_main(w)
    pitch = (H + gap) * 512
    n = T * pitch + 16 * 1024  # elements, with room for the alignment shift
    sentinel = torch.randint(-32768, 32767, (n,), generator=torch.Generator().manual_seed(9),
                             dtype=torch.int16).to(DEV)
    buf = sentinel.clone().view(torch.bfloat16)
    # element offset putting q at `lead` KiB past a 16 KiB boundary
    start = ((16384 - buf.data_ptr() % 16384) % 16384 + lead * 1024) // 2
    q = torch.as_strided(buf, (T, H, 512), (pitch, 512, 1), start)
    assert (q.data_ptr() % 16384) == lead * 1024
    q.copy_(w.q.to(DEV))
    g = w.to(DEV)
    OP(q, g.kv, g.k_cache, g.slot_mapping, g.position_ids, g.cos_sin_cache, g.eps, g.block_size)
    torch.cuda.synchronize()
    assert_q_exact(q.cpu(), ref.q, f"layout {T, H, gap, lead}")
    assert torch.equal(g.k_cache.cpu(), ref.k_cache)
    outside = torch.ones(n, dtype=torch.bool, device=DEV)
    torch.as_strided(outside, (T, H, 512), (pitch, 512, 1), start).fill_(False)
    assert torch.equal(buf.view(torch.int16)[outside], sentinel[outside]), "elements outside q written"


@pytest.mark.parametrize("T", [1, 32, 256])
@pytest.mark.parametrize("H", [64, 128])
def test_real_deepseek_v4_rope(T, H):
    """DeepSeek-V4's YaRN-scaled cos/sin table (scaling 16, 65536 original
    positions; the first 65536 of its 1,048,576 rows) at random positions in
    [0, 4096), as the reference's sibling test draws them
    (tests/test_fused_inv_rope_fp8_quant.py:586-620): q, rope and cache bytes bit
    for bit against the oracle."""
    _say(f"real DeepSeek-V4 rope T={T} H={H}")
    g = torch.Generator().manual_seed(5)
    w = W.Workload(f"yarn T{T} H{H}", W.randn_bf16((T, H, 512), g), W.randn_bf16((T, 512), g),
                   torch.zeros((T + 63) // 64 + 1, 64 * W.HEAD_BYTES, dtype=torch.uint8),
                   torch.randperm(((T + 63) // 64 + 1) * 64, generator=g)[:T].to(torch.int64),
                   torch.randint(0, 4096, (T,), generator=g, dtype=torch.int64),
                   W.make_yarn_cos_sin_cache(65536, rows=65536), 1e-6, 64)
    _check_ref_case(w)


def test_one_dimensional_cache():
    """A 1-D k_cache (one block of numel bytes) carved from a larger buffer:
    slots inside the block are written as the oracle writes them, slots past
    cache_block_size are skipped, and no byte after the cache changes."""
    _say("main op 1-D k_cache")
    bs, T = 16, 12
    g = torch.Generator().manual_seed(12)
    slots = torch.tensor([0, 3, 15, 16, 17, 40, -1, 5, 31, 2, 100, 9], dtype=torch.int64)
    w = W.Workload("1-D cache", W.randn_bf16((T, 8, 512), g), W.randn_bf16((T, 512), g),
                   torch.zeros(1, bs * W.HEAD_BYTES, dtype=torch.uint8), slots,
                   torch.randint(0, 4096, (T,), generator=g, dtype=torch.int64),
                   W.make_cos_sin_cache(4096), 1e-6, bs)
    ref_in = w.clone()
    ref_in.slot_mapping = torch.where(slots < bs, slots, torch.full_like(slots, -1))
    ref = oracle_main(ref_in)
    sentinel = torch.randint(0, 256, (3 * bs * W.HEAD_BYTES,), generator=g, dtype=torch.int32).to(torch.uint8)
    buf = sentinel.clone().to(DEV)
    cache = buf[:bs * W.HEAD_BYTES]
    cache.zero_()
    assert cache.dim() == 1
    d = w.to(DEV)
    OP(d.q, d.kv, cache, d.slot_mapping, d.position_ids, d.cos_sin_cache, d.eps, bs)
    torch.cuda.synchronize()
    assert torch.equal(cache.cpu(), ref.k_cache.view(-1))
    assert torch.equal(buf[bs * W.HEAD_BYTES:].cpu(), sentinel[bs * W.HEAD_BYTES:]), "bytes past the cache written"
    assert_q_exact(d.q.cpu(), ref.q, "1-D cache")


# The reference's largest combined shapes
# (tests/test_fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:525-531):
# up to 131072 tokens x 128 heads = 2^33 q elements (16 GiB), where any 32-bit
# element or byte offset would wrap.
@pytest.mark.parametrize("T", [65536, 131072])
@pytest.mark.parametrize("H", [64, 128])
@pytest.mark.parametrize("bs", [16, 64])
def test_combined_largest(T, H, bs):
    """q and kv drawn on the device (seeded), positions = arange, the rope
    base chosen by max_pos as the reference test does.  Before the call,
    2048 sampled tokens of q are copied to the host (the first and last
    tokens and those on either side of the 2^31-element and 2^32- and
    2^33-byte offsets included); afterwards their q rows are compared bit for
    bit with the C oracle, and the whole cache with the oracle's kv insert
    over all T tokens."""
    _say(f"combined largest T={T} H={H} bs={bs}")
    gen = torch.Generator(device=DEV).manual_seed(7 + T + H + bs)
    q = torch.randn(T, H, 512, generator=gen, device=DEV, dtype=torch.bfloat16)
    kv = torch.randn(T, 512, generator=gen, device=DEV, dtype=torch.bfloat16)
    row_bytes = H * 1024
    edges = set([0, 1, T - 2, T - 1])
    for off in (1 << 31, 1 << 32, 1 << 33):   # bytes; 2^31 elements = 2^32 bytes
        t = off // row_bytes
        edges.update(x for x in (t - 1, t, t + 1) if 0 <= x < T)
    hsel = torch.Generator().manual_seed(T * 3 + H)
    toks = torch.randperm(T, generator=hsel)[:2048 - len(edges)]
    toks = torch.unique(torch.cat([toks, torch.tensor(sorted(edges))]))
    q_in = q[toks.to(DEV)].cpu()
    kv_cpu = kv.cpu()
    positions = torch.arange(T, dtype=torch.int64)
    base = 10000.0 if T <= 8192 else 20000.0 if T <= 32768 else 40000.0 if T <= 65536 \
        else 60000.0 if T <= 98304 else 100000.0
    cos_sin = W.make_cos_sin_cache(T, base=base)
    slots = torch.arange(T, dtype=torch.int64)
    nblk = (T + bs - 1) // bs + 1
    cache = torch.zeros(nblk, bs * W.HEAD_BYTES, dtype=torch.uint8, device=DEV)
    OP(q, kv, cache, slots.to(DEV), positions.to(DEV), cos_sin.to(DEV), 1e-6, bs)
    torch.cuda.synchronize()
    q_out = q[toks.to(DEV)].cpu()
    cache_out = cache.cpu()
    del q, kv, cache
    torch.cuda.empty_cache()

    sub = W.Workload("sampled", q_in, kv_cpu[toks].clone(), torch.zeros(1, bs * W.HEAD_BYTES, dtype=torch.uint8),
                     torch.full((toks.numel(),), -1, dtype=torch.int64), positions[toks].clone(), cos_sin, 1e-6, bs)
    ref = oracle_main(sub)
    assert_q_exact(q_out, ref.q, f"T={T} H={H} sampled q")
    full = W.Workload("kv", torch.zeros(T, 0, 512, dtype=torch.bfloat16), kv_cpu,
                      torch.zeros(nblk, bs * W.HEAD_BYTES, dtype=torch.uint8), slots, positions, cos_sin, 1e-6, bs)
    ref_kv = oracle_main(full)
    assert torch.equal(cache_out, ref_kv.k_cache), f"T={T} H={H} bs={bs}: cache differs"


# Grids around one round of workgroups (T * H from 8192 to 32769 rows, 512 to
# 2049 blocks): head counts that are and are not multiples of the 16-row block
# (one token per block or not), ragged last blocks, H = 1.
# (256, 64), (129, 128), (160, 112), (200, 128) and (496, 64) are one-round
# grids of 1024-2048 workgroups with whole tokens per block: the cos/sin row is
# staged in LDS there (1028, 1041, 1130, 1613 and 2015 workgroups).
@pytest.mark.parametrize("T,H", [(8193, 1), (600, 16), (257, 37), (300, 48), (256, 64), (129, 128),
                                 (160, 112), (200, 128), (496, 64), (512, 64), (8192, 1), (32769, 1)])
def test_mid_size_grids(T, H):
    _say(f"mid-size grid T={T} H={H}")
    g = torch.Generator().manual_seed(T + H)
    nblk = (T + 63) // 64 + 2
    slots = torch.randperm(nblk * 64, generator=g)[:T].to(torch.int64)
    slots[::11] = -1
    w = W.Workload(f"R2 T{T} H{H}", W.randn_bf16((T, H, 512), g), W.randn_bf16((T, 512), g),
                   torch.zeros(nblk, 64 * W.HEAD_BYTES, dtype=torch.uint8), slots,
                   torch.randint(0, 4096, (T,), generator=g, dtype=torch.int64),
                   W.make_cos_sin_cache(4096), 1e-6, 64)
    gw = run_gpu(w)
    ref = oracle_main(w)
    assert_q_exact(gw.q.cpu(), ref.q, w.name)
    assert torch.equal(gw.k_cache.cpu(), ref.k_cache), f"{w.name}: cache differs"


def test_lds_cos_sin_path_clamps_positions():
    """The one-round grid that stages cos/sin in LDS (T = 256, H = 64: 1028
    workgroups) with positions below 0 and past the cache's rows: clamped into
    the table as on every other path, bit-exact against the oracle."""
    _say("main op, LDS cos/sin path with out-of-range positions")
    T, H = 256, 64
    g = torch.Generator().manual_seed(77)
    nblk = (T + 63) // 64 + 2
    slots = torch.randperm(nblk * 64, generator=g)[:T].to(torch.int64)
    pos = torch.randint(0, 2048, (T,), generator=g, dtype=torch.int64)
    pos[::7] = -3
    pos[3::7] = 2048 + 17
    pos[5::7] = 2047
    w = W.Workload("lds cos/sin clamp", W.randn_bf16((T, H, 512), g), W.randn_bf16((T, 512), g),
                   torch.zeros(nblk, 64 * W.HEAD_BYTES, dtype=torch.uint8), slots, pos,
                   W.make_cos_sin_cache(2048), 1e-6, 64)
    gw = run_gpu(w)
    ref = oracle_main(w)
    assert_q_exact(gw.q.cpu(), ref.q, w.name)
    assert torch.equal(gw.k_cache.cpu(), ref.k_cache), f"{w.name}: cache differs"


# The kernel runs blocks in XCD-contiguous order on one-round grids of 256..1152
# workgroups, and in runs of 16 blocks per XCD from 81920 workgroups (also
# taken by c3, c4 and test_combined_largest): a prefix of the grid permuted,
# the tail in place.  Grids at both edges
# (kv blocks included: T q blocks of 16 heads plus ceil(Tins / 16)), one with
# heads not a multiple of 16, all bit-exact against the oracle.
@pytest.mark.parametrize("T,H,n_ins", [(240, 16, 240), (241, 16, 240), (1084, 16, 1084), (1085, 16, 1085),
                                       (1100, 3, 1100), (150, 48, 149)])
def test_block_order_boundaries(T, H, n_ins):
    grid = -(-T * H // 16) + -(-n_ins // 16)
    _say(f"block order T={T} H={H} inserted={n_ins} grid={grid}")
    g = torch.Generator().manual_seed(5 * T + H)
    nblk = (T + 63) // 64 + 2
    slots = torch.randperm(nblk * 64, generator=g)[:n_ins].to(torch.int64)
    slots[::13] = -1
    w = W.Workload(f"order T{T} H{H}", W.randn_bf16((T, H, 512), g), W.randn_bf16((T, 512), g),
                   torch.zeros(nblk, 64 * W.HEAD_BYTES, dtype=torch.uint8), slots,
                   torch.randint(0, 4096, (T,), generator=g, dtype=torch.int64),
                   W.make_cos_sin_cache(4096), 1e-6, 64)
    gw = run_gpu(w)
    ref = oracle_main(w)
    assert_q_exact(gw.q.cpu(), ref.q, w.name)
    assert torch.equal(gw.k_cache.cpu(), ref.k_cache), f"{w.name}: cache differs"


# Just below and above the runs order's 81920 workgroups (T * 8 q blocks at
# H = 128 plus ceil(T / 16) kv blocks): 80625 and 82569, the latter with a
# tail of 9 blocks past the last whole group of 128.  Whole q bit-exact.
@pytest.mark.parametrize("T", [10000, 10241])
def test_block_runs_boundary(T):
    H = 128
    grid = T * H // 16 + -(-T // 16)
    _say(f"block runs T={T} H={H} grid={grid}")
    g = torch.Generator().manual_seed(T)
    nblk = (T + 63) // 64 + 2
    slots = torch.randperm(nblk * 64, generator=g)[:T].to(torch.int64)
    slots[::17] = -1
    w = W.Workload(f"runs T{T}", W.randn_bf16((T, H, 512), g), W.randn_bf16((T, 512), g),
                   torch.zeros(nblk, 64 * W.HEAD_BYTES, dtype=torch.uint8), slots,
                   torch.randint(0, 65536, (T,), generator=g, dtype=torch.int64),
                   W.make_cos_sin_cache(65536), 1e-6, 64)
    gw = run_gpu(w)
    ref = oracle_main(w)
    assert_q_exact(gw.q.cpu(), ref.q, w.name)
    assert torch.equal(gw.k_cache.cpu(), ref.k_cache), f"{w.name}: cache differs"
