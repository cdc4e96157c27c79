"""Seeded random cases of the byte-exact ops, GPU against the CPU oracle.

The per-op test files pin the reference's own shapes and the edge cases it
tests; these draw shapes, strides, alignments and edge patterns (padding
slots, DP padding, gaps between rows, odd head counts) at random from a fixed
seed per case, so a failure names a case that reruns the same way.  Every
comparison is bit for bit, including that nothing outside an output is
written.
"""
import pytest
import torch

import flaggems_vllm
import oracle
from flaggems_vllm import testing as W

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
CASES = range(16)


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _pick(g, options):
    return options[int(torch.randint(0, len(options), (1,), generator=g))]


def _rand(g, lo, hi):
    """Uniform integer in [lo, hi]."""
    return int(torch.randint(lo, hi + 1, (1,), generator=g))


def _sentinel(n, seed):
    return torch.randint(-32768, 32767, (n,), generator=torch.Generator().manual_seed(seed),
                         dtype=torch.int16)


def _placed(host, strides, lead, seed):
    """A device view of `host`'s values with the given element strides,
    starting `lead` elements into a sentinel-filled bf16 buffer; returns the
    view, the buffer and the buffer's original contents."""
    span = 1 + sum((s - 1) * st for s, st in zip(host.shape, strides))
    sent = _sentinel(lead + span + 64, seed).to(DEV)
    buf = sent.clone().view(torch.bfloat16)
    view = torch.as_strided(buf, host.shape, strides, lead)
    view.copy_(host.to(DEV))
    return view, buf, sent


def _untouched_outside(buf, sent, shape, strides, lead):
    inside = torch.zeros(buf.numel(), dtype=torch.bool, device=DEV)
    torch.as_strided(inside, shape, strides, lead).fill_(True)
    return torch.equal(buf.view(torch.int16)[~inside], sent[~inside])


# ------------------------------------------------------------------ main op ----

@pytest.mark.parametrize("case", CASES)
def test_fuzz_main_op(case):
    g = torch.Generator().manual_seed(1000 + case)
    T = _rand(g, 1, 160)
    H = _pick(g, [1, 3, 8, 16, 24, 64, 128])
    bs = _pick(g, [16, 32, 64])
    pad = _pick(g, [0, 0, 1, 5])
    n_ins = max(0, T - pad)
    q_gap = 8 * _pick(g, [0, 0, 1, 64, 128, 512])            # elements between tokens' q rows
    head_stride = _pick(g, [512, 512, 520])
    # any 16-byte offset below 32 KiB, or (half the time) a 1 KiB multiple, where
    # rows of 1 KiB units take the kernel's address-aligned chunk mapping
    lead = 8 * _rand(g, 0, 2047) if _pick(g, [False, True]) else 512 * _rand(g, 0, 31)
    kv_stride = 512 + 8 * _pick(g, [0, 0, 3, 64])
    extra = 8 * _pick(g, [0, 1, 16])                          # cache block stride beyond bs * 584
    max_pos = _pick(g, [64, 4096, 70000])
    eps = _pick(g, [1e-6, 1e-5])
    _say(f"fuzz main op {case}: T={T} H={H} bs={bs} ins={n_ins} gap={q_gap} hs={head_stride} lead={lead} "
         f"kvs={kv_stride} extra={extra}")

    q = W.randn_bf16((T, H, 512), g)
    kv = W.randn_bf16((T, 512), g)
    positions = torch.randint(0, max_pos, (T,), generator=g, dtype=torch.int64)
    nblk = (T + bs - 1) // bs + 2
    slots = torch.randperm(nblk * bs, generator=g)[:n_ins].to(torch.int64)
    slots[torch.rand(n_ins, generator=g) < 0.15] = -1
    cos_sin = W.make_cos_sin_cache(max_pos)
    cache = torch.zeros(nblk, bs * W.HEAD_BYTES + extra, dtype=torch.uint8)

    ref = W.Workload("fuzz", q.clone(), kv.clone(), cache.clone(), slots, positions, cos_sin, eps, bs)
    oracle.qnorm_rope_kv_insert(*ref.args())

    q_strides = (H * head_stride + q_gap, head_stride, 1)
    qd, qbuf, qsent = _placed(q, q_strides, lead, 7 + case)
    kvd, _, _ = _placed(kv, (kv_stride, 1), 0, 8 + case)
    cd = cache.to(DEV)
    flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(
        qd, kvd, cd, slots.to(DEV), positions.to(DEV), cos_sin.to(DEV), eps, bs)
    torch.cuda.synchronize()
    assert torch.equal(qd.cpu().view(torch.int16), ref.q.view(torch.int16)), "q differs"
    assert torch.equal(cd.cpu(), ref.k_cache), "cache differs"
    assert torch.equal(kvd.cpu(), kv), "kv written"
    assert _untouched_outside(qbuf, qsent, q.shape, q_strides, lead), "written outside q"


# ---------------------------------------------------------------- sibling ----

@pytest.mark.parametrize("case", CASES)
def test_fuzz_inv_rope_fp8_quant(case):
    g = torch.Generator().manual_seed(2000 + case)
    T = _rand(g, 1, 90)
    G = _pick(g, [1, 2, 4, 8])
    hpg = _pick(g, [1, 2, 4, 8])
    H = G * hpg
    tma = _pick(g, [False, True])
    head_stride = 512 + 8 * _pick(g, [0, 0, 2])
    tok_gap = 8 * _pick(g, [0, 0, 5, 64])
    max_pos = _pick(g, [128, 4096, 65536])
    scale = _pick(g, [1.0, 1e-3, 50.0])
    _say(f"fuzz sibling {case}: T={T} G={G} hpg={hpg} tma={tma} hs={head_stride} gap={tok_gap} scale={scale}")
    w = W.make_inv_rope_workload(T, H, G, seed=3000 + case, scale=scale, max_pos=max_pos)
    r8, rs = oracle.inv_rope_fp8_quant(w.o, w.positions, w.cos_sin_cache, G, hpg, tma_aligned_scales=tma)
    od, _, _ = _placed(w.o, (H * head_stride + tok_gap, head_stride, 1), 0, 9 + case)
    out, sc = flaggems_vllm.fused_inv_rope_fp8_quant(od, w.positions.to(DEV), w.cos_sin_cache.to(DEV), G, hpg,
                                                      tma_aligned_scales=tma)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().view(torch.uint8), r8)
    assert torch.equal(sc.cpu(), rs)


# ---------------------------------------------------------------- indexer ----

@pytest.mark.parametrize("case", CASES)
def test_fuzz_indexer_q_rope_quant(case):
    g = torch.Generator().manual_seed(4000 + case)
    T = _rand(g, 1, 80)
    H = _pick(g, [1, 3, 4, 8, 16, 64, 128])
    D = _pick(g, [128, 128, 256, 512])
    fp4 = _pick(g, [False, True])
    cs_dtype = _pick(g, [torch.float32, torch.bfloat16])
    w_dtype = _pick(g, [torch.bfloat16, torch.float32])
    head_stride = D + 8 * _pick(g, [0, 0, 2])
    tok_gap = 8 * _pick(g, [0, 0, 7])
    max_pos = _pick(g, [64, 4096])
    sm, hs = float(D) ** -0.5 * _pick(g, [1.0, 0.5]), float(H) ** -0.5
    _say(f"fuzz indexer {case}: T={T} H={H} D={D} fp4={fp4} cs={cs_dtype} w={w_dtype} hs={head_stride} gap={tok_gap}")
    q = W.randn_bf16((T, H, D), g)
    pos = torch.randint(0, max_pos, (T,), generator=g, dtype=torch.int64)
    cs = W.make_cos_sin_cache(max_pos).to(cs_dtype)
    wt = W.randn_bf16((T, H), g).to(w_dtype)
    (oq, ow) = oracle.fused_indexer_q_rope_quant(pos, q, cs, wt, sm, hs, use_fp4=fp4)
    qd, _, _ = _placed(q, (H * head_stride + tok_gap, head_stride, 1), 0, 10 + case)
    res, wo = flaggems_vllm.fused_indexer_q_rope_quant(pos.to(DEV), qd, cs.to(DEV), wt.to(DEV), sm, hs,
                                                       use_fp4=fp4)
    torch.cuda.synchronize()
    if fp4:
        assert torch.equal(res[0].cpu(), oq[0])
        assert torch.equal(res[1].cpu(), oq[1].contiguous().view(torch.int32).reshape(T, H, -1).squeeze(-1))
    else:
        assert torch.equal(res.cpu().view(torch.uint8), oq)
    assert torch.equal(wo.cpu(), ow)


# ----------------------------------------------------------------- gather ----

def _random_cache(g, nblk, bs):
    """Random 584-byte tokens: e4m3 codes without NaN, bf16 RoPE values,
    scale bytes in a finite range."""
    cache = torch.randint(0, 256, (nblk, bs * W.HEAD_BYTES), generator=g, dtype=torch.int32).to(torch.uint8)
    rows = cache[:, :bs * 576].view(nblk, bs, 576)
    codes = rows[:, :, :448]
    codes[(codes & 0x7F) == 0x7F] = 0x7E
    rope = W.randn_bf16((nblk, bs, 64), g)
    rows[:, :, 448:] = rope.view(torch.uint8).view(nblk, bs, 128)
    scl = cache[:, bs * 576:].view(nblk, bs, 8)
    scl[:, :, :7] = torch.randint(100, 150, (nblk, bs, 7), generator=g, dtype=torch.int32).to(torch.uint8)
    scl[:, :, 7] = 0
    return cache


@pytest.mark.parametrize("case", CASES)
def test_fuzz_dequantize_and_gather(case):
    g = torch.Generator().manual_seed(5000 + case)
    reqs = _rand(g, 1, 5)
    bs = _pick(g, [16, 64])
    seq_lens = torch.randint(0, 300, (reqs,), generator=g, dtype=torch.int32)
    use_gather = _pick(g, [False, True])
    gather_lens = (torch.minimum(seq_lens, torch.randint(0, 200, (reqs,), generator=g, dtype=torch.int32))
                   if use_gather else None)
    offset = _pick(g, [0, 0, 3])
    width = int(seq_lens.max()) // bs + 2
    nblk = reqs * width + 3
    bt = torch.randperm(nblk, generator=g)[:reqs * width].to(torch.int32).view(reqs, width)
    rows = int((gather_lens if use_gather else seq_lens).max()) + offset + _pick(g, [0, 5])
    _say(f"fuzz gather {case}: reqs={reqs} bs={bs} seq_lens={seq_lens.tolist()} gather={use_gather} "
         f"offset={offset} rows={rows}")
    cache = _random_cache(g, nblk, bs)
    out0 = _sentinel(reqs * max(rows, 1) * 512, 11 + case).view(torch.bfloat16).view(reqs, max(rows, 1), 512)
    ref = out0.clone()
    oracle.dequantize_and_gather_k_cache(ref, cache, seq_lens, gather_lens, bt, bs, offset=offset)
    od = out0.to(DEV)
    flaggems_vllm.dequantize_and_gather_k_cache(od, cache.to(DEV), seq_lens.to(DEV),
                                                gather_lens.to(DEV) if use_gather else None, bt.to(DEV), bs,
                                                offset)
    torch.cuda.synchronize()
    assert torch.equal(od.cpu().view(torch.int16), ref.view(torch.int16))


# ------------------------------------------------------------- sparse MLA ----

@pytest.mark.parametrize("case", range(12))
def test_fuzz_sparse_mla(case):
    """Random MODEL1 decode cases (rows, heads, query positions, top-k and its
    lengths, an extra list of another page size, the sink, entries that are not
    attended), with and without a workspace: both within the bound of the
    binary64 oracle, and when the extra cache is expanded without a split, the
    two routes agree bit for bit."""
    from flaggems_vllm import _native

    from .test_sparse_mla import _assert_within_bound, _gpu_raw, _oracle, _vmax

    g = torch.Generator().manual_seed(6000 + case)
    batch = _rand(g, 1, 6)
    heads = _pick(g, [64, 64, 128])
    seq_q = _pick(g, [1, 1, 2])
    topk = _pick(g, [1, 7, 64, 130, 300])
    num_pages = _pick(g, [1, 4, 16])
    extra = _pick(g, [False, True, True])
    extra_topk = _pick(g, [1, 40, 256, 600, 2100]) if extra else 0   # 2100: the split schedule
    extra_page = _pick(g, [2, 16, 64])
    extra_pages = _rand(g, 1, 40)
    lengths = _pick(g, [False, True])
    sink = _pick(g, [False, True])
    q_scale = _pick(g, [0.1, 1.0])
    _say(f"fuzz MLA {case}: B={batch} H={heads} SQ={seq_q} topk={topk} pages={num_pages} extra={extra_topk}"
         f"x{extra_page}/{extra_pages} lengths={lengths} sink={sink} q_scale={q_scale}")
    w = W.make_mla_workload(batch=batch, topk=topk, num_pages=num_pages, heads=heads, seq_q=seq_q,
                            extra_topk=extra_topk, extra_page=extra_page, extra_pages=extra_pages,
                            topk_length=lengths, sink=sink, seed=7000 + case, q_scale=q_scale)
    # entries that are not attended: negative, or past the cache
    for idx, entries in ((w.indices, num_pages * 64),
                         (w.extra_indices, extra_pages * extra_page if extra else 0)):
        if idx is None:
            continue
        flat = idx.view(-1)
        pick = torch.rand(flat.numel(), generator=g)
        flat[pick < 0.05] = -1
        flat[(pick >= 0.05) & (pick < 0.08)] = entries + 3
    o64, l64 = _oracle(w)
    vm = _vmax(w)
    out_w, lse_w, nbytes = _gpu_raw(w, workspace=True)
    out_n, lse_n, _ = _gpu_raw(w, workspace=False)
    for out, lse, what in ((out_w, lse_w, "workspace"), (out_n, lse_n, "no workspace")):
        _assert_within_bound(out, o64, vm, what)
        fin = torch.isfinite(l64)
        assert torch.equal(torch.isfinite(lse), fin), what
        assert torch.allclose(lse.double()[fin], l64[fin], rtol=1e-5, atol=1e-5), what
    split_only = _native.lib().fgv_sparse_mla_decode_workspace_bytes(batch, seq_q, heads, topk, extra_topk, 0)
    if nbytes > 0 and split_only == 0:  # expanded, not split: the same order of operations
        assert torch.equal(out_w.view(torch.int16), out_n.view(torch.int16))
        assert torch.equal(lse_w, lse_n)


@pytest.mark.parametrize("case", range(12))
def test_fuzz_sparse_mla_item_order(case):
    """One-item grids of random size around the CU count C (runs order up to C,
    paired order up to 2C, longest first up to 4C, in order beyond): the call
    equals, bit for bit, the same rows computed in calls of at most C items,
    each of which keeps every item on the workgroup of its own index."""
    from .test_sparse_mla import _gpu_raw, _grid, _rows_of

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    g = torch.Generator().manual_seed(6500 + case)
    heads = _pick(g, [64, 64, 128])
    seq_q = _pick(g, [1, 1, 2])
    per_row = seq_q * heads // 64
    lo, hi = [(cus // 2, cus), (cus + 1, 2 * cus), (2 * cus + 1, 4 * cus), (4 * cus + 1, 5 * cus)][case % 4]
    items = _rand(g, lo, hi)
    batch = (items + per_row - 1) // per_row  # C is a multiple of per_row: the count stays in its range
    topk = _pick(g, [32, 64, 96])
    extra = _pick(g, [False, True])
    ws = _pick(g, [False, True])
    _say(f"fuzz MLA item order {case}: items={batch * per_row} (C={cus}) B={batch} H={heads} SQ={seq_q} "
         f"topk={topk} extra={extra} workspace={ws}")
    w = W.make_mla_workload(batch=batch, topk=topk, num_pages=8, heads=heads, seq_q=seq_q,
                            extra_topk=64 if extra else 0, extra_page=64, extra_pages=4,
                            seed=7500 + case, q_scale=0.1)
    lens = torch.randint(-2, topk + 3, (batch,), generator=g, dtype=torch.int32)  # clamped at both ends
    lens[torch.rand(batch, generator=g) < 0.1] = 0
    w.topk_length = lens
    if extra:
        w.extra_topk_length = torch.randint(0, 65, (batch,), generator=g, dtype=torch.int32)
    assert _grid(w) == 0
    out, lse, _ = _gpu_raw(w, workspace=ws)
    step = max(1, cus // per_row)
    for r0 in range(0, batch, step):
        rows = torch.arange(r0, min(batch, r0 + step))
        o_part, l_part, _ = _gpu_raw(_rows_of(w, rows), workspace=ws)
        assert torch.equal(out[rows].view(torch.int16), o_part.view(torch.int16)), f"rows from {r0}"
        assert torch.equal(lse[rows], l_part), f"rows from {r0}"


# ---------------------------------------------------------------- rmsnorm ----

@pytest.mark.parametrize("case", CASES)
def test_fuzz_q_kv_rmsnorm(case):
    import flaggems_vllm

    g = torch.Generator().manual_seed(8000 + case)
    T = _pick(g, [1, 2, 17, 300, 1025])
    qd, kd = 8 * _rand(g, 1, 1024), 8 * _rand(g, 1, 1024)   # row sizes: multiples of 8 up to 8192
    wdtype = _pick(g, [torch.bfloat16, torch.float32])
    q_gap, k_gap = 8 * _pick(g, [0, 0, 3]), 8 * _pick(g, [0, 0, 5])
    eps = _pick(g, [1e-6, 1e-5])
    scale = _pick(g, [1.0, 1e-3, 200.0])
    _say(f"fuzz rmsnorm {case}: T={T} q={qd} kv={kd} w={wdtype} gaps={q_gap},{k_gap} scale={scale}")
    qr = (W.randn_bf16((T, qd), g).float() * scale).to(torch.bfloat16)
    kv = W.randn_bf16((T, kd), g)
    qw, kw = W.randn_bf16((qd,), g).to(wdtype), W.randn_bf16((kd,), g).to(wdtype)
    rq, rk = oracle.fused_q_kv_rmsnorm(qr, kv, qw, kw, eps)
    qrd, _, _ = _placed(qr, (qd + q_gap, 1), 0, 12 + case)
    kvd, _, _ = _placed(kv, (kd + k_gap, 1), 0, 13 + case)
    qo, ko = flaggems_vllm.fused_q_kv_rmsnorm(qrd, kvd, qw.to(DEV), kw.to(DEV), eps)
    torch.cuda.synchronize()
    assert torch.equal(qo.cpu().view(torch.int16), rq.view(torch.int16))
    assert torch.equal(ko.cpu().view(torch.int16), rk.view(torch.int16))


# ----------------------------------------------------------- slot mapping ----

@pytest.mark.parametrize("case", CASES)
def test_fuzz_slot_mapping(case):
    import flaggems_vllm

    g = torch.Generator().manual_seed(9000 + case)
    nreq = _rand(g, 1, 40)
    bs = _pick(g, [1, 16, 64, 128])
    cpw = _pick(g, [1, 1, 2, 4])
    rank = _rand(g, 0, cpw - 1)
    il = _pick(g, [1, 1, 2, 16])
    lens = torch.randint(0, 120, (nreq,), generator=g)
    qsl = torch.zeros(nreq + 1, dtype=torch.int32)
    qsl[1:] = torch.cumsum(lens, 0).to(torch.int32)
    n = int(qsl[-1])
    starts = torch.randint(0, 5000, (nreq,), generator=g)
    pos = torch.cat([s + torch.arange(int(k)) for s, k in zip(starts.tolist(), lens.tolist())] +
                    [torch.zeros(0, dtype=torch.int64)]).to(_pick(g, [torch.int32, torch.int64]))
    maxb = (5200 + bs * cpw - 1) // (bs * cpw)
    bt = torch.randint(0, 1 << 20, (nreq, maxb), generator=g, dtype=torch.int32)
    max_tokens = n + _pick(g, [0, 1, 37])
    pad = _pick(g, [-1, 0, -7])
    _say(f"fuzz slot mapping {case}: reqs={nreq} tokens={n} bs={bs} cp={cpw}/{rank} il={il} pad={pad}")
    kw = dict(cp_world_size=cpw, cp_rank=rank, cp_kv_cache_interleave_size=il, pad_id=pad)
    want = torch.full((max_tokens + 3,), -99, dtype=torch.int64)
    oracle.compute_slot_mapping(n, max_tokens, qsl, nreq, pos, bt, want, bs, **kw)
    got = torch.full((max_tokens + 3,), -99, dtype=torch.int64, device=DEV)
    flaggems_vllm.compute_slot_mapping_parallel(n, max_tokens, qsl.to(DEV), nreq, pos.to(DEV), bt.to(DEV), got, bs,
                                                **kw)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want)
