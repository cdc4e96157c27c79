"""Sparse MLA decode over the 584-byte MODEL1 cache: oracle pins (CPU),
wrapper checks (CPU) and GPU parity.

Reference: src/flaggems_vllm/ops/flash_mla_with_kvcache.py:489-688 (portable
MODEL1 kernel), :852-1073 (wrapper and its assertions);
tests/test_flash_mla_with_kvcache.py:94-140 (cache generator), :236-360
(MODEL1 cases: batch 8 / 64 heads / top-k 128 / 16 pages, seed 43, and the
extra-cache cases (64, 512, 12), (2, 512, 260)), :420-486 (error cases).
The reference checks its kernel against vLLM's CUDA FlashMLA with cosine
similarity above 0.98; vLLM is not available here, so the bar is the binary64
oracle with the rounding bound derived below, plus the reference's own
algorithm restated in torch (oracle.torch_ref).

Tolerance (stated per element): the kernel rounds each probability to bf16
before the PV product (relative error <= 2^-9, as the reference does) and
rounds the output to bf16 (<= 2^-9 relative); fp32 accumulation and exp2 add
~1e-6 relative.  Hence
    |out - out64| <= 2^-9 |out64| + 2^-9 * max_t |V[t, d]| + tiny
and the test allows 2^-8 (|out64| + max_t |V[t, d]|), the maximum taken over
the entries the row attends.  A dropped, duplicated or mis-scaled entry moves
the output by about |V| / topk, far outside this for the shapes tested.
"""
import math

import pytest
import torch

import oracle
from flaggems_vllm import testing as W
from oracle import torch_ref

DEV = torch.device("cuda:0")


# ------------------------------------------------------------ helpers ----

def _attended(w):
    """For each (b, sq): list of (rows tensor, ids) attended, main then extra."""
    lists = [(torch_ref.model1_rows(w.k_cache.cpu()), w.k_cache.shape[0] * w.k_cache.shape[1],
              w.indices.cpu(), w.topk_length)]
    if w.extra_k_cache is not None:
        lists.append((torch_ref.model1_rows(w.extra_k_cache.cpu()),
                      w.extra_k_cache.shape[0] * w.extra_k_cache.shape[1],
                      w.extra_indices.cpu(), w.extra_topk_length))
    B, SQ = w.q.shape[:2]
    out = {}
    for b in range(B):
        for s in range(SQ):
            got = []
            for rows, limit, idx, length in lists:
                topk = idx.shape[-1]
                n = topk if length is None else max(0, min(int(length[b]), topk))
                ids = idx[b, s, :n].long()
                ids = ids[(ids >= 0) & (ids < limit)]
                got.append(rows[ids].float())
            out[(b, s)] = torch.cat(got, 0)
    return out


def _vmax(w):
    """[B, SQ, 1, 512]: max over attended entries of |V[t, d]| (0 if none)."""
    B, SQ = w.q.shape[:2]
    vm = torch.zeros(B, SQ, 1, 512, dtype=torch.float64)
    for (b, s), rows in _attended(w).items():
        if rows.shape[0]:
            vm[b, s, 0] = rows.abs().amax(0).double()
    return vm


def _oracle(w):
    return oracle.sparse_mla_decode_model1(w.q.cpu(), w.k_cache.cpu(), w.indices.cpu(),
                                           **_cpu_kwargs(w))


def _cpu_kwargs(w):
    kw = w.oracle_kwargs()
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in kw.items()}


def _assert_within_bound(out, o64, vm, what=""):
    out = out.cpu().double()
    err = (out - o64).abs()
    tol = 2.0 ** -8 * (o64.abs() + vm)
    bad = ~(err <= tol)  # NaN (an element never written) counts as outside
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} elements outside 2^-8 (|ref| + max|V|); "
        f"worst excess {float((err - tol).max()):.3e}")


def _combined_cache(w):
    """A single cache holding the main cache's pages then the extra cache's
    (same page size), and the index rows that address it."""
    assert w.k_cache.shape[1] == w.extra_k_cache.shape[1]
    cache = torch.cat([w.k_cache, w.extra_k_cache], 0)
    offset = w.k_cache.shape[0] * w.k_cache.shape[1]
    B, SQ = w.q.shape[:2]
    rows = []
    for b in range(B):
        n0 = w.indices.shape[-1] if w.topk_length is None else int(w.topk_length[b])
        n1 = w.extra_indices.shape[-1] if w.extra_topk_length is None else int(w.extra_topk_length[b])
        r = torch.cat([w.indices[b, :, :n0], w.extra_indices[b, :, :n1] + offset], -1)
        rows.append(r)
    width = max(r.shape[-1] for r in rows)
    width = (width + 63) // 64 * 64
    idx = torch.full((B, SQ, width), -1, dtype=torch.int32)
    lens = torch.zeros(B, dtype=torch.int32)
    for b, r in enumerate(rows):
        idx[b, :, :r.shape[-1]] = r
        lens[b] = r.shape[-1]
    return cache, idx, lens


# ------------------------------------------------------- oracle pins ----

def test_oracle_rows_match_the_gather_oracle():
    """The decode oracle's dequantised rows are the rows the (separately
    pinned) dequantize_and_gather oracle produces from the same pages."""
    g = torch.Generator().manual_seed(1)
    cache = W.make_model1_cache(6, 64, g)
    out = torch.zeros(1, 6 * 64, 512, dtype=torch.bfloat16)
    oracle.dequantize_and_gather_k_cache(out, cache.view(6, -1), torch.tensor([6 * 64], dtype=torch.int32),
                                         None, torch.arange(6, dtype=torch.int32)[None], 64)
    for tid in range(0, 6 * 64, 11):
        assert torch.equal(oracle.model1_token_row(cache, tid), out[0, tid])
    assert torch.equal(torch_ref.model1_rows(cache), out[0])


def test_oracle_single_entry_is_that_entry():
    """One attended entry: softmax weight 1, so out = its V row exactly and
    lse = its score; n copies of it: same out, lse + ln(n)."""
    w = W.make_mla_workload(batch=2, topk=64, num_pages=4, sink=False, topk_length=False, seed=3)
    w.indices[:, :, :] = -1
    w.indices[0, 0, 0] = 77
    w.indices[1, 0, :8] = 130
    o64, l64 = _oracle(w)
    r77 = oracle.model1_token_row(w.k_cache, 77).double()
    r130 = oracle.model1_token_row(w.k_cache, 130).double()
    assert torch.equal(o64[0, 0], r77.expand(64, 512))
    assert torch.allclose(o64[1, 0], r130.expand(64, 512), rtol=1e-14, atol=1e-15)
    w.indices[1, 0, 1:8] = -1
    _, l1 = _oracle(w)
    assert torch.allclose(l64[1] - l1[1], torch.full_like(l1[1], math.log(8)), rtol=0, atol=1e-12)
    w.indices[:, :, :] = -1
    o0, l0 = _oracle(w)
    assert bool((o0 == 0).all()) and bool(torch.isinf(l0).all()) and bool((l0 > 0).all())


def test_oracle_sink_limits_and_half_weight():
    """sink = -inf is no sink; sink = +inf zeroes the output; sink = lse gives
    the sink the same weight as all entries together, halving the output."""
    w = W.make_mla_workload(batch=3, topk=128, num_pages=8, seed=5)
    o_none, l_none = _oracle(W.MlaWorkload(**{**w.__dict__, "attn_sink": None}))
    w.attn_sink = torch.full((64,), -math.inf)
    o_minus, l_minus = _oracle(w)
    assert torch.equal(o_minus, o_none) and torch.equal(l_minus, l_none)
    w.attn_sink = torch.full((64,), math.inf)
    o_plus, l_plus = _oracle(w)
    assert bool((o_plus == 0).all()) and torch.equal(l_plus, l_none)
    w.attn_sink = l_none[0, :, 0].float()  # batch row 0's lse per head
    o_half, _ = _oracle(w)
    assert torch.allclose(o_half[0], o_none[0] / 2, rtol=1e-6, atol=1e-12)


def test_oracle_extra_cache_is_a_second_list():
    """Attending a main and an extra list equals attending their union from
    one cache that holds both (invariance of the split), and permuting a
    row's entries changes nothing."""
    w = W.make_mla_workload(batch=4, topk=128, num_pages=6, extra_topk=192, extra_page=64,
                            extra_pages=5, seed=7)
    o_split, l_split = _oracle(w)
    cache, idx, lens = _combined_cache(w)
    o_one, l_one = oracle.sparse_mla_decode_model1(w.q, cache, idx, topk_length=lens,
                                                   attn_sink=w.attn_sink)
    assert torch.allclose(o_split, o_one, rtol=1e-12, atol=1e-14)
    assert torch.allclose(l_split, l_one, rtol=1e-13, atol=0)
    perm = torch.randperm(idx.shape[-1], generator=torch.Generator().manual_seed(0))
    full = W.MlaWorkload("p", w.q, cache, idx[:, :, perm], None, w.attn_sink)
    # without lengths, the -1 padding is what drops entries
    o_perm, _ = _oracle(full)
    assert torch.allclose(o_perm, o_one, rtol=1e-12, atol=1e-14)


def test_oracle_ignores_invalid_entries():
    """Entries past the top-k length, negative ids and ids past the cache are
    not attended: the result equals that of the row with them removed."""
    w = W.make_mla_workload(batch=2, topk=64, num_pages=4, topk_length=False, seed=9)
    o_ref, l_ref = _oracle(w)
    noisy = W.MlaWorkload("n", w.q, w.k_cache, torch.full((2, 1, 192), -1, dtype=torch.int32),
                          torch.tensor([150, 192], dtype=torch.int32), w.attn_sink)
    noisy.indices[:, :, 0:128:2] = w.indices            # valid entries at even slots
    noisy.indices[:, :, 1:128:2] = 4 * 64 + 5            # one past the cache
    noisy.indices[0, 0, 150:] = 3                        # past row 0's length
    o_n, l_n = _oracle(noisy)
    assert torch.allclose(o_n, o_ref, rtol=1e-12, atol=1e-14)
    assert torch.allclose(l_n, l_ref, rtol=1e-13, atol=0)


def test_oracle_against_direct_softmax():
    """Brute force on a tiny case: softmax over the attended rows with
    torch's float64 softmax and logsumexp (rows dequantised by torch's own
    float8 cast)."""
    w = W.make_mla_workload(batch=3, topk=64, num_pages=2, page=64, heads=64, seed=11)
    o64, l64 = _oracle(w)
    rows = _attended(w)
    scale = 512 ** -0.5
    for b in range(3):
        kv = rows[(b, 0)].double()
        s = (w.q[b, 0].double() @ kv.T) * scale
        lse = torch.logsumexp(s, -1)
        wts = torch.exp(s - lse[:, None])
        denom = 1 + torch.exp(w.attn_sink.double() - lse)
        assert torch.allclose(l64[b, :, 0], lse, rtol=1e-13, atol=0)
        assert torch.allclose(o64[b, 0], (wts @ kv) / denom[:, None], rtol=1e-10, atol=1e-14)


@pytest.mark.parametrize("case", ["ref_sink", "extra64", "extra2"])
def test_reference_algorithm_within_bound(case):
    """The reference's chunked bf16-P algorithm (torch restatement) stays
    inside the stated bound of the exact result: the bound is the one the
    reference's own arithmetic needs, not a loosening for the kernel."""
    w = _case(case)
    o64, l64 = _oracle(w)
    out, lse = torch_ref.sparse_mla_decode_model1(w.q, w.k_cache, w.indices, **_cpu_kwargs(w))
    _assert_within_bound(out, o64, _vmax(w), case)
    fin = torch.isfinite(l64)
    assert torch.allclose(lse.double()[fin], l64[fin], rtol=1e-5, atol=1e-5)


def _case(name):
    if name == "ref_sink":   # reference test :236-285
        return W.make_mla_workload(batch=8, topk=128, num_pages=16, seed=43)
    if name == "extra64":    # reference test :287-360, (64, 512, 12)
        return W.make_mla_workload(batch=4, topk=128, num_pages=16, extra_topk=512, extra_page=64,
                                   extra_pages=12, seed=43)
    if name == "extra2":     # (2, 512, 260)
        return W.make_mla_workload(batch=4, topk=128, num_pages=16, extra_topk=512, extra_page=2,
                                   extra_pages=260, seed=43)
    if name == "h128_sq2":
        return W.make_mla_workload(batch=5, topk=192, num_pages=8, heads=128, seq_q=2,
                                   topk_length=False, sink=False, seed=21)
    raise KeyError(name)


# ---------------------------------------------------- wrapper (CPU) ----

def _meta():
    from flaggems_vllm.ops.flash_mla_with_kvcache import get_mla_metadata

    return get_mla_metadata()[0]


def test_error_model1_extra_cache_requires_extra_indices():
    """Reference test :420-438."""
    import flaggems_vllm

    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 1, 64, 512).to(torch.bfloat16)
    kv = W.make_model1_cache(4, 64, g)
    extra = W.make_model1_cache(4, 64, g)
    idx = torch.randint(0, 256, (1, 1, 64), dtype=torch.int32)
    with pytest.raises(AssertionError, match="extra_indices_in_kvcache"):
        flaggems_vllm.flash_mla_with_kvcache(q, kv, None, None, 512, _meta(), is_fp8_kvcache=True,
                                             indices=idx, extra_k_cache=extra)


def test_error_dense_rejects_sparse_only_args():
    """Reference test :441-458."""
    import flaggems_vllm

    q = torch.randn(1, 1, 64, 576).to(torch.bfloat16)
    kv = torch.randn(4, 64, 1, 576).to(torch.bfloat16)
    bt = torch.arange(4, dtype=torch.int32).view(1, 4)
    seqlens = torch.full((1,), 64, dtype=torch.int32)
    with pytest.raises(AssertionError, match="must be None when dense"):
        flaggems_vllm.flash_mla_with_kvcache(q, kv, bt, seqlens, 512, _meta(),
                                             attn_sink=torch.randn(64))


def test_error_sched_meta_reuse_mismatch():
    """Reference test :461-484."""
    import flaggems_vllm
    from flaggems_vllm.ops.flash_mla_with_kvcache import FlashMLASchedMeta

    q = torch.empty(1, 1, 64, 512, dtype=torch.bfloat16)
    kv = torch.empty(4, 64, 1, 584, dtype=torch.uint8)
    meta = FlashMLASchedMeta(have_initialized=True, config=FlashMLASchedMeta.Config(
        b=2, s_q=1, h_q=64, page_block_size=64, h_k=1, causal=False, is_fp8_kvcache=True,
        topk=64, extra_page_block_size=None, extra_topk=None))
    with pytest.raises(AssertionError, match="sched_meta.config.b"):
        flaggems_vllm.flash_mla_with_kvcache(q, kv, None, None, 512, meta)


@pytest.mark.parametrize("bad,match", [
    (dict(topk=96), "divisible by 64"),
    (dict(heads=32), "h_q == 64 or 128"),
    (dict(v32_topk_length=True), "dynamic topk length"),
    (dict(cpu=True), "GPU"),
])
def test_wrapper_asserts(bad, match):
    import flaggems_vllm

    heads = bad.get("heads", 64)
    topk = bad.get("topk", 64)
    q = torch.zeros(1, 1, heads, 512, dtype=torch.bfloat16)
    kv = torch.zeros(2, 64, 1, 584, dtype=torch.uint8)
    idx = torch.zeros(1, 1, topk, dtype=torch.int32)
    kw = {}
    if bad.get("v32_topk_length"):
        q = torch.zeros(1, 1, 64, 576, dtype=torch.bfloat16)
        kv = torch.zeros(2, 64, 1, 656, dtype=torch.uint8)
        kw["topk_length"] = torch.ones(1, dtype=torch.int32)
    with pytest.raises(AssertionError, match=match):
        flaggems_vllm.flash_mla_with_kvcache(q, kv, None, None, 512, _meta(), is_fp8_kvcache=True,
                                             indices=idx, **kw)


def test_c_abi_rejects_bad_arguments():
    from flaggems_vllm import _native

    f = _native.lib().fgv_sparse_mla_decode_model1

    def call(**kw):
        a = dict(q=16, qs=(512 * 64, 512 * 64, 512), cache=16, bst=64 * 584, nb=4, page=64,
                 idx=16, topk=64, out=16, lse=16, B=1, SQ=1, H=64, ecache=None, eidx=None, elen=None,
                 ws=None, ws_bytes=0)
        a.update(kw)
        return f(a["q"], *a["qs"],
                 a["cache"], a["bst"], a["nb"], a["page"],
                 a["idx"], a["topk"], a["topk"], a["topk"], None,
                 a["ecache"], 64 * 584, 4, 64,
                 a["eidx"], a["topk"], a["topk"], a["topk"], a["elen"],
                 None, 0.05,
                 a["out"], 512 * 64, 512 * 64, 512,
                 a["lse"], 64, 1,
                 a["B"], a["SQ"], a["H"], a["ws"], a["ws_bytes"], None)

    assert call(H=96) == -2
    assert call(B=-1) == -2
    assert call(q=None) == -1
    assert call(q=8) == -3
    assert call(cache=8) == -3
    assert call(bst=64 * 584 - 16) == -4
    assert call(page=0) == -2
    assert call(eidx=16) == -2      # extra indices without an extra cache
    assert call(out=8) == -3        # output rows are written with 16-byte stores
    assert call(B=0) == 0           # nothing to do, nothing launched


def test_workspace_query():
    """The balanced split schedule is used for long lists only, and then needs
    two partial slots per workgroup of the grid plus the row prefix sums; an
    extra cache gathered at least 8 times per entry gets a bf16 copy of
    1 KiB per entry (at most 64 MiB)."""
    from flaggems_vllm import _native

    f = _native.lib().fgv_sparse_mla_decode_workspace_bytes
    grid = _native.lib().fgv_sparse_mla_decode_grid
    # (no GPU here: the CU count is taken as MI355X's 256)
    assert f(512, 1, 64, 128, 0, 0) == 0            # decode: one workgroup per item
    assert f(512, 1, 64, 128, 512, 0) == 0          # 20 chunks: still one per item
    assert f(512, 1, 64, 128, 8192, 0) == 0         # long lists, two items per CU: paired, not split
    big = f(200, 1, 64, 128, 8192, 0)               # long lists, at most one item per CU: split
    slot = (64 * 512 + 128) * 4
    prefix = (201 * 4 + 255) // 256 * 256
    assert big > 0 and (big - prefix) % (2 * slot) == 0 and big % 256 == 0
    assert f(600, 1, 64, 128, 8192, 0) > 0          # more than two per CU: split again
    assert f(9000, 1, 64, 128, 8192, 0) == 0        # prefix sums must fit in LDS
    assert f(0, 1, 64, 128, 8192, 0) == 0
    # the benchmark's extra caches: 512 rows x 512 over 32768 entries is 8 per entry
    assert f(512, 1, 64, 128, 512, 32768) == 32768 * 1024
    assert f(511, 1, 64, 128, 512, 32768) == 0      # just below 8 per entry
    assert f(256, 1, 128, 128, 512, 32768) == 32768 * 1024   # two head blocks gather twice
    assert f(256, 2, 64, 128, 512, 32768) == 32768 * 1024    # so do two query positions
    assert f(200, 1, 64, 128, 8192, 1024) == big + 1024 * 1024
    assert f(200, 1, 64, 128, 8192, 65537) == big   # a copy above 64 MiB is not made
    # the grid each size runs: 0 one item per workgroup, 1 split, 2 paired
    assert grid(512, 1, 64, 128, 0) == 0            # the benchmark's decode case
    assert grid(512, 1, 64, 128, 512) == 0          # and its extra512 case
    assert grid(512, 1, 64, 128, 8192) == 2         # and its extra8192 case
    assert grid(257, 1, 64, 2048, 0) == 2           # long lists, 257..512 items
    assert grid(100, 2, 128, 2048, 0) == 2          # 400 items
    assert grid(256, 1, 64, 2048, 0) == 1           # at most one item per CU: split
    assert grid(200, 1, 64, 128, 8192) == 1
    assert grid(600, 1, 64, 128, 8192) == 1         # more than two per CU: split
    assert grid(300, 1, 64, 128, 1888) == 0         # 4 + 59 chunks: short lists
    assert grid(300, 1, 64, 128, 1920) == 2         # 4 + 60: long
    assert grid(9000, 1, 64, 128, 8192) == 0
    assert grid(8, 1, 60, 128, 0) == -1             # heads not a multiple of 64


# --------------------------------------------------------------- GPU ----

def _gpu(w, out=None, q=None):
    import flaggems_vllm

    d = w.to(DEV)
    res = flaggems_vllm.flash_mla_with_kvcache(
        d.q if q is None else q, d.k_cache, None, None, 512, _meta(), is_fp8_kvcache=True,
        indices=d.indices, out=out, **d.kwargs())
    torch.cuda.synchronize()
    return res


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["ref_sink", "extra64", "extra2", "h128_sq2"])
def test_gpu_reference_cases(case):
    print(f"\n[case] sparse MLA {case}", flush=True)
    w = _case(case)
    out, lse = _gpu(w)
    o64, l64 = _oracle(w)
    _assert_within_bound(out, o64, _vmax(w), case)
    fin = torch.isfinite(l64)
    assert torch.equal(torch.isfinite(lse.cpu()), fin)
    assert torch.allclose(lse.cpu().double()[fin], l64[fin], rtol=1e-5, atol=1e-5)
    # the reference's own acceptance check (cosine similarity > 0.98)
    cos = torch.nn.functional.cosine_similarity(out.cpu().double().flatten(), o64.flatten(), dim=0)
    assert float(cos) > 0.999
    # and against the reference's algorithm restated in torch
    emu, _ = torch_ref.sparse_mla_decode_model1(w.q, w.k_cache, w.indices, **_cpu_kwargs(w))
    diff = (out.cpu().double() - emu.double()).abs()
    tol = 2.0 ** -8 * emu.double().abs() + 2.0 ** -10 * _vmax(w)
    assert bool((diff <= tol).all()), float((diff - tol).max())


@pytest.mark.gpu
def test_gpu_single_and_repeated_entry_bit_exact():
    """One attended entry, or 64 copies of one (weights 1 and 1/64, exact in
    binary floating point), give that entry's bf16 V row bit for bit, with no
    sink; the LSE is its score (plus ln 64)."""
    print("\n[case] sparse MLA single/repeated entry", flush=True)
    w = W.make_mla_workload(batch=4, topk=128, num_pages=8, sink=False, seed=13)
    w.topk_length = torch.tensor([1, 64, 128, 0], dtype=torch.int32)
    w.indices[1, 0, :64] = 300
    w.indices[2, 0, :] = -1
    w.indices[2, 0, 100] = 511
    out, lse = _gpu(w)
    out = out.cpu()
    assert torch.equal(out[0, 0], oracle.model1_token_row(w.k_cache, int(w.indices[0, 0, 0])).expand(64, 512))
    assert torch.equal(out[1, 0], oracle.model1_token_row(w.k_cache, 300).expand(64, 512))
    assert torch.equal(out[2, 0], oracle.model1_token_row(w.k_cache, 511).expand(64, 512))
    assert bool((out[3] == 0).all())
    lse = lse.cpu()
    assert bool(torch.isinf(lse[3]).all()) and bool((lse[3] > 0).all())
    _, l64 = _oracle(w)
    assert torch.allclose(lse[:3].double(), l64[:3], rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
def test_gpu_invalid_entries_and_strided_views():
    """Negative ids, ids past the cache, lengths past top-k, a row with only
    invalid entries before its valid ones, and strided q / out views."""
    print("\n[case] sparse MLA invalid entries + strided", flush=True)
    w = W.make_mla_workload(batch=6, topk=256, num_pages=8, seed=17)
    w.indices[0, 0, ::3] = -1
    w.indices[1, 0, 1::2] = 8 * 64 + 3      # past the cache
    w.indices[2, 0, :64] = -5               # the first two chunks attend nothing
    w.topk_length[3] = 1000                 # clamped to top-k
    w.topk_length[4] = -3                   # nothing attended
    qbig = torch.zeros(6, 1, 64, 1024, dtype=torch.bfloat16)
    qbig[..., 256:768] = w.q
    qv = qbig.to(DEV)[..., 256:768]
    obuf = torch.full((6, 1, 64, 640), 7.0, dtype=torch.bfloat16, device=DEV)
    out, lse = _gpu(w, out=obuf[..., 64:576], q=qv)
    o64, l64 = _oracle(w)
    _assert_within_bound(out, o64, _vmax(w), "invalid/strided")
    assert bool((obuf[..., :64] == 7).all()) and bool((obuf[..., 576:] == 7).all())
    assert bool((out[4].cpu() == 0).all()) and bool(torch.isinf(lse[4]).all())


@pytest.mark.gpu
def test_gpu_extreme_scales():
    """Scale bytes across the representable range (tiny and large powers of
    two, and byte 0 = scale 0): the dequantised rows stay exact, so the
    single-entry output is still the bf16 row."""
    print("\n[case] sparse MLA extreme scales", flush=True)
    w = W.make_mla_workload(batch=7, topk=64, num_pages=2, sink=False, seed=19)
    page_bytes = w.k_cache.view(2, -1)
    scl = page_bytes[:, 64 * 576:].view(2, 64, 8)
    choices = torch.tensor([0, 1, 20, 100, 127, 150, 140], dtype=torch.uint8)
    for i in range(7):
        scl[0, i, :7] = choices[i]
    w.topk_length = torch.ones(7, dtype=torch.int32)
    w.indices[:, 0, 0] = torch.arange(7, dtype=torch.int32)
    out, _ = _gpu(w)
    out = out.cpu()
    for i in range(7):
        row = oracle.model1_token_row(w.k_cache, i)
        assert torch.equal(out[i, 0], row.expand(64, 512)), int(choices[i])


_FINITE_E4M3 = [c for c in range(256) if c not in (0x7F, 0xFF)]


def _scale_sweep_cache(finite_rows_only):
    """A [4, 64, 1, 584] MODEL1 cache whose entry b (b = 0..254) has all seven
    scale bytes b and NoPE codes cycling through the 254 finite e4m3 codes
    (starting at code index 7b, so each code meets every group); entry 255
    repeats byte 127.  With finite_rows_only, codes whose dequantised value
    overflows bf16 (bytes 247..254 only) are replaced by the finite-valued
    codes in turn, so every row is finite and attention over it stays finite.
    RoPE bytes are seeded bf16 N(0, 0.1)."""
    g = torch.Generator().manual_seed(41)
    cache = W.make_model1_cache(4, 64, g)
    pages = cache.view(4, -1)
    data = pages[:, :64 * 576].view(4, 64, 576)   # views into the cache
    scl = pages[:, 64 * 576:].view(4, 64, 8)
    for b in range(256):
        byte = b if b < 255 else 127
        scl[b // 64, b % 64, :7] = byte
        codes = [_FINITE_E4M3[(7 * b + i) % 254] for i in range(448)]
        if finite_rows_only:
            ok = [c for c in _FINITE_E4M3
                  if torch.isfinite(oracle.e4m3fn_decode(torch.tensor([c], dtype=torch.uint8)).double()
                                    * 2.0 ** (byte - 127)).all()
                  and abs(float(oracle.e4m3fn_decode(torch.tensor([c], dtype=torch.uint8)))) * 2.0 ** (byte - 127)
                  < 3.3895e38]
            codes = [c if c in ok else ok[i % len(ok)] for i, c in enumerate(codes)]
        data[b // 64, b % 64, :448] = torch.tensor(codes, dtype=torch.uint8)
    return cache


def test_scale_sweep_cache_rows():
    """The sweep cache's rows (oracle dequantisation): every byte 0..254 and
    all 254 finite codes occur in every entry; with finite_rows_only every row
    is finite, without it bytes 247..254 hold infinite values."""
    full = _scale_sweep_cache(False)
    fin = _scale_sweep_cache(True)
    for b in range(255):
        codes = set(full.view(4, -1)[b // 64, (b % 64) * 576:(b % 64) * 576 + 448].tolist())
        assert codes == set(_FINITE_E4M3)
        assert bool(torch.isfinite(oracle.model1_token_row(fin, b).float()).all())
        assert bool(torch.isfinite(oracle.model1_token_row(full, b).float()).all()) == (b < 247)


@pytest.mark.gpu
def test_gpu_scaled_dequant_every_scale_byte():
    """v_cvt_scalef32_pk_bf16_fp8 in the chunk loop, for every scale byte
    0..254 and every finite code: batch row b attends entry b alone
    (topk_length 1, no sink), so its softmax weight is exactly 1 and every
    head's output is that entry's bf16 row, which must equal the oracle's
    bf16(f32(code) * 2^(byte - 127)) (byte 0: scale 0) bit for bit.  q row b
    is scaled down for large bytes so the score stays finite in fp32.  The
    sign of zero is not compared: the output is the fp32 sum 0 + 1 * V, in
    which a -0 of V becomes +0, as in the reference's accumulation."""
    print("\n[case] sparse MLA scaled dequant, scale bytes 0..254", flush=True)
    cache = _scale_sweep_cache(True)
    g = torch.Generator().manual_seed(42)
    B = 255
    q = torch.randn(B, 1, 64, 512, generator=g)
    for b in range(B):
        q[b] *= 2.0 ** -max(0, b - 200)
    idx = torch.randint(0, 256, (B, 1, 64), generator=g, dtype=torch.int32)
    idx[:, 0, 0] = torch.arange(B, dtype=torch.int32)
    w = W.MlaWorkload("scale sweep", q.to(torch.bfloat16), cache, idx,
                      torch.ones(B, dtype=torch.int32), None)
    out, lse = _gpu(w)
    out = out.cpu()
    bad, detail = [], ""
    for b in range(B):
        row = oracle.model1_token_row(cache, b)
        zero_as_pos = lambda x: torch.where((x & 0x7FFF) == 0, torch.zeros_like(x), x)
        got = zero_as_pos(out[b, 0].view(torch.int16))
        want = zero_as_pos(row.expand(64, 512).view(torch.int16))
        if not torch.equal(got, want):
            if not bad:
                diff = torch.nonzero(got != want)
                detail = "; first byte's differences (head, dim, gpu bits, oracle bits): " + ", ".join(
                    f"({h}, {d}, {int(got[h, d]) & 0xFFFF:#06x}, {int(want[h, d]) & 0xFFFF:#06x})"
                    for h, d in diff[:12].tolist()) + f" of {diff.shape[0]}"
            bad.append(b)
    assert not bad, f"{len(bad)} scale bytes whose attended row differs from the oracle's: {bad}{detail}"


@pytest.mark.gpu
def test_gpu_expanded_copy_every_scale_byte():
    """The expanded-cache copy (mla_expand_cache_kernel, the conversion the
    chunk loop uses, scale byte 0 included) for every scale byte 0..254 and
    every finite code, overflowing ones included: the bf16 rows it leaves at
    the start of the workspace equal the oracle's rows bit for bit (values
    past the bf16 maximum become +-inf in both)."""
    print("\n[case] sparse MLA expanded copy, scale bytes 0..254", flush=True)
    w = W.make_mla_workload(batch=8, topk=64, num_pages=2, sink=False, seed=43)
    w.extra_k_cache = _scale_sweep_cache(False)
    g = torch.Generator().manual_seed(44)
    w.extra_indices = torch.randint(0, 256, (8, 1, 256), generator=g, dtype=torch.int32)
    # 8 rows x 256 extra entries gather the 256-entry cache 8 times: expanded
    _, _, nbytes, ws = _gpu_raw(w, workspace=True, keep_ws=True)
    assert nbytes >= 256 * 1024
    rows = ws[:256 * 1024].cpu().view(torch.bfloat16).view(256, 512)
    bad = [b for b in range(256)
           if not torch.equal(rows[b].view(torch.int16),
                              oracle.model1_token_row(w.extra_k_cache, b).view(torch.int16))]
    assert not bad, f"expanded rows that differ from the oracle's: {bad[:16]}"


@pytest.mark.gpu
@pytest.mark.parametrize("pages", [4095, 4096, 4097])
def test_gpu_expanded_copy_sizes(pages):
    """The expanded copy around 8192 entries, where its workgroups go from two
    entries per half-wave to four (pages of 2: 8190, 8192 and 8194 entries, the
    last with a partial workgroup): every row equals the oracle's bit for bit."""
    print(f"\n[case] sparse MLA expanded copy, {2 * pages} entries", flush=True)
    w = W.make_mla_workload(batch=16, topk=64, num_pages=2, extra_topk=4200, extra_page=2, extra_pages=pages,
                            sink=False, seed=91, q_scale=0.1)
    entries = 2 * pages
    # 16 rows x 4200 extra entries gather the cache more than 8 times per entry: expanded
    _, _, nbytes, ws = _gpu_raw(w, workspace=True, keep_ws=True)
    assert nbytes >= entries * 1024
    rows = ws[:entries * 1024].cpu().view(torch.int16).view(entries, 512)
    bad = [e for e in range(entries)
           if not torch.equal(rows[e], oracle.model1_token_row(w.extra_k_cache, e).view(torch.int16))]
    assert not bad, f"expanded rows that differ from the oracle's: {bad[:16]}"


@pytest.mark.gpu
def test_gpu_bench_case_against_oracle():
    """The benchmark's decode case at full size (batch 512, top-k 128 over 512
    pages, sink, top-k lengths)."""
    print("\n[case] sparse MLA bench decode case", flush=True)
    w = W.make_mla_case("decode")
    out, lse = _gpu(w)
    o64, l64 = _oracle(w)
    _assert_within_bound(out, o64, _vmax(w), "decode")
    assert torch.allclose(lse.cpu().double(), l64, rtol=1e-5, atol=1e-5)


def _rows_of(w, rows):
    """The workload restricted to batch rows `rows` (same caches)."""
    pick = lambda t: None if t is None else t[rows]
    return W.MlaWorkload(w.name, w.q[rows], w.k_cache, w.indices[rows], pick(w.topk_length), w.attn_sink,
                         w.extra_k_cache, pick(w.extra_indices), pick(w.extra_topk_length))


def _sampled_rows(w, n, seed):
    """n batch rows: the first and last 8, the 16 with the longest lists (main
    plus extra), the rest drawn at random."""
    B = w.q.shape[0]
    total = torch.zeros(B, dtype=torch.long)
    for idx, length in ((w.indices, w.topk_length), (w.extra_indices, w.extra_topk_length)):
        if idx is not None:
            total += (torch.full((B,), idx.shape[-1]) if length is None
                      else length.long().clamp(0, idx.shape[-1]))
    chosen = list(range(8)) + list(range(B - 8, B)) + total.argsort(descending=True)[:16].tolist()
    rest = [r for r in torch.randperm(B, generator=torch.Generator().manual_seed(seed)).tolist()
            if r not in chosen]
    chosen = sorted(set(chosen)) + rest
    return torch.tensor(sorted(chosen[:n]))


@pytest.mark.gpu
@pytest.mark.parametrize("case,grid,rows", [("extra512", 0, None), ("extra8192", 2, 160)])
def test_gpu_bench_extra_cases_against_oracle(case, grid, rows):
    """The benchmark's two extra-cache cases at full size, through the wrapper
    exactly as bench.py times them (its workspace holds the expanded bf16 copy
    of the extra cache): extra512 on the one-item grid, extra8192 on the paired
    grid.  extra512 is compared with the binary64 oracle on every batch row,
    extra8192 on `rows` sampled rows; every output element is finite."""
    from flaggems_vllm import _native

    print(f"\n[case] sparse MLA bench {case} case", flush=True)
    w = W.make_mla_case(case)
    B, SQ, HQ, _ = w.q.shape
    entries = w.extra_k_cache.shape[0] * w.extra_k_cache.shape[1]
    assert _grid(w) == grid, f"{case} must take grid {grid}"
    need = _native.lib().fgv_sparse_mla_decode_workspace_bytes(B, SQ, HQ, w.indices.shape[-1],
                                                               w.extra_indices.shape[-1], entries)
    assert need == entries * 1024, "the extra cache must be expanded, with no split partials"
    out, lse = _gpu(w)
    out, lse = out.cpu(), lse.cpu()
    assert bool(torch.isfinite(out.float()).all())
    sel = torch.arange(B) if rows is None else _sampled_rows(w, rows, seed=17)
    sub = _rows_of(w, sel)
    o64, l64 = _oracle(sub)
    _assert_within_bound(out[sel], o64, _vmax(sub), case)
    assert torch.allclose(lse[sel].double(), l64, rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
def test_gpu_deterministic():
    print("\n[case] sparse MLA determinism", flush=True)
    w = _case("extra64")
    a, la = _gpu(w)
    b, lb = _gpu(w)
    assert torch.equal(a, b) and torch.equal(la, lb)


# ------------------------------------------------------- GPU: split grid ----

def _gpu_raw(w, workspace, ws_bytes=None, keep_ws=False):
    """Calls the C ABI directly, with or without a workspace (of the queried
    size, or `ws_bytes`); with keep_ws the workspace tensor is returned too.
    out and lse start as NaN, so an element the call never writes fails the
    bound."""
    from flaggems_vllm import _native

    d = w.to(DEV)
    B, SQ, HQ, _ = d.q.shape
    out = torch.full((B, SQ, HQ, 512), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse = torch.full((B, HQ, SQ), float("nan"), dtype=torch.float32, device=DEV)
    L = _native.lib()
    etopk = d.extra_indices.shape[-1] if d.extra_indices is not None else 0
    ek, ei = d.extra_k_cache, d.extra_indices
    entries = ek.shape[0] * ek.shape[1] if ek is not None else 0
    nbytes = L.fgv_sparse_mla_decode_workspace_bytes(B, SQ, HQ, d.indices.shape[-1], etopk, entries)
    if ws_bytes is not None:
        nbytes = ws_bytes
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=DEV) if workspace else None
    ptr = lambda t: t.data_ptr() if t is not None else None
    rc = L.fgv_sparse_mla_decode_model1(
        d.q.data_ptr(), d.q.stride(0), d.q.stride(1), d.q.stride(2),
        d.k_cache.data_ptr(), d.k_cache.stride(0), d.k_cache.shape[0], d.k_cache.shape[1],
        d.indices.data_ptr(), d.indices.stride(0), d.indices.stride(1), d.indices.shape[-1],
        ptr(d.topk_length),
        ptr(ek), ek.stride(0) if ek is not None else 0, ek.shape[0] if ek is not None else 0,
        ek.shape[1] if ek is not None else 1,
        ptr(ei), ei.stride(0) if ei is not None else 0, ei.stride(1) if ei is not None else 0, etopk,
        ptr(d.extra_topk_length), ptr(d.attn_sink), 512 ** -0.5,
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        lse.data_ptr(), lse.stride(0), lse.stride(1), B, SQ, HQ,
        ptr(ws), nbytes if workspace else 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    if keep_ws:
        return out.cpu(), lse.cpu(), nbytes, ws
    return out.cpu(), lse.cpu(), nbytes


def _split_case(name):
    if name == "long":        # like the benchmark's extra8192 case, 24 rows
        return W.make_mla_workload(batch=24, topk=128, num_pages=64, extra_topk=8192, extra_page=2,
                                   extra_pages=512, seed=31, q_scale=0.1)
    if name == "edges":       # empty rows, 128 heads, two query positions
        w = W.make_mla_workload(batch=5, topk=2048, num_pages=40, heads=128, seq_q=2, seed=33)
        w.topk_length = torch.tensor([0, 2048, 1, 0, 1500], dtype=torch.int32)
        return w
    if name == "tiny":        # fewer chunks than workgroups: most split ranges are empty
        w = W.make_mla_workload(batch=3, topk=2048, num_pages=40, seed=35)
        w.topk_length = torch.tensor([5, 0, 40], dtype=torch.int32)
        return w
    raise KeyError(name)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["long", "edges", "tiny"])
def test_gpu_split_grid_against_oracle(case):
    print(f"\n[case] sparse MLA split grid {case}", flush=True)
    w = _split_case(case)
    out, lse, nbytes = _gpu_raw(w, workspace=True)
    assert nbytes > 0, "the case must take the split path"
    o64, l64 = _oracle(w)
    _assert_within_bound(out, o64, _vmax(w), case)
    fin = torch.isfinite(l64)
    assert torch.equal(torch.isfinite(lse), fin)
    assert torch.allclose(lse.double()[fin], l64[fin], rtol=1e-5, atol=1e-5)
    # the same call without a workspace (the paired grid) agrees
    out1, lse1, _ = _gpu_raw(w, workspace=False)
    _assert_within_bound(out1, o64, _vmax(w), case + " unsplit")
    assert torch.allclose(lse1.double()[fin], lse.double()[fin], rtol=1e-6, atol=1e-6)


# ------------------------------------------------- GPU: expanded extra cache ----

def _expanded_case(heads=64, seq_q=1):
    """An extra cache of 256 entries gathered 16 x 512 times (32 per entry), with
    per-row lengths, repeated entries and entries that are not attended
    (negative, past the cache): short enough to stay unsplit."""
    w = W.make_mla_workload(batch=16, topk=64, num_pages=8, extra_topk=512, extra_page=64, extra_pages=4,
                            heads=heads, seq_q=seq_q, seed=41, q_scale=0.1)
    g = torch.Generator().manual_seed(7)
    ei = w.extra_indices.clone()
    flat = ei.view(-1)
    pick = torch.randperm(flat.numel(), generator=g)[:400]
    flat[pick[:200]] = -1
    flat[pick[200:300]] = 256 + torch.randint(0, 1000, (100,), generator=g, dtype=torch.int32)
    flat[pick[300:]] = 5  # a repeated entry
    w.extra_indices = ei
    return w


@pytest.mark.gpu
@pytest.mark.parametrize("heads,seq_q", [(64, 1), (128, 2)])
def test_gpu_expanded_extra_cache_bit_exact(heads, seq_q):
    """The extra cache dequantised once into bf16 rows gives the same bits as
    dequantising each gathered chunk: same K rows, same order of operations."""
    from flaggems_vllm import _native

    print(f"\n[case] sparse MLA expanded extra cache vs in-chunk dequantisation H={heads} SQ={seq_q}",
          flush=True)
    w = _expanded_case(heads, seq_q)
    B, SQ, HQ, _ = w.q.shape
    need = _native.lib().fgv_sparse_mla_decode_workspace_bytes(B, SQ, HQ, w.indices.shape[-1],
                                                               w.extra_indices.shape[-1], 256)
    assert need == 256 * 1024, "the case must take the expanded route and no split"
    out_x, lse_x, _ = _gpu_raw(w, workspace=True)
    out_d, lse_d, _ = _gpu_raw(w, workspace=False)
    assert torch.equal(out_x.view(torch.int16), out_d.view(torch.int16))
    assert torch.equal(lse_x, lse_d)
    o64, l64 = _oracle(w)
    _assert_within_bound(out_x, o64, _vmax(w), "expanded")


@pytest.mark.gpu
def test_gpu_split_grid_expanded_matches_split_alone():
    """The split schedule over an expanded extra cache (segments starting on
    even and odd extra chunks) gives the same bits as the split schedule with a
    workspace too small for the copy, which dequantises in the chunk loop."""
    from flaggems_vllm import _native

    print("\n[case] sparse MLA split grid, expanded vs not", flush=True)
    w = _split_case("long")
    B, SQ, HQ, _ = w.q.shape
    f = _native.lib().fgv_sparse_mla_decode_workspace_bytes
    entries = w.extra_k_cache.shape[0] * w.extra_k_cache.shape[1]
    split_only = f(B, SQ, HQ, w.indices.shape[-1], w.extra_indices.shape[-1], 0)
    both = f(B, SQ, HQ, w.indices.shape[-1], w.extra_indices.shape[-1], entries)
    assert both == split_only + entries * 1024 and split_only > 0
    out_x, lse_x, _ = _gpu_raw(w, workspace=True)
    out_s, lse_s, _ = _gpu_raw(w, workspace=True, ws_bytes=split_only)
    assert torch.equal(out_x.view(torch.int16), out_s.view(torch.int16))
    assert torch.equal(lse_x, lse_s)


# ------------------------------------------------------ GPU: paired grid ----

def _grid(w):
    from flaggems_vllm import _native

    B, SQ, HQ, _ = w.q.shape
    etopk = w.extra_indices.shape[-1] if w.extra_indices is not None else 0
    return _native.lib().fgv_sparse_mla_decode_grid(B, SQ, HQ, w.indices.shape[-1], etopk)


def _lengths(n, hi, seed):
    return torch.randint(0, hi + 1, (n,), generator=torch.Generator().manual_seed(seed), dtype=torch.int32)


def _pair_case(name):
    """Calls the paired grid takes (long lists, 256 CUs < items <= 512): the
    workgroups whose first item is among the shortest take a second one.  The
    lists' capacity (top-k) is long; most rows attend a few hundred entries
    and a few the whole list, so the binary64 oracle stays quick."""
    if name == "pairs":       # 300 items: 44 workgroups take a second item
        w = W.make_mla_workload(batch=300, topk=2048, num_pages=64, seed=51, q_scale=0.1)
        w.topk_length = _lengths(300, 160, 1)
        w.topk_length[::7] = 0       # rows that attend nothing
        w.topk_length[1::5] = 128    # many equal chunk counts (ties go by item index)
        w.topk_length[[3, 50, 299]] = torch.tensor([2048, 2000, 1999], dtype=torch.int32)
        return w
    if name == "full":        # 512 items: every workgroup takes two
        w = W.make_mla_workload(batch=512, topk=2048, num_pages=64, seed=53, q_scale=0.1)
        w.topk_length = _lengths(512, 256, 2)
        w.topk_length[[0, 255, 256, 511]] = 2048
        return w
    if name == "extra":       # an extra list, odd main chunk counts, empty extra rows
        w = W.make_mla_workload(batch=300, topk=128, num_pages=16, extra_topk=2048, extra_page=64,
                                extra_pages=16, seed=55, q_scale=0.1)
        w.extra_topk_length = _lengths(300, 300, 3)
        w.extra_topk_length[::9] = 0
        w.extra_topk_length[[7, 123]] = 2048
        return w
    if name == "h128_sq2":    # 100 rows x 2 query positions x 2 head blocks = 400 items
        w = W.make_mla_workload(batch=100, topk=2048, num_pages=32, heads=128, seq_q=2, seed=57,
                                q_scale=0.1)
        w.topk_length = _lengths(100, 200, 4)
        return w
    if name == "clamped":     # chunk counts past the 255 ordered exactly, and ties among them
        w = W.make_mla_workload(batch=260, topk=8192, num_pages=160, seed=59, q_scale=0.1)
        lens = _lengths(260, 96, 3)
        lens[[0, 40, 41, 200, 259]] = torch.tensor([8192, 8100, 8192, 8190, 8161], dtype=torch.int32)
        w.topk_length = lens
        return w
    raise KeyError(name)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["pairs", "full", "extra", "h128_sq2", "clamped"])
def test_gpu_pair_grid_against_oracle(case):
    print(f"\n[case] sparse MLA paired grid {case}", flush=True)
    w = _pair_case(case)
    assert _grid(w) == 2, "the case must take the paired grid"
    out, lse, _ = _gpu_raw(w, workspace=False)  # (the extra list dequantised per chunk)
    o64, l64 = _oracle(w)
    _assert_within_bound(out, o64, _vmax(w), case)
    fin = torch.isfinite(l64)
    assert torch.equal(torch.isfinite(lse), fin) and bool((lse[~fin] > 0).all())
    assert torch.allclose(lse.double()[fin], l64[fin], rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
def test_gpu_pair_grid_expanded_bit_exact():
    """Paired grid with the extra cache expanded once into bf16 rows (a
    workspace) and dequantised per chunk (none): the same bits, within the
    bound."""
    from flaggems_vllm import _native

    print("\n[case] sparse MLA paired grid, expanded vs not", flush=True)
    w = _pair_case("extra")
    B, SQ, HQ, _ = w.q.shape
    need = _native.lib().fgv_sparse_mla_decode_workspace_bytes(B, SQ, HQ, w.indices.shape[-1],
                                                               w.extra_indices.shape[-1], 1024)
    assert need == 1024 * 1024 and _grid(w) == 2
    out_x, lse_x, _ = _gpu_raw(w, workspace=True, ws_bytes=need)
    out_d, lse_d, _ = _gpu_raw(w, workspace=False)
    assert torch.equal(out_x.view(torch.int16), out_d.view(torch.int16))
    assert torch.equal(lse_x, lse_d)
    o64, _ = _oracle(w)
    _assert_within_bound(out_x, o64, _vmax(w), "paired expanded")


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["main", "expanded"])
def test_gpu_one_item_grid_against_oracle(case):
    """More than 512 items: one workgroup per item."""
    print(f"\n[case] sparse MLA one-item grid {case}", flush=True)
    if case == "main":
        w = W.make_mla_workload(batch=520, topk=64, num_pages=64, seed=61, q_scale=0.1)
    else:
        w = W.make_mla_workload(batch=520, topk=64, num_pages=16, extra_topk=128, extra_page=64, extra_pages=8,
                                seed=63, q_scale=0.1)
    assert _grid(w) == 0
    out, lse, nbytes = _gpu_raw(w, workspace=True)
    assert nbytes == (512 * 1024 if case == "expanded" else 0)
    o64, l64 = _oracle(w)
    _assert_within_bound(out, o64, _vmax(w), case)
    fin = torch.isfinite(l64)
    assert torch.equal(torch.isfinite(lse), fin)
    assert torch.allclose(lse.double()[fin], l64[fin], rtol=1e-5, atol=1e-5)


def _paired_order_case(name):
    """One-item grids of C < items <= 2C (C = CUs): workgroups j and C + j
    share a CU and the kernel ranks each window of 32 such pairs by list
    length, so the items land on other workgroups than their own."""
    if name == "partial":     # 300 items: a whole window, a window of 12 pairs, unpartnered workgroups
        w = W.make_mla_workload(batch=300, topk=256, num_pages=32, seed=71, q_scale=0.1)
        w.topk_length = _lengths(300, 256, 5)
        w.topk_length[::11] = 0
        w.topk_length[[4, 9, 260]] = torch.tensor([-3, 100000, 257], dtype=torch.int32)  # clamped
        return w
    if name == "h128_sq2":    # 100 rows x 2 query positions x 2 head blocks = 400 items
        w = W.make_mla_workload(batch=100, topk=128, num_pages=16, heads=128, seq_q=2, seed=73,
                                q_scale=0.1)
        w.topk_length = _lengths(100, 128, 6)
        return w
    if name == "no_lengths":  # 257 items, every list full: one pair, equal keys
        return W.make_mla_workload(batch=257, topk=64, num_pages=8, topk_length=False, seed=75, q_scale=0.1)
    if name in ("extra_fp8", "extra_expanded"):  # 480 items; extra chunks weigh 2 or 1
        w = W.make_mla_workload(batch=480, topk=64, num_pages=16, extra_topk=128, extra_page=64,
                                extra_pages=8, seed=77, q_scale=0.1)
        w.extra_topk_length = _lengths(480, 128, 7)
        w.extra_topk_length[::13] = 0
        return w
    raise KeyError(name)


def _check_item_order(w, case, ws, rounds):
    """The call against the oracle, and bit for bit against the same rows
    computed in calls of at most C items (C = CUs), which keep each item on
    the workgroup of its own index; `rounds` bounds items / C."""
    B, SQ, HQ, _ = w.q.shape
    items = B * SQ * (HQ // 64)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    lo, hi = rounds
    assert lo * cus < items <= hi * cus, "the case must take the order under test"
    assert _grid(w) == 0
    out, lse, nbytes = _gpu_raw(w, workspace=ws)
    if case == "extra_expanded":
        assert nbytes > 0, "the extra cache must be expanded"
    o64, l64 = _oracle(w)
    _assert_within_bound(out, o64, _vmax(w), case)
    fin = torch.isfinite(l64)
    assert torch.equal(torch.isfinite(lse), fin)
    assert torch.allclose(lse.double()[fin], l64[fin], rtol=1e-5, atol=1e-5)
    per_row = items // B
    step = cus // per_row
    for r0 in range(0, B, step):
        rows = torch.arange(r0, min(B, r0 + step))
        o_part, l_part, _ = _gpu_raw(_rows_of(w, rows), workspace=ws)
        assert torch.equal(out[rows].view(torch.int16), o_part.view(torch.int16)), f"rows from {r0}"
        assert torch.equal(lse[rows], l_part), f"rows from {r0}"


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["partial", "h128_sq2", "no_lengths", "extra_fp8", "extra_expanded"])
def test_gpu_paired_order_against_oracle(case):
    """One-item grids of C < items <= 2C: long items paired with short ones."""
    print(f"\n[case] sparse MLA one-item grid, paired order, {case}", flush=True)
    _check_item_order(_paired_order_case(case), case, case != "extra_fp8", (1, 2))


def _longest_first_case(name):
    """One-item grids of 2C < items <= 4C: each window of 256 workgroups takes
    its own items longest first."""
    if name == "partial":     # 600 items: two whole windows and one of 88
        w = W.make_mla_workload(batch=600, topk=128, num_pages=32, seed=81, q_scale=0.1)
        w.topk_length = _lengths(600, 128, 8)
        w.topk_length[::9] = 0
        w.topk_length[[5, 300, 599]] = torch.tensor([-1, 5000, 129], dtype=torch.int32)  # clamped
        return w
    if name == "h128":        # 300 rows x 2 head blocks = 600 items
        w = W.make_mla_workload(batch=300, topk=64, num_pages=16, heads=128, seed=83, q_scale=0.1)
        w.topk_length = _lengths(300, 64, 9)
        return w
    if name == "no_lengths":  # 513 items, every list full: equal keys
        return W.make_mla_workload(batch=513, topk=64, num_pages=8, topk_length=False, seed=85, q_scale=0.1)
    if name in ("extra_fp8", "extra_expanded"):  # 700 items; extra chunks weigh 2 or 1
        w = W.make_mla_workload(batch=700, topk=64, num_pages=16, extra_topk=128, extra_page=64,
                                extra_pages=8, seed=87, q_scale=0.1)
        w.extra_topk_length = _lengths(700, 128, 10)
        w.extra_topk_length[::7] = 0
        return w
    raise KeyError(name)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["partial", "h128", "no_lengths", "extra_fp8", "extra_expanded"])
def test_gpu_longest_first_order_against_oracle(case):
    print(f"\n[case] sparse MLA one-item grid, longest first, {case}", flush=True)
    _check_item_order(_longest_first_case(case), case, case != "extra_fp8", (2, 4))
