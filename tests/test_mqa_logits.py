"""Sparse-indexer logits: fp8_fp4_mqa_logits and fp8_fp4_paged_mqa_logits.

Reference ops: src/flaggems_vllm/ops/fp8_fp4_mqa_logits.py:88-358, 523-651 and
src/flaggems_vllm/ops/fp8_fp4_paged_mqa_logits.py:68-225, 410-579.  Reference
tests: tests/test_fp8_fp4_mqa_logits.py:152-221 (H = 64, D = 128, the decode and
prefill (M, N) shapes, clean on and off, FP8 and MXFP4 q; FP8 against vLLM's
DeepGEMM, MXFP4 against the float32 ``reference_fp4_mqa_logits``, atol 5e-2 /
0.15) and tests/test_fp8_fp4_paged_mqa_logits.py:29-263 (nine (batch, next_n,
context) shapes, 64-entry blocks, max_model_len 111 Ki).  vLLM is not
available here; the FP8 path is held to the same float32 formulation.

This is floating-point work, so parity is a bound, not bits: the C oracle
computes every logit in binary64 (the products of 4-bit significands and
their 128-term sums are exact) together with a rigorous error bound for a
binary32 implementation (oracle/dsv4_oracle.c, oracle_mqa_logits), and the
GPU result must lie within it.  Masked positions (-inf, or the paged fill)
are compared exactly.  The reference's own tolerance against its float32
formulation (oracle.torch_ref.mqa_logits) is checked as well.
"""
import ctypes
import inspect

import pytest
import torch

import flaggems_vllm
import oracle
from flaggems_vllm import _native
from flaggems_vllm import testing as W
from oracle import torch_ref

DEV = torch.device("cuda:0")
FP8 = torch.float8_e4m3fn


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _within(got, want, bound, what, slack=1.0):
    """got (float32) against the oracle's binary64 values: infinities equal,
    finite values within the bound."""
    got = got.double()
    inf = torch.isinf(want)
    assert torch.equal(torch.isinf(got), inf), f"{what}: -inf positions differ"
    assert torch.equal(got[inf], want[inf]), f"{what}: infinite values differ"
    err = (got[~inf] - want[~inf]).abs()
    lim = bound[~inf] * slack + 1e-30
    bad = err > lim
    ratio = float((err / lim).max()) if err.numel() else 0.0
    print(f"  {what}: max |err| {float(err.max()) if err.numel() else 0:.3e}, max err/bound {ratio:.3f}",
          flush=True)
    if bool(bad.any()):
        i = int(torch.nonzero(bad.flatten())[0])
        raise AssertionError(f"{what}: {int(bad.sum())} logits outside the bound; first flat index {i}: "
                             f"gpu {float(got[~inf][i])} oracle {float(want[~inf][i])} bound {float(lim[i])}")


def _sample_rows(M, n=12, seed=0):
    if M <= n:
        return torch.arange(M)
    g = torch.Generator().manual_seed(seed)
    r = torch.randperm(M, generator=g)[:n - 2]
    return torch.unique(torch.cat([r, torch.tensor([0, M - 1])]))


def _dev(q, kv, w, ks, ke):
    return ((q[0].to(DEV), q[1].to(DEV) if q[1] is not None else None), (kv[0].to(DEV), kv[1].to(DEV)),
            w.to(DEV), ks.to(DEV), ke.to(DEV))


# ------------------------------------------------------------------- CPU ----

def test_signatures_match_reference():
    p = inspect.signature(flaggems_vllm.fp8_fp4_mqa_logits).parameters
    assert list(p) == ["q", "kv", "weights", "cu_seqlen_ks", "cu_seqlen_ke", "clean_logits"]
    assert p["clean_logits"].default is True
    p = inspect.signature(flaggems_vllm.fp8_fp4_paged_mqa_logits).parameters
    assert list(p) == ["q", "kv_cache", "weights", "context_lens", "block_tables", "schedule_metadata",
                       "max_model_len", "clean_logits"]
    assert p["clean_logits"].default is False


def test_oracle_known_answers_fp8():
    """One-hot queries: head h has 2.0 at dim d_h, so its dot with key n is
    2 k[n, d_h]; the logit is sum_h ReLU(2 k[n, d_h] s_n) w_h.  Keys carry
    +-1.5 / 0 at those dims, so the ReLU gate, the weights and the scale can
    each be read off; clean_logits puts -inf outside [ks, ke)."""
    H, N = 16, 6
    q = torch.zeros(1, H, 128)
    dims = [7 * h + 3 for h in range(H)]
    for h in range(H):
        q[0, h, dims[h]] = 2.0
    k = torch.zeros(N, 128)
    k[0, dims[0]] = 1.5           # head 0 only, positive
    k[1, dims[1]] = -1.5          # head 1 only, negative: gated to 0
    k[2, dims[2]], k[2, dims[3]] = 1.5, 1.5
    k[3, dims[5]] = 448.0         # e4m3 maximum
    k[5, 100] = 1.0               # a dim no head reads
    s = torch.tensor([0.5, 0.25, 2.0, 2.0 ** -9, 1.0, 3.0])
    w = torch.arange(1, H + 1, dtype=torch.float32)[None, :] * 0.5
    w[0, 3] = -4.0
    out, bound = oracle.mqa_logits((q.to(FP8), None), (k.to(FP8), s), w, torch.tensor([1]), torch.tensor([5]), True)
    want = [float("-inf"), 0.0, 2 * 1.5 * 2.0 * 1.5 + 2 * 1.5 * 2.0 * (-4.0), 2 * 448 * 2.0 ** -9 * 3.0, 0.0,
            float("-inf")]
    assert out[0].tolist() == want
    out, _ = oracle.mqa_logits((q.to(FP8), None), (k.to(FP8), s), w, None, None, False)
    assert out[0, 0] == 2 * 1.5 * 0.5 * 0.5 and out[0, 5] == 0.0
    assert bool((bound >= 0).all())


def test_oracle_known_answers_mxfp4():
    """MXFP4 q: nibble code c at dim d decodes to E2M1(c) * 2^(byte_{d/32} - 127).
    Every code 0..15 in every 32-block with distinct scale bytes, read through
    one-hot keys."""
    H = 16
    mags = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    q = torch.zeros(1, H, 64, dtype=torch.uint8)
    scale = torch.zeros(1, H, dtype=torch.int64)
    expect = {}
    for h in range(H):
        d = 33 * (h % 4) + (h // 4)           # block (d // 32) = h % 4 for these dims
        code = h                               # codes 0..15 (8..15 negative)
        q[0, h, d // 2] = code << (4 * (d % 2))
        bytes_ = [127 - 3, 127 + 2, 127 + 5, 127 - 7]
        for b in range(4):
            scale[0, h] |= bytes_[b] << (8 * b)
        val = (-1.0 if code & 8 else 1.0) * mags[code & 7] * 2.0 ** (bytes_[d // 32] - 127)
        expect[h] = (d, val)
    scale = scale.to(torch.int32)
    N = H
    k = torch.zeros(N, 128)
    for h in range(H):
        k[h, expect[h][0]] = 1.0
    w = torch.ones(1, H)
    out, _ = oracle.mqa_logits((q, scale), (k.to(FP8), torch.ones(N)), w, None, None, False)
    for h in range(H):
        # key h hits dim d_h; heads sharing that dim contribute too
        want = sum(max(expect[h2][1], 0.0) for h2 in range(H) if expect[h2][0] == expect[h][0])
        assert out[0, h] == want, (h, float(out[0, h]), want)


@pytest.mark.parametrize("fp4", [False, True])
@pytest.mark.parametrize("clean", [True, False])
def test_reference_formulation_within_oracle_bound(fp4, clean):
    """The reference test's float32 formulation (a binary32 implementation of
    the same sum) lies within the oracle's bound, on the reference's inputs
    with causal windows."""
    M, N = 6, 300
    q, kv, w, ks, ke = W.make_mqa_logits_inputs(M, N, fp4=fp4, seed=3)
    ks = torch.tensor([0, 5, 17, 100, 0, 299], dtype=torch.int32)
    ke = torch.tensor([300, 40, 17, 250, 1, 300], dtype=torch.int32)
    out, bound = oracle.mqa_logits(q, kv, w, ks, ke, clean)
    ref = torch_ref.mqa_logits(q, kv, w, ks, ke, clean)
    _within(ref, out, bound, "torch float32 formulation")


def test_paged_oracle_matches_dense_on_gathered_keys():
    """A paged row equals the dense oracle on the keys its block table
    selects; positions past the context get the fill value."""
    q, cache, w, ctx, bt = W.make_paged_mqa_inputs(3, 2, 200, seed=4)
    mml = 400
    for clean in (False, True):
        out, bound = oracle.paged_mqa_logits(q, cache, w, ctx, bt, mml, clean)
        ref = torch_ref.paged_mqa_logits(q, cache, w, ctx, bt, mml, clean)
        _within(ref, out, bound, f"paged torch formulation clean={clean}")
        nblk, bs = cache.shape[0], cache.shape[1]
        flat = cache.reshape(nblk, -1)
        kdata = flat[:, :bs * 128].reshape(-1, 128)
        kscale = flat[:, bs * 128:].contiguous().view(torch.float32).reshape(-1)
        r = 3  # batch 1, second query
        c = int(ctx[1, 1])
        pos = torch.arange(c)
        idx = bt[1, pos // bs].long() * bs + pos % bs
        dense, _ = oracle.mqa_logits((q[0].reshape(6, 64, 128)[r:r + 1], None),
                                     (kdata[idx].view(FP8), kscale[idx]), w[r:r + 1], None, None, False)
        assert torch.equal(out[r, :c], dense[0])
        assert bool((out[r, c:] == (float("-inf") if clean else 0.0)).all())


def test_wrappers_refuse_cpu_tensors():
    q, kv, w, ks, ke = W.make_mqa_logits_inputs(2, 32)
    with pytest.raises(AssertionError):
        flaggems_vllm.fp8_fp4_mqa_logits(q, kv, w, ks, ke)
    q, cache, w, ctx, bt = W.make_paged_mqa_inputs(2, 1, 64)
    with pytest.raises(AssertionError):
        flaggems_vllm.fp8_fp4_paged_mqa_logits(q, cache, w, ctx, bt, None, 128)


def _call_dense(**kw):
    a = dict(q=256, qsm=64 * 128, qsh=128, qs=None, k=256, ksn=128, ksc=256, w=256, wsm=64, wsh=1, ks=256, ke=256,
             out=256, osm=64, M=2, N=64, H=64, D=128, clean=1)
    a.update(kw)
    return _native.lib().fgv_fp8_fp4_mqa_logits(
        a["q"], a["qsm"], a["qsh"], a["qs"], 0, 0, a["k"], a["ksn"], a["ksc"], a["w"], a["wsm"], a["wsh"],
        a["ks"], a["ke"], a["out"], a["osm"], a["M"], a["N"], a["H"], a["D"], a["clean"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(H=48), -2), (dict(D=256), -2), (dict(M=-1), -2), (dict(q=None), -1), (dict(ks=None), -1),
    (dict(q=264), -3), (dict(qsh=136), -3), (dict(ksn=72), -3),
])
def test_dense_c_abi_rejects_bad_arguments(kw, code):
    assert _call_dense(**kw) == code
    assert _native.lib().fgv_last_error()


def test_dense_c_abi_empty_and_unclean_calls():
    assert _call_dense(M=0, q=None) == 0
    assert _call_dense(N=0, k=None) == 0


def _call_paged(**kw):
    a = dict(q=256, qsr=64 * 128, qsh=128, kv=256, kvs=64 * 132, nblk=4, bs=64, hd=128, w=256, wsr=64, wsh=1,
             ctx=256, plen=1, bt=256, bts=4, maxb=4, ptab=1, out=256, osr=1024, rows=2, H=64, mml=1024, clean=0)
    a.update(kw)
    return _native.lib().fgv_fp8_fp4_paged_mqa_logits(
        a["q"], a["qsr"], a["qsh"], None, 0, 0, a["kv"], a["kvs"], a["nblk"], a["bs"], a["hd"], a["w"], a["wsr"],
        a["wsh"], a["ctx"], a["plen"], a["bt"], a["bts"], a["maxb"], a["ptab"], a["out"], a["osr"], a["rows"],
        a["H"], a["mml"], a["clean"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(H=8), -2), (dict(hd=64), -2), (dict(bs=0), -2), (dict(nblk=0), -2), (dict(plen=0), -2),
    (dict(rows=70000), -5), (dict(kv=None), -1), (dict(kvs=64 * 132 - 16), -4), (dict(kv=264), -3),
])
def test_paged_c_abi_rejects_bad_arguments(kw, code):
    assert _call_paged(**kw) == code
    assert _native.lib().fgv_last_error()


def test_paged_c_abi_empty_calls():
    assert _call_paged(rows=0, q=None) == 0
    assert _call_paged(mml=0) == 0


# ------------------------------------------------------------------- GPU ----

def _check_dense(q, kv, w, ks, ke, clean, rows=None, ref_atol=None):
    gq, gkv, gw, gks, gke = _dev(q, kv, w, ks, ke)
    got = flaggems_vllm.fp8_fp4_mqa_logits(gq, gkv, gw, gks, gke, clean_logits=clean)
    torch.cuda.synchronize()
    got = got.cpu()
    M = w.shape[0]
    rows = _sample_rows(M) if rows is None else rows
    want, bound = oracle.mqa_logits(q, kv, w, ks, ke, clean, rows=rows)
    _within(got[rows], want, bound, "gpu vs binary64 oracle")
    if ref_atol is not None:
        sub = (q[0][rows], q[1][rows] if q[1] is not None else None)
        ref = torch_ref.mqa_logits(sub, kv, w[rows], ks[rows], ke[rows], clean)
        torch.testing.assert_close(got[rows], ref, atol=ref_atol, rtol=1.3e-6, equal_nan=True)
    return got


@pytest.mark.gpu
@pytest.mark.parametrize("fp4", [False, True])
@pytest.mark.parametrize("clean", [True, False])
@pytest.mark.parametrize("shape", W.MQA_DECODE_SHAPES + W.MQA_PREFILL_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_gpu_reference_shapes(shape, clean, fp4):
    """The reference test's 10 (M, N) shapes x clean x {FP8, MXFP4}, H = 64,
    D = 128, its input distributions; sampled rows against the oracle bound
    and the reference's own tolerance."""
    M, N = shape
    _say(f"mqa logits M={M} N={N} clean={clean} fp4={fp4}")
    q, kv, w, ks, ke = W.make_mqa_logits_inputs(M, N, fp4=fp4)
    _check_dense(q, kv, w, ks, ke, clean, ref_atol=0.15 if fp4 else 5e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("fp4", [False, True])
def test_gpu_causal_windows(fp4):
    """Prefill with per-row windows [ks, ke) (causal, empty, single key,
    whole range): -inf outside exactly, every row checked; and clean_logits
    off computes the same finite values inside."""
    M, N = 200, 1000
    _say(f"mqa logits causal windows fp4={fp4}")
    q, kv, w, _, _ = W.make_mqa_logits_inputs(M, N, fp4=fp4, seed=5)
    g = torch.Generator().manual_seed(6)
    ks = torch.randint(0, 400, (M,), generator=g, dtype=torch.int32)
    ke = (ks + torch.randint(0, 700, (M,), generator=g, dtype=torch.int32)).clamp(max=N)
    ks[0], ke[0] = 0, 0          # empty
    ks[1], ke[1] = 999, 1000     # last key only
    ks[2], ke[2] = 0, N
    ks[3], ke[3] = 500, 400      # inverted: empty
    a = _check_dense(q, kv, w, ks, ke, True, rows=torch.arange(M))
    b = _check_dense(q, kv, w, ks, ke, False, rows=torch.arange(0, M, 7))
    inside = torch.isfinite(a)
    assert torch.equal(a[inside], b[inside])


@pytest.mark.gpu
@pytest.mark.parametrize("H", [16, 32, 128])
@pytest.mark.parametrize("fp4", [False, True])
def test_gpu_head_counts(H, fp4):
    _say(f"mqa logits H={H} fp4={fp4}")
    q, kv, w, ks, ke = W.make_mqa_logits_inputs(37, 333, H=H, fp4=fp4, seed=H)
    _check_dense(q, kv, w, ks, ke, True, rows=torch.arange(37))


@pytest.mark.gpu
@pytest.mark.parametrize("fp4", [False, True])
def test_gpu_zero_and_negative_k_scale(fp4):
    """The kernels apply k_scale once to the ReLU'd head sum, the reference
    inside each head's ReLU.  For k_scale = 0 both give 0 (pinned against the
    oracle, which follows the reference's order); for k_scale > 0 they agree;
    for k_scale < 0 (outside the op's stated precondition) the kernels return
    k_scale * sum_h w_h ReLU(dot_h), which is -(the oracle's logit at |k_scale|)."""
    _say(f"mqa logits k_scale zero and negative fp4={fp4}")
    M, N = 24, 200
    q, kv, w, ks, ke = W.make_mqa_logits_inputs(M, N, fp4=fp4, seed=9)
    k_scale = kv[1].reshape(N).clone()
    k_scale[::5] = 0.0
    k_scale[1::5] = -k_scale[1::5].abs()
    neg = k_scale < 0
    gq, gkv, gw, gks, gke = _dev(q, (kv[0], k_scale), w, ks, ke)
    got = flaggems_vllm.fp8_fp4_mqa_logits(gq, gkv, gw, gks, gke, clean_logits=True)
    torch.cuda.synchronize()
    got = got.cpu()
    rows = torch.arange(M)
    want, bound = oracle.mqa_logits(q, (kv[0], k_scale), w, ks, ke, True, rows=rows)
    _within(got[:, ~neg], want[:, ~neg], bound[:, ~neg], "k_scale >= 0 vs oracle")
    inside = torch.isfinite(want)
    assert bool((got[:, ::5][inside[:, ::5]] == 0).all()), "k_scale = 0 gives 0"
    want_abs, bound_abs = oracle.mqa_logits(q, (kv[0], k_scale.abs()), w, ks, ke, True, rows=rows)
    fin = torch.isfinite(want_abs[:, neg])
    _within(-got[:, neg][fin], want_abs[:, neg][fin], bound_abs[:, neg][fin], "k_scale < 0 (documented)")


@pytest.mark.gpu
def test_gpu_strided_inputs():
    """q and k as slices of wider buffers, weights transposed, k_scale [N, 1]."""
    _say("mqa logits strided inputs")
    M, N = 19, 150
    q, kv, w, ks, ke = W.make_mqa_logits_inputs(M, N, seed=8)
    qbuf = torch.zeros(M, 64, 160, dtype=torch.uint8)
    qbuf[:, :, 16:144] = q[0].view(torch.uint8)
    kbuf = torch.zeros(N, 176, dtype=torch.uint8)
    kbuf[:, 32:160] = kv[0].view(torch.uint8)
    wt = w.t().contiguous().t()
    want, bound = oracle.mqa_logits(q, kv, w, ks, ke, True)
    gq = qbuf.to(DEV)[:, :, 16:144].view(FP8)
    gk = kbuf.to(DEV)[:, 32:160].view(FP8)
    got = flaggems_vllm.fp8_fp4_mqa_logits((gq, None), (gk, kv[1].reshape(N, 1).to(DEV)), wt.to(DEV),
                                           ks.to(DEV), ke.to(DEV))
    torch.cuda.synchronize()
    _within(got.cpu(), want, bound, "strided")


@pytest.mark.gpu
def test_gpu_mxfp4_every_scale_byte():
    """The hardware block scales over UE8M0 bytes 20..200: each (row, head)
    uses four consecutive bytes, one per 32-element block, with q nibbles of
    every code; keys of magnitude >= 1 so no product is subnormal."""
    _say("mqa logits MXFP4 scale bytes 20..200")
    H, N = 16, 64
    nbytes = 200 - 20 + 1
    M = (nbytes + H - 1) // H
    g = torch.Generator().manual_seed(9)
    packed = torch.randint(0, 256, (M, H, 64), generator=g, dtype=torch.int32).to(torch.uint8)
    scale = torch.zeros(M, H, dtype=torch.int64)
    for m in range(M):
        for h in range(H):
            b0 = 20 + (m * H + h) % nbytes
            for b in range(4):
                scale[m, h] |= min(200, b0 + b) << (8 * b)
    scale = scale.to(torch.int32)
    kf = torch.randn(N, 128, generator=g).sign() * (1 + torch.rand(N, 128, generator=g) * 3)
    k = kf.to(FP8)
    ksc = torch.rand(N, generator=g) + 0.5
    w = torch.randn(M, H, generator=g)
    q = (packed, scale)
    _check_dense(q, (k, ksc), w, torch.zeros(M, dtype=torch.int32), torch.full((M,), N, dtype=torch.int32), False,
                 rows=torch.arange(M))


def _check_paged(q, cache, w, ctx, bt, mml, clean, rows=None, ref_rows=0, atol=None):
    gq = (q[0].to(DEV), q[1].to(DEV) if q[1] is not None else None)
    got = flaggems_vllm.fp8_fp4_paged_mqa_logits(gq, cache.to(DEV), w.to(DEV), ctx.to(DEV), bt.to(DEV), None,
                                                 mml, clean_logits=clean)
    torch.cuda.synchronize()
    got = got.cpu()
    nrows = w.shape[0]
    rows = _sample_rows(nrows, 8) if rows is None else rows
    want, bound = oracle.paged_mqa_logits(q, cache, w, ctx, bt, mml, clean, rows=rows)
    _within(got[rows], want, bound, "paged gpu vs binary64 oracle")
    fill = float("-inf") if clean else 0.0
    flat_ctx = ctx.reshape(-1)[:nrows] if ctx.dim() == 2 else ctx.repeat_interleave(nrows // ctx.shape[0])
    for r in range(nrows):   # the fill of every row, whole
        c = min(max(int(flat_ctx[r]), 0), mml)
        assert bool((got[r, c:] == fill).all()), f"row {r}: fill past the context"
    if ref_rows:
        ref = torch_ref.paged_mqa_logits(q, cache, w, ctx, bt, mml, clean)
        rr = rows[:ref_rows]
        torch.testing.assert_close(got[rr], ref[rr], atol=atol, rtol=1.3e-6, equal_nan=True)
    return got


@pytest.mark.gpu
@pytest.mark.parametrize("fp4", [False, True])
@pytest.mark.parametrize("shape", W.PAGED_MQA_SHAPES, ids=lambda s: f"B{s[0]}_N{s[1]}_L{s[2]}")
def test_gpu_paged_reference_shapes(shape, fp4):
    """The reference test's nine shapes, 64-entry blocks, max_model_len
    111 Ki, clean_logits off as it runs them; sampled rows against the oracle
    bound, two against the reference's float32 formulation (atol 0.15 as its
    MXFP4 check), and every row's fill."""
    B, nn, L = shape
    _say(f"paged mqa logits B={B} next_n={nn} ctx~{L} fp4={fp4}")
    q, cache, w, ctx, bt = W.make_paged_mqa_inputs(B, nn, L, fp4=fp4, seed=0)
    _check_paged(q, cache, w, ctx, bt, W.PAGED_MAX_MODEL_LEN, False, ref_rows=2, atol=0.15)


@pytest.mark.gpu
@pytest.mark.parametrize("fp4", [False, True])
def test_gpu_paged_edge_cases(fp4):
    """clean_logits on; 1-D context_lens; next_n = 3; zero-length and
    max_model_len-truncated contexts; -1 and out-of-range block-table entries
    (clamped into the cache as the reference clamps them); block size 16."""
    _say(f"paged mqa logits edge cases fp4={fp4}")
    q, cache, w, ctx, bt = W.make_paged_mqa_inputs(5, 3, 300, fp4=fp4, block_size=16, seed=11)
    ctx1 = ctx[:, 0].clone()
    ctx1[1] = 0
    ctx1[2] = 5000      # beyond max_model_len and the table
    bt[3, 2] = -1
    bt[4, 1] = cache.shape[0] + 7
    mml = 700
    _check_paged(q, cache, w, ctx1, bt, mml, True, rows=torch.arange(15))
    _check_paged(q, cache, w, ctx, bt, mml, False, rows=torch.arange(15))


@pytest.mark.gpu
def test_gpu_pipeline_from_indexer_ops():
    """The DeepSeek-V4 indexer chain on the GPU: fused_indexer_q_rope_quant
    (FP8 and MXFP4 q, folded weights) -> indexer_k_quant_and_cache (keys into
    the paged cache) -> cp_gather_indexer_k_quant_cache -> both logits ops;
    dense and paged logits agree with the oracle on the same bytes, and with
    each other position for position."""
    _say("indexer pipeline: q quant -> key cache -> gather -> logits")
    g = torch.Generator().manual_seed(12)
    T, H, L, bs = 48, 64, 700, 64
    nblk = (L + bs - 1) // bs + 3
    pos = torch.randint(0, 4096, (T,), generator=g)
    index_q = W.randn_bf16((T, H, 128), g)
    cs = W.make_cos_sin_cache(4096).to(DEV)
    iw = W.randn_bf16((T, H), g)
    keys = W.randn_bf16((L, 128), g)
    # one sequence of L keys in random blocks; its slots follow its block table
    table = torch.zeros(1, (L + bs - 1) // bs, dtype=torch.int32)
    perm = torch.randperm(nblk, generator=g)[:table.shape[1]].to(torch.int32)
    table[0] = perm
    slots = (perm[torch.arange(L) // bs].to(torch.int64) * bs + torch.arange(L) % bs)
    cache = torch.zeros(nblk, bs, 132, dtype=torch.uint8, device=DEV)
    flaggems_vllm.indexer_k_quant_and_cache(keys.to(DEV), cache, slots.to(DEV), 128, "ue8m0")
    kf = torch.empty(L, 128, dtype=torch.uint8, device=DEV)
    ksb = torch.empty(L, 4, dtype=torch.uint8, device=DEV)
    cu = torch.tensor([0, L], dtype=torch.int32, device=DEV)
    flaggems_vllm.cp_gather_indexer_k_quant_cache(cache, kf, ksb, table.to(DEV), cu)
    for fp4 in (False, True):
        qo, wo = flaggems_vllm.fused_indexer_q_rope_quant(pos.to(DEV), index_q.to(DEV), cs, iw.to(DEV),
                                                          128 ** -0.5, H ** -0.5, use_fp4=fp4)
        q = qo if fp4 else (qo, None)
        ks = torch.zeros(T, dtype=torch.int32, device=DEV)
        ke = torch.full((T,), L, dtype=torch.int32, device=DEV)
        dense = flaggems_vllm.fp8_fp4_mqa_logits(q, (kf.view(FP8), ksb.view(torch.float32).reshape(L)), wo, ks, ke)
        qp = (q[0].unsqueeze(1), q[1].reshape(T, 1, H) if fp4 else None)
        paged = flaggems_vllm.fp8_fp4_paged_mqa_logits(
            qp, cache.view(nblk, bs, 1, 132), wo, torch.full((T,), L, dtype=torch.int32, device=DEV),
            table.to(DEV).expand(T, -1).contiguous(), None, 1024, clean_logits=True)
        torch.cuda.synchronize()
        qc = tuple(x.cpu() if x is not None else None for x in q)
        want, bound = oracle.mqa_logits(qc, (kf.cpu().view(FP8), ksb.cpu().view(torch.float32).reshape(L)),
                                        wo.cpu(), ks.cpu(), ke.cpu(), True)
        _within(dense.cpu(), want, bound, f"pipeline dense fp4={fp4}")
        assert torch.equal(paged[:, :L].cpu(), dense.cpu()), "paged and dense logits differ"
        assert bool((paged[:, L:] == float("-inf")).all())


@pytest.mark.gpu
def test_gpu_graph_capture_replays():
    """Both ops captured in one HIP graph (outputs allocated at capture) and
    replayed three times with new inputs copied in and eager work between."""
    _say("mqa logits graph replays")
    M, N = 24, 500
    q, kv, w, ks, ke = W.make_mqa_logits_inputs(M, N, seed=13)
    pq, cache, pw, ctx, bt = W.make_paged_mqa_inputs(4, 1, 400, seed=14)
    d_q, d_k, d_s = q[0].to(DEV), kv[0].to(DEV), kv[1].to(DEV)
    d_w, d_ks, d_ke = w.to(DEV), ks.to(DEV), ke.to(DEV)
    d_pq, d_cache, d_pw, d_ctx, d_bt = pq[0].to(DEV), cache.to(DEV), pw.to(DEV), ctx.to(DEV), bt.to(DEV)

    def run():
        a = flaggems_vllm.fp8_fp4_mqa_logits((d_q, None), (d_k, d_s), d_w, d_ks, d_ke)
        b = flaggems_vllm.fp8_fp4_paged_mqa_logits((d_pq, None), d_cache, d_pw, d_ctx, d_bt, None, 600)
        return a, b

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run()
    for rep in range(3):
        q2, kv2, w2, _, _ = W.make_mqa_logits_inputs(M, N, seed=100 + rep)
        d_q.copy_(q2[0].to(DEV))
        d_k.copy_(kv2[0].to(DEV))
        d_s.copy_(kv2[1].to(DEV))
        d_w.copy_(w2.to(DEV))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want, bound = oracle.mqa_logits(q2, kv2, w2, ks, ke, True)
        _within(outs[0].cpu(), want, bound, f"replay {rep} dense")
        pw_want, pw_bound = oracle.paged_mqa_logits(pq, cache, pw, ctx, bt, 600, False)
        _within(outs[1].cpu(), pw_want, pw_bound, f"replay {rep} paged")
        _ = (d_w * 2).sum().item()


@pytest.mark.gpu
def test_gpu_mqa_logits_within_bound_on_wide_magnitudes():
    """Keys whose per-token scales span 2^-20..2^20 and weights of both signs:
    the bound, not an absolute tolerance, is what holds."""
    _say("mqa logits wide magnitudes")
    M, N = 16, 256
    q, kv, w, ks, ke = W.make_mqa_logits_inputs(M, N, seed=15)
    g = torch.Generator().manual_seed(16)
    ksc = torch.exp2(torch.randint(-20, 21, (N,), generator=g).float()) * (1 + torch.rand(N, generator=g))
    w = torch.randn(M, 64, generator=g) * 10
    _check_dense(q, (kv[0], ksc), w, ks, ke, False, rows=torch.arange(M))
