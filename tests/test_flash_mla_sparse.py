"""Sparse MLA prefill over bf16 rows (flash_mla_sparse_fwd): oracle pins
(CPU), wrapper and C-ABI checks (CPU) and GPU parity.

Reference: src/flaggems_vllm/ops/flashmla_sparse.py:1045-1206 (wrapper and
its assertions), :50-195 (kernel); tests/test_flash_mla_sparse_fwd.py:93-150
(the definitions of out, max_logits and lse), :152-164 and :196-214 (the two
case lists), :166-194 and :294-370 (input generators), :373-502 (the tests and
their tolerances).  The reference compares against vLLM's FlashMLA when it is
installed, else against its torch definition in float32; neither is available
here, so the bar is the binary64 oracle (oracle.sparse_mla_prefill) and a
float64 torch restatement of the same definition (_ref64, pinned to the oracle
on the CPU below) for the GPU-sized cases, at the reference's own tolerances:
    out         atol 8e-4, rtol 3.01/128   (the reference's FlashMLA cases)
    max_logits  atol 1e-6, rtol 2.01/65536
    lse         atol 1e-6, rtol 2.01/65536
and, for its first case list (randn inputs, scale d_qk^-0.5), out atol 1e-2
with bf16's rtol 1.6e-2, max_logits and lse atol 1e-4 with float32's rtol.
"""
import math

import pytest
import torch

import oracle
from flaggems_vllm import testing as W
from oracle import torch_ref

DEV = torch.device("cuda:0")
OUT_TOL = dict(atol=8e-4, rtol=3.01 / 128)
STAT_TOL = dict(atol=1e-6, rtol=2.01 / 65536)


# ------------------------------------------------------------ helpers ----

def _ref64(w):
    """float64 restatement of the reference test's definition
    (tests/test_flash_mla_sparse_fwd.py:93-150), on w's device: a gather of
    the selected rows, masked scores, torch's logsumexp, the sink merged as a
    second logsumexp term.  Returns (out, max_logits, lse) in float64."""
    q = w.q.double()
    s_q, h_q, d_qk = q.shape
    s_kv, topk = w.kv.shape[0], w.indices.shape[-1]
    idx = w.indices.reshape(s_q, topk).long()
    valid = (idx >= 0) & (idx < s_kv)
    if w.topk_length is not None:
        lens = w.topk_length.long().clamp(0, topk)
        valid &= torch.arange(topk, device=idx.device)[None, :] < lens[:, None]
    rows = w.kv.reshape(s_kv, d_qk).double()[torch.where(valid, idx, 0)]  # [s_q, topk, d_qk]
    p = torch.matmul(q, rows.transpose(1, 2).contiguous()) * w.sm_scale
    p.masked_fill_(~valid[:, None, :], float("-inf"))
    lse = torch.logsumexp(p, -1)
    max_logits = p.amax(-1) if topk else torch.full_like(lse, float("-inf"))
    lse_o = lse
    if w.attn_sink is not None:
        lse_o = torch.logsumexp(torch.stack([lse, w.attn_sink.double()[None, :].expand_as(lse)]), 0)
    lse_o = torch.where(lse_o == float("-inf"), float("inf"), lse_o)
    out = torch.matmul(torch.exp(p - lse_o[..., None]), rows[..., :512])
    lse = torch.where(lse == float("-inf"), float("inf"), lse)
    return out, max_logits, lse


def _oracle(w):
    return oracle.sparse_mla_prefill(w.q, w.kv, w.indices, w.sm_scale, w.attn_sink, w.topk_length)


def _close(got, want, what, **tol):
    torch.testing.assert_close(got.double().cpu(), want.double().cpu(), equal_nan=False, msg=lambda m: f"{what}: {m}",
                               **tol)


def _check(res, ref, what, out_tol=OUT_TOL, stat_tol=STAT_TOL):
    out, ml, lse = res
    r_out, r_ml, r_lse = ref
    assert out.dtype == torch.bfloat16 and ml.dtype == torch.float32 and lse.dtype == torch.float32
    _close(out, r_out, f"{what} out", **out_tol)
    _close(ml, r_ml, f"{what} max_logits", **stat_tol)
    _close(lse, r_lse, f"{what} lse", **stat_tol)


# Reference case list 2 (FlashMLA's): s_q x h_q x d_qk x (s_kv, topk) x sink x topk_length
FLASHMLA_CASES = [
    (s_q, h_q, d_qk, s_kv, topk, sink, tl)
    for s_q in (1, 62, 213)
    for h_q in (128, 64)
    for d_qk in (512, 576)
    for s_kv, topk in ((592, 128), (1840, 256), (1592, 384), (1521, 512), (95, 128), (153, 256), (114, 384))
    for sink in (True, False)
    for tl in (True, False)
]

# Reference case list 1: s_q x s_kv x h_q (64, 128; 256 is not supported) x d_qk 576 x topk
FIRST_CASES = [
    (s_q, s_kv, h_q, topk)
    for s_q in (64, 128, 512)
    for s_kv in (1024, 2048, 4096)
    for h_q in (64, 128)
    for topk in (64, 128, 256)
]


def _first_case_inputs(s_q, s_kv, h_q, topk, d_qk=576, seed=42):
    """The reference's make_input (tests/test_flash_mla_sparse_fwd.py:166-194):
    q, kv ~ randn (bf16), token t's row a random permutation of [0, max(1, t))
    (its first topk), padded with s_kv (invalid)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(s_q, h_q, d_qk, generator=g).to(torch.bfloat16)
    kv = torch.randn(s_kv, 1, d_qk, generator=g).to(torch.bfloat16)
    idx = torch.full((s_q, 1, topk), s_kv, dtype=torch.int32)
    for t in range(s_q):
        perm = torch.randperm(max(1, t), generator=g)[:topk]
        idx[t, 0, :len(perm)] = perm.to(torch.int32)
    return W.MlaSparseInputs(q, kv, idx, None, None, d_qk ** -0.5)


# ------------------------------------------------------- oracle pins ----

@pytest.mark.parametrize("d_qk", [512, 576])
@pytest.mark.parametrize("sink,tl", [(True, True), (False, False), (True, False)])
def test_oracle_against_library_softmax(d_qk, sink, tl):
    """The oracle against torch's float64 logsumexp / matmul restatement
    (_ref64) on the reference's input distribution, sink +-inf included."""
    w = W.make_mla_sparse_inputs(7, 95, 128, h_q=64, d_qk=d_qk, have_attn_sink=sink, have_topk_length=tl,
                                 seed=3 + d_qk)
    o, m, l = _oracle(w)
    ro, rm, rl = _ref64(w)
    assert torch.allclose(o, ro, rtol=1e-10, atol=1e-14)
    assert torch.equal(torch.isinf(m), torch.isinf(rm)) and torch.allclose(m, rm, rtol=1e-12, atol=1e-15)
    assert torch.equal(torch.isinf(l), torch.isinf(rl)) and torch.allclose(l, rl, rtol=1e-12, atol=1e-15)


def test_oracle_agrees_with_the_decode_oracle():
    """Prefill over the dequantised rows of a MODEL1 cache is the decode over
    that cache (token t = batch row t): the decode oracle is pinned
    independently (tests/test_sparse_mla.py)."""
    mw = W.make_mla_workload(batch=6, topk=128, num_pages=4, page=64, heads=64, seed=5)
    o_dec, l_dec = oracle.sparse_mla_decode_model1(mw.q, mw.k_cache, mw.indices, topk_length=mw.topk_length,
                                                   attn_sink=mw.attn_sink)
    rows = torch_ref.model1_rows(mw.k_cache)  # [256, 512] bf16
    w = W.MlaSparseInputs(mw.q[:, 0].contiguous(), rows.view(-1, 1, 512), mw.indices.view(6, 1, 128).clone(),
                          mw.attn_sink, mw.topk_length, 512 ** -0.5)
    o, m, l = _oracle(w)
    assert torch.allclose(o, o_dec[:, 0], rtol=1e-12, atol=1e-15)
    assert torch.allclose(l, l_dec[:, :, 0], rtol=1e-13, atol=0)


def test_oracle_closed_forms():
    """Single entry: out = V, lse = max_logits = the score.  n copies of one
    entry: lse = s + log n, out = V.  Sink +inf: out = 0, lse unchanged.
    Length 0: out 0, max_logits -inf, lse +inf.  d_qk 576 with a zero q tail
    equals d_qk 512 on the first 512 dims."""
    w = W.make_mla_sparse_inputs(4, 64, 8, h_q=64, d_qk=576, seed=9)
    idx = w.indices.clone()
    idx[0, 0, :] = -1
    idx[0, 0, 0] = 17
    idx[1, 0, :] = 23
    idx[2, 0, :] = 5
    idx[3, 0, :] = 3
    lens = torch.tensor([8, 5, 8, 0], dtype=torch.int32)
    sink = torch.full((64,), float("-inf"))
    sink[::2] = float("inf")
    w2 = W.MlaSparseInputs(w.q, w.kv, idx, sink, lens, 0.25)
    o, m, l = _oracle(w2)
    kv = w.kv[:, 0].double()
    q = w.q.double()
    s17 = (q[0] @ kv[17]) * 0.25
    s23 = (q[1] @ kv[23]) * 0.25
    assert torch.allclose(m[0], s17, rtol=1e-14) and torch.allclose(l[0], s17, rtol=1e-14)
    assert torch.allclose(l[1], s23 + math.log(5), rtol=1e-14)
    odd = torch.arange(64) % 2 == 1
    assert torch.allclose(o[0][odd], kv[17, :512].expand(32, 512), rtol=1e-14, atol=0)
    assert torch.allclose(o[1][odd], kv[23, :512].expand(32, 512), rtol=1e-13, atol=0)
    assert bool((o[:3][:, ~odd] == 0).all())
    assert bool((o[3] == 0).all()) and bool((m[3] == float("-inf")).all()) and bool((l[3] == float("inf")).all())

    qz = w.q.clone()
    qz[..., 512:] = 0
    a = W.MlaSparseInputs(qz, w.kv, w.indices, None, None, 0.3)
    b = W.MlaSparseInputs(qz[..., :512].contiguous(), w.kv[..., :512].contiguous(), w.indices, None, None, 0.3)
    for x, y in zip(_oracle(a), _oracle(b)):
        assert torch.allclose(x, y, rtol=1e-13, atol=1e-16)


@pytest.mark.parametrize("d_qk", [512, 576])
def test_float32_definition_within_reference_tolerance(d_qk):
    """The float32 restatement (the benchmark's CPU baseline) against the
    oracle at the reference's tolerances."""
    w = W.make_mla_sparse_inputs(12, 600, 256, h_q=64, d_qk=d_qk, have_attn_sink=True, have_topk_length=True,
                                 seed=21)
    got = torch_ref.flash_mla_sparse_fwd(w.q, w.kv, w.indices, w.sm_scale, w.attn_sink, w.topk_length)
    _check(got, _oracle(w), f"float32 definition d{d_qk}")


def test_input_generator_follows_the_reference():
    """Index rows: distinct valid ids (min(s_kv, topk) of them) then only
    invalid padding drawn from the reference's candidates; sink has +-inf
    entries; lengths lie in [0, topk]."""
    w = W.make_mla_sparse_inputs(20, 95, 128, h_q=64, have_attn_sink=True, have_topk_length=True, seed=1)
    idx = w.indices[:, 0].long()
    for t in range(20):
        head = idx[t, :95]
        assert head.unique().numel() == 95 and bool(((head >= 0) & (head < 95)).all())
        assert bool(((idx[t, 95:] < 0) | (idx[t, 95:] >= 95)).all())
    assert bool(torch.isinf(w.attn_sink).any()) and bool((w.topk_length >= 0).all())
    assert bool((w.topk_length <= 128).all())
    a = W.make_mla_sparse_inputs(6, 1000, 256, h_q=64, seed=2, affine=True)
    for t in range(6):
        assert a.indices[t, 0].unique().numel() == 256


# ------------------------------------------------ wrapper and C ABI ----

def _cpu_inputs(s_q=2, h_q=64, d_qk=512, s_kv=16, topk=8):
    return (torch.zeros(s_q, h_q, d_qk, dtype=torch.bfloat16), torch.zeros(s_kv, 1, d_qk, dtype=torch.bfloat16),
            torch.zeros(s_q, 1, topk, dtype=torch.int32))


@pytest.mark.parametrize("bad,match", [
    ("q_strided", None), ("q_fp16", None), ("d_v", "Unsupported d_v"), ("kv_dim", None), ("idx_shape", None),
    ("sink_dtype", None), ("sink_shape", "attn_sink error shape"), ("len_dtype", None),
    ("len_shape", "topk_length error shape"), ("h_kv", "h_kv is expected to be 1"), ("h_q", "Unsupported h_q"),
    ("d_qk", "Unsupported d_qk"), ("cpu", "GPU"),
])
def test_wrapper_asserts(bad, match):
    """The reference's assertions, in its order (flashmla_sparse.py:1081-1108),
    then the device check; all raise before anything touches a GPU."""
    from flaggems_vllm import flash_mla_sparse_fwd

    q, kv, idx = _cpu_inputs()
    sink = lens = None
    d_v = 512
    if bad == "q_strided":
        q = torch.zeros(64, 2, 512, dtype=torch.bfloat16).transpose(0, 1)
    elif bad == "q_fp16":
        q = q.half()
    elif bad == "d_v":
        d_v = 256
    elif bad == "kv_dim":
        kv = torch.zeros(16, 1, 576, dtype=torch.bfloat16)
    elif bad == "idx_shape":
        idx = torch.zeros(3, 1, 8, dtype=torch.int32)
    elif bad == "sink_dtype":
        sink = torch.zeros(64, dtype=torch.float64)
    elif bad == "sink_shape":
        sink = torch.zeros(32)
    elif bad == "len_dtype":
        lens = torch.zeros(2, dtype=torch.int64)
    elif bad == "len_shape":
        lens = torch.zeros(3, dtype=torch.int32)
    elif bad == "h_kv":
        kv = torch.zeros(16, 2, 512, dtype=torch.bfloat16)
        idx = torch.zeros(2, 2, 8, dtype=torch.int32)
    elif bad == "h_q":
        q = torch.zeros(2, 32, 512, dtype=torch.bfloat16)
    elif bad == "d_qk":
        q, kv, idx = _cpu_inputs(d_qk=256)
    with pytest.raises(AssertionError, match=match):
        flash_mla_sparse_fwd(q, kv, idx, 0.5, d_v, sink, lens)


def test_c_abi_rejects_bad_arguments():
    from flaggems_vllm import _native

    f = _native.lib().fgv_flash_mla_sparse_fwd

    def call(**kw):
        a = dict(q=16, qs=(64 * 512, 512), kv=16, kvs=512, skv=64, idx=16, its=8, topk=8, tl=None, sink=None,
                 sq=2, hq=64, d=512, out=16, os=(64 * 512, 512), ml=16, mls=64, lse=16, ls=64)
        a.update(kw)
        return f(a["q"], *a["qs"], a["kv"], a["kvs"], a["skv"], a["idx"], a["its"], a["topk"], a["tl"], a["sink"],
                 0.5, a["sq"], a["hq"], a["d"], a["out"], *a["os"], a["ml"], a["mls"], a["lse"], a["ls"], None)

    assert call(d=500, kvs=500) == -2
    assert call(hq=96) == -2
    assert call(sq=-1) == -2
    assert call(q=None) == -1
    assert call(lse=None) == -1
    assert call(q=8) == -3
    assert call(kv=8) == -3
    assert call(kvs=504) == -4
    assert call(os=(64 * 512, 256)) == -4
    assert call(mls=32) == -4
    assert call(out=8) == -3
    assert call(sq=0) == 0  # nothing to do, nothing launched


# --------------------------------------------------------- GPU parity ----

def _gpu(w):
    from flaggems_vllm import flash_mla_sparse_fwd

    d = w.to(DEV)
    res = flash_mla_sparse_fwd(*d.args())
    torch.cuda.synchronize()
    return d, res


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(FLASHMLA_CASES)),
                         ids=[f"sq{c[0]}-h{c[1]}-d{c[2]}-kv{c[3]}-k{c[4]}-sink{int(c[5])}-len{int(c[6])}"
                              for c in FLASHMLA_CASES])
def test_gpu_flashmla_cases(case):
    """The reference's FlashMLA case list (sm_scale 0.5) against _ref64."""
    s_q, h_q, d_qk, s_kv, topk, sink, tl = FLASHMLA_CASES[case]
    w = W.make_mla_sparse_inputs(s_q, s_kv, topk, h_q=h_q, d_qk=d_qk, have_attn_sink=sink, have_topk_length=tl,
                                 seed=case)
    print(f"flash_mla_sparse case {case}: {FLASHMLA_CASES[case]}", flush=True)
    d, res = _gpu(w)
    _check(res, _ref64(d), f"case {case}")


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(FIRST_CASES)),
                         ids=[f"sq{c[0]}-kv{c[1]}-h{c[2]}-k{c[3]}" for c in FIRST_CASES])
def test_gpu_first_cases(case):
    """The reference's first case list (randn inputs, d_qk 576, causal-style
    index rows padded with s_kv) at its tolerances."""
    s_q, s_kv, h_q, topk = FIRST_CASES[case]
    w = _first_case_inputs(s_q, s_kv, h_q, topk)
    print(f"flash_mla_sparse first case {case}: {FIRST_CASES[case]}", flush=True)
    d, res = _gpu(w)
    _check(res, _ref64(d), f"first case {case}", out_tol=dict(atol=1e-2, rtol=1.6e-2),
           stat_tol=dict(atol=1e-4, rtol=1.3e-6))


@pytest.mark.gpu
@pytest.mark.parametrize("d_qk", [512, 576])
def test_gpu_against_the_oracle(d_qk):
    """Small cases straight against the binary64 C oracle."""
    w = W.make_mla_sparse_inputs(9, 300, 256, h_q=128, d_qk=d_qk, have_attn_sink=True, have_topk_length=True,
                                 all_invalid_rows=True, seed=77)
    _, res = _gpu(w)
    _check(res, _oracle(w), f"oracle d{d_qk}")


@pytest.mark.gpu
@pytest.mark.parametrize("d_qk", [512, 576])
def test_gpu_edge_rows(d_qk):
    """Rows with nothing attended (all invalid, length 0, length clamped from
    above and below), one entry, duplicated entries, and sink +-inf."""
    w = W.make_mla_sparse_inputs(8, 200, 96, h_q=64, d_qk=d_qk, have_attn_sink=True, seed=5)
    idx = w.indices.clone()
    idx[0] = -1                      # nothing valid
    idx[1, 0, :] = 199               # one entry, 96 times
    idx[2, 0, 1:] = 200              # one valid entry then s_kv
    idx[3, 0, 48:] = idx[3, 0, :48]  # every entry twice
    lens = torch.tensor([96, 96, 96, 96, 0, -5, 1000, 33], dtype=torch.int32)
    w = W.MlaSparseInputs(w.q, w.kv, idx, w.attn_sink, lens, w.sm_scale)
    _, res = _gpu(w)
    ref = _oracle(w)
    _check(res, ref, "edge rows")
    out, ml, lse = (r.cpu() for r in res)
    for t in (0, 4, 5):
        assert bool((out[t] == 0).all()) and bool((ml[t] == float("-inf")).all())
        assert bool((lse[t] == float("inf")).all())
    keep = w.attn_sink != float("inf")
    row = w.kv[199, 0, :512]
    assert torch.equal(out[1][keep & (w.attn_sink == float("-inf"))],
                       row.expand(int((keep & (w.attn_sink == float("-inf"))).sum()), 512))
    assert bool((out[:, ~keep] == 0).all())


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [4.0, 40.0])
def test_gpu_wide_score_range(scale):
    """Scores spread over tens of units (sm_scale 4 and 40 on the reference's
    inputs): the running maximum is raised and O rescaled many times."""
    w = W.make_mla_sparse_inputs(16, 2048, 1024, h_q=64, d_qk=576, seed=8, sm_scale=scale)
    _, res = _gpu(w)
    _check(res, _oracle(w), f"scale {scale}")


@pytest.mark.gpu
def test_gpu_bench_case_sampled():
    """The reference benchmark's first case (s_q 4096, s_kv 8192, topk 2048,
    h_q 128, d_qk 576, sink) on the GPU, 24 tokens checked against _ref64."""
    s_kv, topk, h_q, d_qk = W.MLA_SPARSE_CASES["v32_8k"]
    w = W.make_mla_sparse_inputs(4096, s_kv, topk, h_q=h_q, d_qk=d_qk, have_attn_sink=True, seed=0)
    d, res = _gpu(w)
    pick = torch.linspace(0, 4095, 24).long()
    sub = W.MlaSparseInputs(d.q[pick], d.kv, d.indices[pick], d.attn_sink, None, d.sm_scale)
    _check(tuple(r[pick] for r in res), _ref64(sub), "bench case")


@pytest.mark.gpu
def test_gpu_deterministic_and_torch_op():
    """Two calls give the same bits; torch.ops.flaggems_vllm.flash_mla_sparse_fwd
    returns the same tensors as the function."""
    w = W.make_mla_sparse_inputs(33, 1500, 512, h_q=128, d_qk=512, have_attn_sink=True, have_topk_length=True,
                                 seed=12).to(DEV)
    from flaggems_vllm import flash_mla_sparse_fwd

    a = flash_mla_sparse_fwd(*w.args())
    b = flash_mla_sparse_fwd(*w.args())
    c = torch.ops.flaggems_vllm.flash_mla_sparse_fwd(*w.args())
    for x, y, z in zip(a, b, c):
        assert torch.equal(x, y) and torch.equal(x, z)


@pytest.mark.gpu
def test_gpu_empty():
    from flaggems_vllm import flash_mla_sparse_fwd

    w = W.make_mla_sparse_inputs(0, 64, 128, h_q=64, seed=1).to(DEV)
    out, ml, lse = flash_mla_sparse_fwd(*w.args())
    assert out.shape == (0, 64, 512) and ml.shape == (0, 64) and lse.shape == (0, 64)
    w = W.make_mla_sparse_inputs(3, 64, 0, h_q=64, seed=1).to(DEV)
    out, ml, lse = flash_mla_sparse_fwd(*w.args())
    torch.cuda.synchronize()
    assert bool((out == 0).all()) and bool((ml == float("-inf")).all()) and bool((lse == float("inf")).all())
