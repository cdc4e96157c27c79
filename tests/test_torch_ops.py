"""torch.ops.flaggems_vllm registrations: schemas, fake shapes, and identity
with the plain functions on the GPU.

The plain Python functions are the reference API; these tests check that the
registered custom ops declare exactly the tensors each op writes (the main op
writes q and k_cache, as vLLM's op schema marks them) and that they compute
the same bytes as the functions they wrap.
"""
import pytest
import torch

import flaggems_vllm
from flaggems_vllm import library
from flaggems_vllm import testing as W

from .test_gather import _ref_fixture
from .test_indexer import _case as _indexer_case
from .test_rmsnorm import _inputs as _rmsnorm_inputs
from .test_slot_mapping import _ragged_inputs

DEV = torch.device("cuda:0")

WRITES = {
    "fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert": {"q", "k_cache"},
    "fused_inv_rope_fp8_quant": set(),
    "fused_q_kv_rmsnorm": set(),
    "dequantize_and_gather_k_cache": {"out"},
    "fused_indexer_q_rope_quant": set(),
    "compute_slot_mapping_parallel": {"slot_mapping"},
    "indexer_k_quant_and_cache": {"kv_cache"},
    "cp_gather_indexer_k_quant_cache": {"k_fp8", "k_fp8_scale"},
    "compute_global_topk_indices_and_lens": set(),
    "combine_topk_swa_indices": set(),
    "top_k_per_row_decode": {"indices"},
    "top_k_per_row_prefill": {"indices"},
    "fp8_einsum": set(),
    "fp8_einsum_out": {"out"},
    "persistent_topk": {"output", "workspace"},
    "flash_mla_sparse_fwd": set(),
}


def _op(name):
    return getattr(torch.ops.flaggems_vllm, name).default


# ------------------------------------------------------------------- CPU ----

@pytest.mark.parametrize("name", library.REGISTERED)
def test_schema_declares_exactly_the_written_tensors(name):
    schema = _op(name)._schema
    written = {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}
    assert written == WRITES[name]
    # the main op keeps the reference's positional order
    if name == "fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert":
        assert [a.name for a in schema.arguments] == ["q", "kv", "k_cache", "slot_mapping", "position_ids",
                                                       "cos_sin_cache", "eps", "cache_block_size"]
        assert len(schema.returns) == 0


@pytest.mark.parametrize("tma", [False, True])
@pytest.mark.parametrize("T", [1, 6, 8])
def test_sibling_fake_layout(T, tma):
    """Shapes, dtypes and strides of the fake outputs: fp8 [T, G, d] with
    strides (d, T*d, 1); scales [T, G, K] token-fastest with Tpad = T rounded up to 4."""
    H, G = 16, 4
    o = torch.empty(T, H, 512, dtype=torch.bfloat16, device="meta")
    pos = torch.empty(T, dtype=torch.int64, device="meta")
    cs = torch.empty(4096, 64, dtype=torch.float32, device="meta")
    fp8, scale = _op("fused_inv_rope_fp8_quant")(o, pos, cs, G, H // G, tma_aligned_scales=tma)
    d = (H // G) * 512
    tpad = (T + 3) // 4 * 4
    k = d // 128
    inner = (k + 3) // 4 if tma else k
    assert fp8.shape == (T, G, d) and fp8.dtype == torch.float8_e4m3fn and fp8.stride() == (d, T * d, 1)
    assert scale.shape == (T, G, inner) and scale.stride() == (1, inner * tpad, tpad)
    assert scale.dtype == (torch.int32 if tma else torch.float32)


@pytest.mark.parametrize("fp4", [False, True])
@pytest.mark.parametrize("D", [128, 256, 512])
def test_indexer_fake_layout(fp4, D):
    """The fake outputs have the real op's layouts: FP8 codes like index_q
    (its rows, which may exceed the token count); MXFP4 nibbles [T, H, D/2]
    and the UE8M0 bytes as the int32 view [T, H, D/128], squeezed to [T, H]
    at D = 128 (reference ops/fused_indexer_q_rope_quant.py:378-391); weights
    like index_weights in float32."""
    pos = torch.empty(5, dtype=torch.int64, device="meta")
    q = torch.empty(7, 8, D, dtype=torch.bfloat16, device="meta")
    cs = torch.empty(64, 64, dtype=torch.float32, device="meta")
    w = torch.empty(6, 8, dtype=torch.bfloat16, device="meta")
    qo, sc, wo = _op("fused_indexer_q_rope_quant")(pos, q, cs, w, 0.1, 0.2, fp4)
    assert wo.shape == (6, 8) and wo.dtype == torch.float32
    if fp4:
        assert qo.shape == (5, 8, D // 2) and qo.dtype == torch.uint8
        assert sc.dtype == torch.int32
        assert sc.shape == ((5, 8) if D == 128 else (5, 8, D // 128))
    else:
        assert qo.shape == (7, 8, D) and qo.dtype == torch.float8_e4m3fn and sc.numel() == 0


# ------------------------------------------------------------------- GPU ----

def _say(msg):
    print(f"\n[case] {msg}", flush=True)


@pytest.mark.gpu
def test_gpu_main_op_matches_function_and_opcheck():
    _say("torch.ops main op, config 0")
    w = W.make_workload(0).to(DEV)
    a, b = w.clone(), w.clone()
    flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(*a.args())
    _op("fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert")(*b.args())
    torch.cuda.synchronize()
    assert torch.equal(a.q.view(torch.int16), b.q.view(torch.int16))
    assert torch.equal(a.k_cache, b.k_cache)
    c = w.clone()
    torch.library.opcheck(_op("fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert"), tuple(c.args()),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
@pytest.mark.parametrize("tma", [False, True])
def test_gpu_sibling_matches_function_and_fake_layout(tma):
    _say(f"torch.ops sibling tma={tma}")
    w = W.make_inv_rope_workload(37, 16, 4, seed=3).to(DEV)
    args = (w.o, w.positions, w.cos_sin_cache, w.n_groups, w.heads_per_group)
    f8, fs = flaggems_vllm.fused_inv_rope_fp8_quant(*args, tma_aligned_scales=tma)
    o8, os_ = _op("fused_inv_rope_fp8_quant")(*args, tma_aligned_scales=tma)
    torch.cuda.synchronize()
    assert o8.stride() == f8.stride() and os_.stride() == fs.stride()
    assert torch.equal(o8.view(torch.uint8), f8.view(torch.uint8))
    assert torch.equal(os_.view(torch.int32), fs.view(torch.int32))
    torch.library.opcheck(_op("fused_inv_rope_fp8_quant"), args, {"tma_aligned_scales": tma},
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
def test_gpu_rmsnorm_indexer_gather_slot_match_functions():
    _say("torch.ops rmsnorm / indexer / gather / slot mapping")
    qr, kv, qw, kw = (t.to(DEV) for t in _rmsnorm_inputs(9, 1536, 512, 4))
    a = flaggems_vllm.fused_q_kv_rmsnorm(qr, kv, qw, kw, 1e-6)
    b = _op("fused_q_kv_rmsnorm")(qr, kv, qw, kw, 1e-6)
    assert all(torch.equal(x.view(torch.int16), y.view(torch.int16)) for x, y in zip(a, b))

    pos, q, cs, wt, sm, hs = _indexer_case(11, seed=5)
    pos, q, cs, wt = pos.to(DEV), q.to(DEV), cs.to(DEV), wt.to(DEV)
    for fp4 in (False, True):
        fq, fw = flaggems_vllm.fused_indexer_q_rope_quant(pos, q, cs, wt, sm, hs, use_fp4=fp4)
        oq, osc, ow = _op("fused_indexer_q_rope_quant")(pos, q, cs, wt, sm, hs, fp4)
        assert torch.equal(fw, ow)
        if fp4:
            assert torch.equal(fq[0], oq) and torch.equal(fq[1], osc)
        else:
            assert torch.equal(fq.view(torch.uint8), oq.view(torch.uint8)) and osc.numel() == 0

    cache, expected, seq_lens, gather_lens, bt, slots = _ref_fixture(2, 12, 5, 64, 448, 64)
    out_f = torch.zeros_like(expected, device=DEV)
    out_o = torch.zeros_like(expected, device=DEV)
    gargs = (cache.to(DEV), seq_lens.to(DEV), gather_lens.to(DEV), bt.to(DEV), 64)
    flaggems_vllm.dequantize_and_gather_k_cache(out_f, *gargs)
    _op("dequantize_and_gather_k_cache")(out_o, *gargs)
    assert torch.equal(out_f.cpu(), expected) and torch.equal(out_o.cpu(), expected)

    qsl, p, table = _ragged_inputs(2)
    n = int(qsl[-1])
    sl_f = torch.full((n + 5,), -7, dtype=torch.int64, device=DEV)
    sl_o = sl_f.clone()
    sargs = (n, n + 5, qsl.to(DEV), qsl.numel() - 1, p.to(DEV), table.to(DEV))
    flaggems_vllm.compute_slot_mapping_parallel(*sargs, sl_f, 16)
    _op("compute_slot_mapping_parallel")(*sargs, sl_o, 16)
    torch.cuda.synchronize()
    assert torch.equal(sl_f, sl_o)


@pytest.mark.gpu
@pytest.mark.parametrize("fp4", [False, True])
@pytest.mark.parametrize("D", [128, 256])
def test_gpu_indexer_opcheck(fp4, D):
    """Schema and fake-tensor checks of the indexer op in both modes: the
    fake's dtypes, shapes and strides equal the real outputs' (int32 UE8M0
    view, squeezed at D = 128), with index_q holding more rows than there are
    positions, as the reference's assert allows."""
    _say(f"torch.ops indexer opcheck fp4={fp4} D={D}")
    pos, q, cs, wt, sm, hs = _indexer_case(9, H=16, D=D, seed=6)
    qbig = torch.cat([q, q[:3]]).to(DEV)  # 12 rows for 9 positions
    args = (pos.to(DEV), qbig, cs.to(DEV), wt.to(DEV), sm, hs, fp4)
    oq, osc, ow = _op("fused_indexer_q_rope_quant")(*args)
    torch.cuda.synchronize()
    if fp4:
        assert osc.dtype == torch.int32 and osc.shape == ((9, 16) if D == 128 else (9, 16, D // 128))
    else:
        assert oq.shape == qbig.shape and oq.stride() == qbig.stride()
    torch.library.opcheck(_op("fused_indexer_q_rope_quant"), args,
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
def test_gpu_topk_index_ops_opcheck():
    """The index-row ops through torch.ops: same outputs as the functions, and
    the fakes' shapes, dtypes and strides equal the real outputs'."""
    _say("torch.ops global top-k indices / combine top-k + window opcheck")
    g = torch.Generator().manual_seed(2)
    local = torch.randint(-1, 64 * 4, (37, 24), generator=g, dtype=torch.int32).to(DEV)
    req = torch.randint(0, 3, (37,), generator=g, dtype=torch.int32).to(DEV)
    bt = torch.randint(0, 999, (3, 4), generator=g, dtype=torch.int32).to(DEV)
    valid = torch.randint(0, 2, (37,), generator=g, dtype=torch.int32).to(DEV)
    a = (local, req, bt, 64, valid)
    f = flaggems_vllm.compute_global_topk_indices_and_lens(*a)
    o = _op("compute_global_topk_indices_and_lens")(*a)
    torch.cuda.synchronize()
    assert torch.equal(f[0], o[0]) and torch.equal(f[1], o[1])
    torch.library.opcheck(_op("compute_global_topk_indices_and_lens"), a, test_utils=("test_schema", "test_faketensor"))
    qsl = torch.tensor([0, 20, 37], dtype=torch.int32, device=DEV)
    seq = torch.tensor([100, 40], dtype=torch.int32, device=DEV)
    gat = torch.tensor([50, 40], dtype=torch.int32, device=DEV)
    c = (local, qsl, seq, gat, 16, 4, 24, 1000, 500)
    f = flaggems_vllm.combine_topk_swa_indices(*c)
    o = _op("combine_topk_swa_indices")(*c)
    torch.cuda.synchronize()
    assert torch.equal(f[0], o[0]) and torch.equal(f[1], o[1])
    torch.library.opcheck(_op("combine_topk_swa_indices"), c, test_utils=("test_schema", "test_faketensor"))


@pytest.mark.gpu
def test_gpu_top_k_per_row_ops():
    """The top-k ops through torch.ops write the same index sets as the functions."""
    _say("torch.ops top_k_per_row decode / prefill")
    g = torch.Generator().manual_seed(3)
    lg = torch.randn(6, 20000, generator=g).to(DEV)
    seq = torch.tensor([20000, 9000, 300, 20000, 15000, 12345], dtype=torch.int32, device=DEV)
    a = torch.empty(6, 512, dtype=torch.int32, device=DEV)
    b = torch.empty_like(a)
    flaggems_vllm.top_k_per_row_decode(lg, 1, seq, a, 6, lg.stride(0), lg.stride(1), 512)
    _op("top_k_per_row_decode")(lg, 1, seq, b, 6, lg.stride(0), lg.stride(1), 512)
    torch.cuda.synchronize()
    assert torch.equal(a.sort(1).values, b.sort(1).values)
    st = torch.tensor([0, 100, 5000, 0, 7, 19000], dtype=torch.int32, device=DEV)
    flaggems_vllm.top_k_per_row_prefill(lg, st, seq, a, 6, lg.stride(0), lg.stride(1), 512)
    _op("top_k_per_row_prefill")(lg, st, seq, b, 6, lg.stride(0), lg.stride(1), 512)
    torch.cuda.synchronize()
    assert torch.equal(a.sort(1).values, b.sort(1).values)


@pytest.mark.gpu
def test_gpu_fp8_einsum_ops():
    """torch.ops.flaggems_vllm.fp8_einsum / fp8_einsum_out: the function's
    bytes, fake layout and opcheck."""
    from .test_fp8_einsum import make_inputs

    x, xs, y, ys = (t.to(DEV) for t in make_inputs(3, 2, 256, 128, seed=4))
    ref = flaggems_vllm.fp8_einsum("bhr,hdr->bhd", x, xs, y, ys)
    got = torch.ops.flaggems_vllm.fp8_einsum("bhr,hdr->bhd", x, xs, y, ys, [128, 128], torch.bfloat16)
    assert torch.equal(got, ref)
    out = torch.empty_like(ref)
    torch.ops.flaggems_vllm.fp8_einsum_out("bhr,hdr->bhd", x, xs, y, ys, [128, 128], torch.bfloat16, out)
    assert torch.equal(out, ref)
    # opcheck's schema test multiplies float8 inputs, which torch cannot do on
    # the GPU; the fake-tensor and autograd-registration tests run
    utils = ("test_faketensor", "test_autograd_registration")
    torch.library.opcheck(torch.ops.flaggems_vllm.fp8_einsum.default,
                          ("bhr,hdr->bhd", x, xs, y, ys, [128, 128], torch.float32), test_utils=utils)
    torch.library.opcheck(torch.ops.flaggems_vllm.fp8_einsum_out.default,
                          ("bhr,hdr->bhd", x, xs, y, ys, [128, 128], torch.bfloat16, out), test_utils=utils)


@pytest.mark.gpu
def test_gpu_flash_mla_sparse_op():
    """torch.ops.flaggems_vllm.flash_mla_sparse_fwd: the function's bytes, fake
    layout and opcheck."""
    from flaggems_vllm import testing as W

    w = W.make_mla_sparse_inputs(5, 300, 128, h_q=64, d_qk=576, have_attn_sink=True, have_topk_length=True,
                                 seed=3).to(DEV)
    ref = flaggems_vllm.flash_mla_sparse_fwd(*w.args())
    got = torch.ops.flaggems_vllm.flash_mla_sparse_fwd(*w.args())
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    torch.library.opcheck(_op("flash_mla_sparse_fwd"), w.args(),
                          test_utils=("test_schema", "test_faketensor", "test_autograd_registration"))
