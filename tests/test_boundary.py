"""CPU tests of the drop-in boundary: the C-ABI library loads and exports what
include/flaggems_vllm_amd.h declares, its argument checks return the
documented codes without launching anything, and the Python wrappers keep the
reference's signatures and AssertionErrors (reference wrappers:
ops/fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:320-333,
ops/fused_inv_rope_fp8_quant.py:184-205)."""
import ctypes
import inspect
import os
import re

import pytest
import torch

import flaggems_vllm
from flaggems_vllm import _native
from flaggems_vllm import testing as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    syms = set()
    for name in os.listdir(os.path.join(ROOT, "include")):
        if name.endswith(".h"):
            text = open(os.path.join(ROOT, "include", name)).read()
            syms |= set(re.findall(r"^\s*(?:int|int64_t|const char\s*\*)\s+(fgv_\w+)\s*\(", text, re.M))
    return syms


def test_library_exports_every_declared_symbol():
    syms = declared_symbols()
    assert syms == set(_native.EXPORTED_SYMBOLS)
    L = ctypes.CDLL(_native.LIB_PATH)
    for s in syms:
        assert hasattr(L, s), s
    assert _native.lib().fgv_version() == 100


def _call_main(**kw):
    args = dict(q=16, q_st=8 * 512, q_sh=512, kv=16, kv_st=512, cache=16, stride=64 * 584,
                nblk=4, slots=16, n_ins=4, pos=16, cs=16, cs_st=64, max_pos=16, T=4, H=8,
                eps=1e-6, bs=64)
    args.update(kw)
    a = args
    return _native.lib().fgv_qnorm_rope_kv_rope_quant_insert(
        a["q"], a["q_st"], a["q_sh"], a["kv"], a["kv_st"], a["cache"], a["stride"], a["nblk"],
        a["slots"], a["n_ins"], a["pos"], a["cs"], a["cs_st"], a["max_pos"], a["T"], a["H"],
        a["eps"], a["bs"], None)


@pytest.mark.parametrize("kw,code", [
    (dict(n_ins=5), -2),                       # slot_mapping longer than q
    (dict(T=-1), -2),
    (dict(q=None), -1),
    (dict(q=17), -3),                          # q not 16-byte aligned
    (dict(q_st=8 * 512 + 4), -4),              # token stride not a multiple of 8
    (dict(cs_st=66), -4),
    (dict(stride=64 * 584 - 8), -4),           # block stride below bs * 584
    (dict(cache=20), -3),                      # cache not 8-byte aligned
    (dict(max_pos=0), -2),
    (dict(bs=0), -2),
    (dict(T=1 << 20, H=1 << 12, n_ins=0), -5),  # 2^32 q rows
])
def test_c_abi_rejects_bad_arguments(kw, code):
    assert _call_main(**kw) == code
    assert _native.lib().fgv_last_error()


def test_c_abi_empty_call_is_a_no_op():
    assert _call_main(T=0, n_ins=0, q=None, kv=None) == 0


def test_inv_rope_c_abi_rejects_bad_arguments():
    f = _native.lib().fgv_inv_rope_fp8_quant
    ok = dict(o=16, ost=64 * 512, osh=512, pos=16, cs=16, css=64, mp=16, T=4, G=8, hpg=8, nope=448, rope=64,
              grp=128, f8=16, f8g=4 * 4096, f8t=4096, sc=16, scg=32 * 4, sck=4, tpad=4, eps=1e-10, tma=0)

    def call(**kw):
        a = dict(ok, **kw)
        return f(a["o"], a["ost"], a["osh"], a["pos"], a["cs"], a["css"], a["mp"], a["T"], a["G"],
                 a["hpg"], a["nope"], a["rope"], a["grp"], a["f8"], a["f8g"], a["f8t"], a["sc"], a["scg"],
                 a["sck"], a["tpad"], a["eps"], a["tma"], None)

    assert call(tpad=9) == -2
    assert call(G=0) == -2
    assert call(o=24) == -3
    assert call(eps=0.0) == -2
    assert call(T=0, tpad=0) == 0
    # geometry: the reference's conditions, then this build's limits
    assert call(nope=440) == -2                       # rope not inside the last chunk
    assert call(rope=63, nope=449) == -2              # odd rope_dim
    assert call(nope=448, rope=64, grp=96) == -2      # group does not divide head_dim
    assert call(nope=64, rope=64, grp=128, tma=0, T=0, tpad=0) == 0  # D = 128: accepted
    assert call(nope=960, rope=64, grp=128) == -2     # D = 1024: beyond this build's 512
    assert call(nope=448, rope=64, grp=64, tma=1) == -2   # 8 chunks cannot be packed
    assert call(nope=192, rope=64, grp=128, tma=1) == -2  # 2 chunks packed, 8 heads per group
    assert call(nope=192, rope=64, grp=128, tma=1, hpg=1, G=64, T=0, tpad=0) == 0


def test_signatures_match_reference():
    p = inspect.signature(flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert).parameters
    assert list(p) == ["q", "kv", "k_cache", "slot_mapping", "position_ids", "cos_sin_cache",
                       "eps", "cache_block_size"]
    p = inspect.signature(flaggems_vllm.fused_inv_rope_fp8_quant).parameters
    assert list(p) == ["o", "positions", "cos_sin_cache", "n_groups", "heads_per_group",
                       "nope_dim", "rope_dim", "quant_group_size", "eps", "dtype",
                       "tma_aligned_scales"]
    assert [p[k].default for k in ("nope_dim", "rope_dim", "quant_group_size", "eps", "dtype",
                                   "tma_aligned_scales")] == [448, 64, 128, 1e-10, None, False]
    assert flaggems_vllm.ops_deepseek_v4_qnorm_rope_kv_rope_quant_insert is \
        flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert
    assert flaggems_vllm.ops_inv_rope_fp8_quant is flaggems_vllm.fused_inv_rope_fp8_quant
    assert flaggems_vllm.SUPPORTED_FP8_DTYPE == torch.float8_e4m3fn


def _args(**over):
    w = W.make_workload(0)
    a = dict(q=w.q, kv=w.kv, k_cache=w.k_cache, slot_mapping=w.slot_mapping,
             position_ids=w.position_ids, cos_sin_cache=w.cos_sin_cache, eps=1e-6,
             cache_block_size=64)
    a.update(over)
    return a


@pytest.mark.parametrize("bad", [
    dict(q=torch.zeros(16, 8, 256, dtype=torch.bfloat16)),
    dict(kv=torch.zeros(15, 512, dtype=torch.bfloat16)),
    dict(q=torch.zeros(16, 8, 512, dtype=torch.float16)),
    dict(k_cache=torch.zeros(4, 64 * 584, dtype=torch.int8)),
    dict(slot_mapping=torch.zeros(17, dtype=torch.int64)),
    dict(slot_mapping=torch.zeros(16, dtype=torch.int32)),
    dict(position_ids=torch.zeros(16, dtype=torch.int32)),
    dict(cos_sin_cache=torch.zeros(16, 32)),
    dict(cos_sin_cache=torch.zeros(16, 64, dtype=torch.float64)),
])
def test_main_wrapper_asserts_like_reference(bad):
    with pytest.raises(AssertionError):
        flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(**_args(**bad))


def test_main_wrapper_refuses_cpu_tensors():
    """No CPU fallback: valid CPU inputs fail loudly instead of computing."""
    with pytest.raises(AssertionError, match="GPU"):
        flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(**_args())


@pytest.mark.parametrize("bad,kw", [
    ({}, dict(dtype=torch.float16)),
    ({}, dict(n_groups=3)),
    ({"o": torch.zeros(4, 64, 256, dtype=torch.bfloat16)}, {}),
    ({"positions": torch.zeros(5, dtype=torch.int64)}, {}),
    ({}, dict(nope_dim=192, rope_dim=64)),             # head_dim 512 != 192 + 64
    ({}, dict(nope_dim=440, rope_dim=72)),             # rope not inside the last chunk
    ({"o": torch.zeros(4, 64, 1024, dtype=torch.bfloat16)}, dict(nope_dim=960, rope_dim=64)),  # D beyond 512
    ({}, dict(quant_group_size=64, tma_aligned_scales=True)),  # 8 chunks cannot be packed
    ({"cos_sin_cache": torch.zeros(16, 64, dtype=torch.float64)}, {}),
    ({}, {}),  # valid, but CPU tensors
])
def test_sibling_wrapper_asserts(bad, kw):
    a = dict(o=torch.zeros(4, 64, 512, dtype=torch.bfloat16), positions=torch.zeros(4, dtype=torch.int64),
             cos_sin_cache=torch.zeros(16, 64), n_groups=8, heads_per_group=8)
    a.update(bad)
    a.update(kw)
    with pytest.raises(AssertionError):
        flaggems_vllm.fused_inv_rope_fp8_quant(**a)


def _rms_args(**over):
    a = dict(qr=torch.zeros(4, 1536, dtype=torch.bfloat16), kv=torch.zeros(4, 512, dtype=torch.bfloat16),
             q_weight=torch.zeros(1536, dtype=torch.bfloat16), kv_weight=torch.zeros(512, dtype=torch.bfloat16),
             eps=1e-6)
    a.update(over)
    return a


@pytest.mark.parametrize("bad,match", [
    (dict(qr=torch.zeros(4, 2, 768, dtype=torch.bfloat16)), 'must be 2D'),            # not 2D
    (dict(kv=torch.zeros(5, 512, dtype=torch.bfloat16)), 'token count mismatch'),               # token counts differ
    (dict(qr=torch.zeros(1536, 4, dtype=torch.bfloat16).t()), 'rows must be contiguous'),          # rows not contiguous
    (dict(q_weight=torch.zeros(3072, dtype=torch.bfloat16)[::2]), 'weights must be contiguous'),      # weight not contiguous
    (dict(qr=torch.zeros(4, 1536, dtype=torch.float16)), 'bf16 activations'),               # not bf16
    (dict(kv_weight=torch.zeros(512)), 'both bf16 or both float32'),                                 # weight dtypes differ
    (dict(q_weight=torch.zeros(1535, dtype=torch.bfloat16)), 'weight sizes'),           # weight size != row size
    ({}, 'GPU'),                                                               # valid, but CPU tensors
])
def test_rmsnorm_wrapper_asserts(bad, match):
    with pytest.raises(AssertionError, match=match):
        flaggems_vllm.fused_q_kv_rmsnorm(**_rms_args(**bad))


def test_rmsnorm_wrapper_empty_rows_allocate_only():
    """No tokens: the outputs are allocated and nothing is checked further or launched."""
    qo, ko = flaggems_vllm.fused_q_kv_rmsnorm(**_rms_args(qr=torch.zeros(0, 1536, dtype=torch.bfloat16),
                                                          kv=torch.zeros(0, 512, dtype=torch.bfloat16)))
    assert qo.shape == (0, 1536) and ko.shape == (0, 512)


def _gather_args(**over):
    a = dict(out=torch.zeros(2, 64, 512, dtype=torch.bfloat16), k_cache=torch.zeros(4, 64 * W.HEAD_BYTES,
                                                                                    dtype=torch.uint8),
             seq_lens=torch.full((2,), 64, dtype=torch.int32), gather_lens=None,
             block_table=torch.zeros(2, 2, dtype=torch.int32), block_size=64)
    a.update(over)
    return a


@pytest.mark.parametrize("bad,match", [
    (dict(out=torch.zeros(2, 64, 512, dtype=torch.float32)), '3D bfloat16'),           # out not bf16
    (dict(seq_lens=torch.full((2, 1), 64, dtype=torch.int32)), 'must be 1D'),         # seq_lens not 1D
    (dict(block_table=torch.zeros(3, 2, dtype=torch.int32)), 'request count'),           # request counts differ
    (dict(out=torch.zeros(1, 64, 512, dtype=torch.bfloat16)), 'request count'),          # more requests than out rows
    (dict(nope_dim=480), 'must fit'),                                               # nope + rope beyond out's last dim
    (dict(k_cache=torch.zeros(4 * 64 * W.HEAD_BYTES, dtype=torch.uint8)), '2D or 3D'),  # 1D cache
    (dict(out=torch.zeros(2, 512, 64, dtype=torch.bfloat16).transpose(1, 2)), 'out rows must be contiguous'),  # rows not contiguous
    (dict(k_cache=torch.zeros(64 * W.HEAD_BYTES, 4, dtype=torch.uint8).t()), 'contiguous bytes'),    # blocks not contiguous
    (dict(block_table=torch.zeros(2, 4, dtype=torch.int32)[:, ::2]), 'block_table rows'),   # block-table rows not contiguous
    ({}, 'GPU'),                                                               # valid, but CPU tensors
])
def test_gather_wrapper_asserts(bad, match):
    with pytest.raises(AssertionError, match=match):
        flaggems_vllm.dequantize_and_gather_k_cache(**_gather_args(**bad))


def _indexer_args(**over):
    a = dict(positions=torch.zeros(4, dtype=torch.int64), index_q=torch.zeros(4, 8, 128, dtype=torch.bfloat16),
             index_q_cos_sin_cache=torch.zeros(16, 64), index_weights=torch.zeros(4, 8, dtype=torch.bfloat16),
             index_weights_softmax_scale=128 ** -0.5, index_weights_head_scale=8 ** -0.5)
    a.update(over)
    return a


@pytest.mark.parametrize("bad,match", [
    (dict(positions=torch.zeros(4, 1, dtype=torch.int64)), 'positions must be 1D'),             # positions not 1D
    (dict(index_q=torch.zeros(4, 1024, dtype=torch.bfloat16)), 'index_q must be \\['),         # index_q not 3D
    (dict(index_q=torch.zeros(4, 8, 128, dtype=torch.float16)), 'bfloat16 with contiguous rows'),        # not bf16
    (dict(index_q=torch.zeros(3, 8, 128, dtype=torch.bfloat16)), 'fewer rows'),       # fewer rows than positions
    (dict(index_q_cos_sin_cache=torch.zeros(16, 32)), 'rope dim 64'),                  # rope dim not 64
    (dict(index_q_cos_sin_cache=torch.zeros(16, 64, dtype=torch.float64)), 'float32 or bfloat16'),
    (dict(index_weights=torch.zeros(4, 8, dtype=torch.float16)), 'bfloat16 or float32'),       # weights dtype
    (dict(index_weights=torch.zeros(4, 16, dtype=torch.bfloat16)), 'num_heads\\]'),     # weights per head count
    (dict(index_q=torch.zeros(4, 8, 192, dtype=torch.bfloat16)), 'head_dim 128'),       # head_dim not 128/256/512
    ({}, 'GPU'),                                                               # valid, but CPU tensors
])
def test_indexer_wrapper_asserts(bad, match):
    with pytest.raises(AssertionError, match=match):
        flaggems_vllm.fused_indexer_q_rope_quant(**_indexer_args(**bad))


def _slot_args(**over):
    a = dict(num_tokens=8, max_num_tokens=16, query_start_loc=torch.tensor([0, 4, 8], dtype=torch.int32),
             num_reqs=2, positions=torch.zeros(8, dtype=torch.int64), block_table=torch.zeros(2, 4, dtype=torch.int32),
             slot_mapping=torch.zeros(16, dtype=torch.int64), block_size=16)
    a.update(over)
    return a


@pytest.mark.parametrize("bad,match", [
    (dict(slot_mapping=torch.zeros(16, dtype=torch.int32)), 'contiguous int64'),            # not int64
    (dict(slot_mapping=torch.zeros(15, dtype=torch.int64)), 'max_num_tokens'),            # fewer than max_num_tokens
    (dict(query_start_loc=torch.tensor([0, 4, 8], dtype=torch.int64)), 'num_reqs \\+ 1'),  # not int32
    (dict(query_start_loc=torch.tensor([0, 4], dtype=torch.int32)), 'num_reqs \\+ 1'),    # fewer than num_reqs + 1
    (dict(positions=torch.zeros(8, dtype=torch.float32)), 'int32 or int64'),              # positions dtype
    (dict(block_table=torch.zeros(2, 4, dtype=torch.int64)), '2D int32'),           # block table not int32
    (dict(block_table=torch.zeros(2, 8, dtype=torch.int32)[:, ::2]), 'rows must be contiguous'),   # block-table rows not contiguous
    ({}, 'GPU'),                                                               # valid, but CPU tensors
])
def test_slot_mapping_wrapper_asserts(bad, match):
    with pytest.raises(AssertionError, match=match):
        flaggems_vllm.compute_slot_mapping_parallel(**_slot_args(**bad))


def test_product_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "flaggems-vllm_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "from oracle" not in text, f
                assert "liboracle" not in text, f


@pytest.mark.parametrize("shape,expected", [
    ((4, 64 * 584), (4, 64 * 584)),
    ((3, 16, 1, 584), (3, 16 * 584)),
    ((64 * 584 * 2,), (1, 64 * 584 * 2)),   # 1-D: one block of numel bytes
    ((100,), (1, 100)),
])
def test_main_cache_geometry(shape, expected):
    """Block count and stride handed to the C ABI.  A 1-D cache is one block,
    so the kernel's block bound (blk < num_blocks) skips every slot past
    cache_block_size instead of writing past the allocation."""
    from flaggems_vllm.ops.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert import cache_geometry

    assert cache_geometry(torch.zeros(shape, dtype=torch.uint8)) == expected
    # a padded 2-D view keeps its row stride
    padded = torch.zeros(4, 64 * 584 + 256, dtype=torch.uint8)[:, :64 * 584]
    assert cache_geometry(padded) == (4, 64 * 584 + 256)
