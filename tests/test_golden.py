"""Committed small vectors (tests/golden/dsv4_small.pt, written by
tests/golden/make_golden.py from the torch restatement of the reference
oracle) reproduced by the C oracle, the torch restatement and, on a GPU, the
HIP kernels, all bit for bit."""
import os

import pytest
import torch

import oracle
from flaggems_vllm import testing as W
from oracle import torch_ref

from ._helpers import slot_byte_index

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dsv4_small.pt")


@pytest.fixture(scope="module")
def gold():
    return torch.load(GOLDEN, weights_only=True)


def _main_inputs(g):
    cs = W.make_cos_sin_cache(int(g["main.max_pos"]))
    assert torch.equal(cs[g["main.cos_sin_row_ids"]], g["main.cos_sin_rows"]), "cos/sin formula drifted"
    cache = torch.zeros(int(g["main.num_blocks"]), 64 * 584, dtype=torch.uint8)
    return W.Workload("golden", g["main.q"].clone(), g["main.kv"].clone(), cache,
                      g["main.slot_mapping"].clone(), g["main.position_ids"].clone(), cs, 1e-6, 64)


def _check_main(g, q, cache):
    slots = g["main.slot_mapping"][g["main.slot_mapping"] >= 0]
    idx = slot_byte_index(slots, 64, 64 * 584)
    assert torch.equal(q, g["main.out.q"])
    assert torch.equal(cache.view(-1)[idx], g["main.out.slot_bytes"])
    assert int(torch.count_nonzero(cache)) == int(g["main.out.cache_nonzero"])


def test_c_oracle_reproduces_golden(gold):
    w = _main_inputs(gold)
    oracle.qnorm_rope_kv_insert(*w.args())
    _check_main(gold, w.q, w.k_cache)


def test_torch_ref_reproduces_golden(gold):
    w = _main_inputs(gold)
    torch_ref.qnorm_rope_kv_insert(*w.args())
    _check_main(gold, w.q, w.k_cache)


def _inv_inputs(g):
    cs = W.make_cos_sin_cache(4096)
    assert torch.equal(cs[g["inv.cos_sin_row_ids"]], g["inv.cos_sin_rows"])
    return g["inv.o"], g["inv.positions"], cs


@pytest.mark.parametrize("tma", [False, True])
def test_sibling_oracles_reproduce_golden(gold, tma):
    o, pos, cs = _inv_inputs(gold)
    f8, sc = oracle.inv_rope_fp8_quant(o, pos, cs, 2, 8, tma_aligned_scales=tma)
    t8, ts = torch_ref.inv_rope_fp8_quant(o, pos, cs, 2, 8, tma_aligned_scales=tma)
    key8, keys = ("inv.out.fp8_tma", "inv.out.scale_packed") if tma else ("inv.out.fp8", "inv.out.scale_f32")
    assert torch.equal(f8.contiguous(), gold[key8]) and torch.equal(t8, gold[key8])
    assert torch.equal(sc.contiguous(), gold[keys]) and torch.equal(ts, gold[keys])


@pytest.mark.gpu
def test_hip_reproduces_golden(gold):
    import flaggems_vllm

    dev = torch.device("cuda:0")
    w = _main_inputs(gold).to(dev)
    flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(*w.args())
    torch.cuda.synchronize()
    _check_main(gold, w.q.cpu(), w.k_cache.cpu())
    o, pos, cs = _inv_inputs(gold)
    for tma, key8, keys in ((False, "inv.out.fp8", "inv.out.scale_f32"),
                            (True, "inv.out.fp8_tma", "inv.out.scale_packed")):
        f8, sc = flaggems_vllm.fused_inv_rope_fp8_quant(o.to(dev), pos.to(dev), cs.to(dev), 2, 8,
                                                        tma_aligned_scales=tma)
        torch.cuda.synchronize()
        assert torch.equal(f8.cpu().view(torch.uint8).contiguous(), gold[key8])
        assert torch.equal(sc.cpu().contiguous(), gold[keys])
