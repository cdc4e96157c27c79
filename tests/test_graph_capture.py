"""Every op inside a captured HIP graph: each launches on the caller's current
stream, allocates nothing outside torch's allocator, records no memset, and
reads no device value back to the host, so a graph of one call replays it.
Each graph is replayed several times, with the inputs reset and other eager
work between replays, and every replay must equal the eager call bit for bit.
"""
import pytest
import torch

import flaggems_vllm
from flaggems_vllm import testing as W

from .test_gather import _ref_fixture
from .test_indexer import _case as _indexer_case
from .test_slot_mapping import _ragged_inputs

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
REPLAYS = 4


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _bits(t):
    return t.view(torch.uint8) if t.element_size() == 1 else t.view(torch.int16 if t.element_size() == 2
                                                                    else torch.int32 if t.element_size() == 4
                                                                    else torch.int64)


def _flat(x):
    if isinstance(x, (tuple, list)):
        return [y for e in x for y in _flat(e)]
    return [x] if isinstance(x, torch.Tensor) else []


def replay_matches_eager(reset, run, outputs=None):
    """reset() restores the inputs (eagerly); run() makes one call and returns
    its output tensors; `outputs` (if given) returns the tensors an in-place
    op writes.  Checks REPLAYS graph replays against one eager call."""
    pick = outputs or (lambda res: res)
    reset()
    expect = [t.clone() for t in _flat(pick(run()))]
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the capture, as torch asks
        reset()
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    reset()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        got = _flat(pick(run()))
    for i in range(REPLAYS):
        reset()
        torch.randn(1 << 20, device=DEV).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k, (g, e) in enumerate(zip(got, expect)):
            assert torch.equal(_bits(g), _bits(e)), f"replay {i}, output {k} differs from the eager call"


def test_graph_main_op():
    _say("graph: main op, configs 0 and 1")
    for cfg in (0, 1):
        w0 = W.make_workload(cfg).to(DEV)
        w = w0.clone()

        def reset():
            w.q.copy_(w0.q)
            w.k_cache.copy_(w0.k_cache)

        replay_matches_eager(
            reset,
            lambda: flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(*w.args()),
            outputs=lambda _: (w.q, w.k_cache))


@pytest.mark.parametrize("tma", [False, True])
def test_graph_sibling(tma):
    _say(f"graph: sibling tma={tma}")
    w = W.make_inv_rope_workload(37, 64, 8, seed=1).to(DEV)
    replay_matches_eager(lambda: None, lambda: flaggems_vllm.fused_inv_rope_fp8_quant(
        w.o, w.positions, w.cos_sin_cache, w.n_groups, w.heads_per_group, tma_aligned_scales=tma))


def test_graph_rmsnorm_indexer_gather_slots():
    _say("graph: rmsnorm, indexer (FP8, MXFP4), gather, slot mapping")
    g = torch.Generator().manual_seed(6)
    qr, kv = W.randn_bf16((33, 1536), g).to(DEV), W.randn_bf16((33, 512), g).to(DEV)
    qw, kw = W.randn_bf16((1536,), g).to(DEV), W.randn_bf16((512,), g).to(DEV)
    replay_matches_eager(lambda: None, lambda: flaggems_vllm.fused_q_kv_rmsnorm(qr, kv, qw, kw, 1e-6))

    pos, q, cs, wt, sm, hs = _indexer_case(11, seed=5)
    pos, q, cs, wt = pos.to(DEV), q.to(DEV), cs.to(DEV), wt.to(DEV)
    for fp4 in (False, True):
        replay_matches_eager(lambda: None, lambda: flaggems_vllm.fused_indexer_q_rope_quant(
            pos, q, cs, wt, sm, hs, use_fp4=fp4))

    cache, expected, seq_lens, gather_lens, bt, _ = _ref_fixture(2, 12, 5, 64, 448, 64)
    out = torch.zeros_like(expected, device=DEV)
    gargs = (cache.to(DEV), seq_lens.to(DEV), gather_lens.to(DEV), bt.to(DEV), 64)
    replay_matches_eager(lambda: out.fill_(7), lambda: flaggems_vllm.dequantize_and_gather_k_cache(out, *gargs),
                         outputs=lambda _: (out,))
    assert torch.equal(out.cpu(), expected)

    qsl, p, table = _ragged_inputs(2)
    n = int(qsl[-1])
    slots = torch.full((n + 5,), -7, dtype=torch.int64, device=DEV)
    sargs = (n, n + 5, qsl.to(DEV), qsl.numel() - 1, p.to(DEV), table.to(DEV))
    replay_matches_eager(lambda: slots.fill_(-7),
                         lambda: flaggems_vllm.compute_slot_mapping_parallel(*sargs, slots, 16),
                         outputs=lambda _: (slots,))


@pytest.mark.parametrize("extra", [False, True, "paired"])
def test_graph_sparse_mla(extra):
    """Decode over the main list; with `extra`, a long extra list that takes
    the expanded cache and the split grid + combine kernel (workspace
    allocated by the wrapper inside the capture); "paired": long lists over
    300 items, the paired grid."""
    _say(f"graph: sparse MLA extra={extra}")
    if extra == "paired":
        w = W.make_mla_workload(batch=300, topk=2048, num_pages=16, seed=9, q_scale=0.1)
        w.topk_length = torch.randint(0, 200, (300,), generator=torch.Generator().manual_seed(1), dtype=torch.int32)
        w = w.to(DEV)
        from flaggems_vllm import _native

        assert _native.lib().fgv_sparse_mla_decode_grid(300, 1, 64, 2048, 0) == 2
        extra = False
    else:
        kw = dict(extra_topk=2048, extra_page=2, extra_pages=256) if extra else {}
        w = W.make_mla_workload(batch=8, topk=128, num_pages=16, seed=9, q_scale=0.1, **kw).to(DEV)
    meta, _ = flaggems_vllm.get_mla_metadata()
    B, SQ, HQ = w.q.shape[:3]
    if extra:
        from flaggems_vllm import _native

        query = _native.lib().fgv_sparse_mla_decode_workspace_bytes
        entries = w.extra_k_cache.shape[0] * w.extra_k_cache.shape[1]
        split_only = query(B, SQ, HQ, 128, 2048, 0)
        assert split_only > 0 and query(B, SQ, HQ, 128, 2048, entries) > split_only, \
            "this case is meant to take the split grid and the expanded cache"
    out = torch.empty(B, SQ, HQ, 512, dtype=torch.bfloat16, device=DEV)
    replay_matches_eager(lambda: out.fill_(3.0), lambda: flaggems_vllm.flash_mla_with_kvcache(
        w.q, w.k_cache, None, None, 512, meta, is_fp8_kvcache=True, indices=w.indices, out=out,
        **w.kwargs()))


def test_graph_topk_index_ops():
    """compute_global_topk_indices_and_lens and combine_topk_swa_indices (their
    outputs allocated by the wrappers inside the capture)."""
    _say("graph: global top-k indices, combine top-k + window")
    g = torch.Generator().manual_seed(4)
    local = torch.randint(-1, 64 * 20, (300, 128), generator=g, dtype=torch.int32).to(DEV)
    req = torch.randint(0, 4, (300,), generator=g, dtype=torch.int32).to(DEV)
    bt = torch.randint(0, 5000, (4, 20), generator=g, dtype=torch.int32).to(DEV)
    replay_matches_eager(lambda: None, lambda: flaggems_vllm.compute_global_topk_indices_and_lens(
        local, req, bt, 64))
    qsl = torch.tensor([0, 100, 300], dtype=torch.int32, device=DEV)
    seq = torch.tensor([4000, 900], dtype=torch.int32, device=DEV)
    gat = torch.tensor([1000, 500], dtype=torch.int32, device=DEV)
    replay_matches_eager(lambda: None, lambda: flaggems_vllm.combine_topk_swa_indices(
        local, qsl, seq, gat, 128, 4, 128, 45056, 40960))


def test_graph_top_k_per_row():
    """top_k_per_row_decode over rows held in LDS and over long rows; the
    captured replays select the same index sets as the eager call (their
    order within a row may differ from call to call)."""
    _say("graph: top_k_per_row decode")
    g = torch.Generator().manual_seed(8)
    for V in (5000, 70000):
        lg = torch.randn(9, V, generator=g).to(DEV)
        seq = torch.full((9,), V, dtype=torch.int32, device=DEV)
        idx = torch.empty(9, 512, dtype=torch.int32, device=DEV)
        run = lambda: (flaggems_vllm.top_k_per_row_decode(lg, 1, seq, idx, 9, lg.stride(0), 1, 512),
                       idx.sort(1).values)[1]
        replay_matches_eager(lambda: idx.fill_(-5), run)


def test_graph_fp8_einsum():
    """fp8_einsum on its three schedules (b 4: skinny; b 200: tiled; b 100
    with 16 K blocks: split-K, its workspace allocated inside the capture)
    into a preallocated output; the replays give the eager bytes."""
    from flaggems_vllm import _native
    from .test_fp8_einsum import random_inputs

    _say("graph: fp8_einsum")
    assert _native.lib().fgv_fp8_einsum_workspace_bytes(100, 2, 2048, 256) > 0
    for b, r in ((4, 1024), (200, 1024), (100, 2048)):
        x, xs, y, ys = (t.to(DEV) for t in random_inputs(b, 2, r, 256, seed=b))
        out = torch.empty((b, 2, 256), dtype=torch.bfloat16, device=DEV)
        run = lambda: flaggems_vllm.fp8_einsum("bhr,hdr->bhd", x, xs, y, ys, out=out)
        replay_matches_eager(lambda: out.fill_(7.0), run)


@pytest.mark.parametrize("d_qk", [512, 576])
def test_graph_flash_mla_sparse(d_qk):
    """Sparse prefill (outputs allocated inside the capture) with the sink and
    top-k lengths; the replays give the eager bytes of all three outputs."""
    _say(f"graph: flash_mla_sparse_fwd d_qk={d_qk}")
    w = W.make_mla_sparse_inputs(40, 700, 256, h_q=128, d_qk=d_qk, have_attn_sink=True, have_topk_length=True,
                                 seed=d_qk).to(DEV)
    replay_matches_eager(lambda: None, lambda: flaggems_vllm.flash_mla_sparse_fwd(*w.args()))
