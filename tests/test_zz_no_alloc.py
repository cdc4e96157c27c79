"""fgv_sparse_mla_decode_model1_no_alloc: the sparse MLA decode with its
workspace in the library's fixed device scratch instead of a caller buffer.

It has no counterpart in the reference; it is for callers that cannot
allocate (HIP graph capture, serving loops).  Its output must equal
fgv_sparse_mla_decode_model1's with the workspace that call's query asks for,
bit for bit (same schedule), on consecutive calls that reuse the scratch (the
second smaller than the first), and under graph replay; a call whose
workspace does not fit the 64 MiB scratch is refused before anything runs.
"""
import ctypes

import pytest
import torch

from flaggems_vllm import _native
from flaggems_vllm import testing as W

DEV = torch.device("cuda:0")
SCRATCH = 64 << 20
FGV_E_TOO_LARGE = -5


def _args(d, out, lse):
    """The argument list shared by both entry points, up to the workspace."""
    B, SQ, HQ, _ = d.q.shape
    ek, ei = d.extra_k_cache, d.extra_indices
    ptr = lambda t: t.data_ptr() if t is not None else None
    return [
        d.q.data_ptr(), d.q.stride(0), d.q.stride(1), d.q.stride(2),
        d.k_cache.data_ptr(), d.k_cache.stride(0), d.k_cache.shape[0], d.k_cache.shape[1],
        d.indices.data_ptr(), d.indices.stride(0), d.indices.stride(1), d.indices.shape[-1],
        ptr(d.topk_length),
        ptr(ek), ek.stride(0) if ek is not None else 0, ek.shape[0] if ek is not None else 0,
        ek.shape[1] if ek is not None else 1,
        ptr(ei), ei.stride(0) if ei is not None else 0, ei.stride(1) if ei is not None else 0,
        ei.shape[-1] if ei is not None else 0,
        ptr(d.extra_topk_length), ptr(d.attn_sink), 512 ** -0.5,
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        lse.data_ptr(), lse.stride(0), lse.stride(1), B, SQ, HQ]


def _workspace_bytes(d):
    B, SQ, HQ, _ = d.q.shape
    ek, ei = d.extra_k_cache, d.extra_indices
    entries = ek.shape[0] * ek.shape[1] if ek is not None else 0
    etopk = ei.shape[-1] if ei is not None else 0
    return _native.lib().fgv_sparse_mla_decode_workspace_bytes(B, SQ, HQ, d.indices.shape[-1], etopk, entries)


def _outputs(d, fill):
    B, SQ, HQ, _ = d.q.shape
    out = torch.full((B, SQ, HQ, 512), fill, dtype=torch.bfloat16, device=DEV)
    lse = torch.full((B, HQ, SQ), fill, dtype=torch.float32, device=DEV)
    return out, lse


def _with_workspace(d):
    """The existing entry point with a torch-allocated workspace of the
    queried size."""
    out, lse = _outputs(d, 3.0)
    nbytes = _workspace_bytes(d)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=DEV)
    rc = _native.lib().fgv_sparse_mla_decode_model1(*_args(d, out, lse), ws.data_ptr(), nbytes,
                                                    torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return out, lse, nbytes


def _no_alloc(d, out, lse):
    return _native.lib().fgv_sparse_mla_decode_model1_no_alloc(*_args(d, out, lse),
                                                               torch.cuda.current_stream().cuda_stream)


def _expanded_case(batch, topk, pages, extra_topk, extra_pages, seed):
    """An extra cache gathered 8 times per entry, so the call expands it into
    the workspace (and, with long lists, would split)."""
    w = W.make_mla_workload(batch=batch, topk=topk, num_pages=pages, extra_topk=extra_topk, extra_page=64,
                            extra_pages=extra_pages, seed=seed, q_scale=0.1)
    return w.to(DEV)


@pytest.mark.gpu
def test_gpu_no_alloc_matches_workspace_entry_on_consecutive_calls():
    """Two calls in a row through the scratch, the second smaller: both equal
    the workspace entry point's output and LSE bit for bit."""
    cases = [("first: batch 64, extra top-k 512 over 4096 entries", _expanded_case(64, 128, 16, 512, 64, 71)),
             ("second, smaller: batch 16, extra top-k 256 over 512 entries", _expanded_case(16, 64, 4, 256, 8, 72))]
    for name, d in cases:
        print(f"\n[case] no-alloc MLA {name}", flush=True)
        need = _workspace_bytes(d)
        assert 0 < need <= SCRATCH, need
        ref_out, ref_lse, _ = _with_workspace(d)
        out, lse = _outputs(d, 5.0)
        rc = _no_alloc(d, out, lse)
        assert rc == 0, (rc, _native.lib().fgv_last_error())
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), name
        assert torch.equal(lse.view(torch.int32), ref_lse.view(torch.int32)), name


@pytest.mark.gpu
def test_gpu_no_alloc_without_workspace_need_and_graph_replay():
    """A decode call whose schedule needs no workspace, then the expanded case
    captured in a HIP graph and replayed three times with other eager work
    (another no-alloc call on the same scratch) in between: every replay
    equals the workspace entry point."""
    d0 = W.make_mla_workload(batch=8, topk=128, num_pages=16, seed=73).to(DEV)
    assert _workspace_bytes(d0) == 0
    print("\n[case] no-alloc MLA decode without workspace need", flush=True)
    ref_out, ref_lse, _ = _with_workspace(d0)
    out, lse = _outputs(d0, 5.0)
    assert _no_alloc(d0, out, lse) == 0
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
    assert torch.equal(lse.view(torch.int32), ref_lse.view(torch.int32))

    print("[case] no-alloc MLA graph replay", flush=True)
    d = _expanded_case(32, 128, 16, 512, 32, 74)
    other = _expanded_case(16, 64, 4, 256, 8, 75)
    ref_out, ref_lse, _ = _with_workspace(d)
    out, lse = _outputs(d, 5.0)
    assert _no_alloc(d, out, lse) == 0          # eager first (the scratch address is looked up here)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert _no_alloc(d, out, lse) == 0
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        rc = _no_alloc(d, out, lse)
    assert rc == 0
    o2, l2 = _outputs(other, 5.0)
    for i in range(3):
        out.fill_(7.0)
        lse.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), f"replay {i}"
        assert torch.equal(lse.view(torch.int32), ref_lse.view(torch.int32)), f"replay {i}"
        assert _no_alloc(other, o2, l2) == 0     # eager work on the same scratch between replays
        torch.cuda.synchronize()


@pytest.mark.gpu
def test_gpu_no_alloc_refuses_what_does_not_fit():
    """A call long enough for the split grid (its partial slots exceed the
    scratch) is refused with FGV_E_TOO_LARGE and writes nothing."""
    d = W.make_mla_workload(batch=4, topk=2048, num_pages=40, seed=76).to(DEV)
    assert _workspace_bytes(d) > SCRATCH
    print("\n[case] no-alloc MLA refusal", flush=True)
    out, lse = _outputs(d, 5.0)
    rc = _no_alloc(d, out, lse)
    torch.cuda.synchronize()
    assert rc == FGV_E_TOO_LARGE
    assert b"64 MiB" in _native.lib().fgv_last_error()
    assert bool((out == 5.0).all()) and bool((lse == 5.0).all())
