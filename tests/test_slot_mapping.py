"""compute_slot_mapping_parallel: CPU pins of its oracle and GPU parity.

Reference: src/flaggems_vllm/runtime/backend/_ascend/ops/slot_mapping.py:42-144 and
tests/test_slot_mapping.py:27-111 (the FULL_CASES shapes below, per-request
reference ``_ref_slot_mapping``).
"""
import pytest
import torch

import oracle
from flaggems_vllm import testing as W
from oracle import torch_ref

DEV = torch.device("cuda:0")

# reqs, tokens per request, max tokens, block size (reference tests/test_slot_mapping.py:31-43)
REF_CASES = [(4, 200, 8192, 128), (8, 200, 8192, 128), (12, 200, 8192, 128), (16, 200, 8192, 128),
             (4, 200, 8192, 16), (32, 200, 8192, 128), (128, 64, 8192, 128), (8, 200, 8192, 16),
             (8, 200, 16384, 128), (1, 200, 8192, 128)]


def _ref_inputs(nreq, tlen, bs):
    """The reference test's inputs: positions 0..tlen-1 per request, block
    table arange % 900."""
    qsl = torch.arange(nreq + 1, dtype=torch.int32) * tlen
    pos = torch.cat([torch.arange(tlen, dtype=torch.int32) for _ in range(nreq)])
    maxb = (nreq * tlen + bs - 1) // bs + 1
    bt = (torch.arange(nreq * maxb, dtype=torch.int32).reshape(nreq, maxb) % 900)
    return qsl, pos, bt


def _ragged_inputs(seed, nreq=9, bs=16, cpw=1):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(0, 50, (nreq,), generator=g)
    qsl = torch.zeros(nreq + 1, dtype=torch.int32)
    qsl[1:] = torch.cumsum(lens, 0).to(torch.int32)
    starts = torch.randint(0, 300, (nreq,), generator=g)
    pos = torch.cat([s + torch.arange(int(n)) for s, n in zip(starts.tolist(), lens.tolist())]).to(torch.int64)
    maxb = (400 + bs * cpw - 1) // (bs * cpw)
    bt = torch.randint(0, 5000, (nreq, maxb), generator=g, dtype=torch.int32)
    return qsl, pos, bt


def _run_oracle(num_tokens, max_tokens, qsl, pos, bt, bs, **kw):
    out = torch.full((max_tokens,), -7, dtype=torch.int64)
    oracle.compute_slot_mapping(num_tokens, max_tokens, qsl, qsl.numel() - 1, pos, bt, out, bs, **kw)
    return out


@pytest.mark.parametrize("case", REF_CASES)
def test_oracle_vs_reference_loop(case):
    nreq, tlen, maxtok, bs = case
    qsl, pos, bt = _ref_inputs(nreq, tlen, bs)
    n = nreq * tlen
    out = _run_oracle(n, maxtok, qsl, pos, bt, bs)
    assert torch.equal(out, torch_ref.slot_mapping(n, qsl, pos, bt, bs, max_num_tokens=maxtok))
    assert bool((out[n:] == -1).all())


@pytest.mark.parametrize("cpw,rank,il", [(1, 0, 1), (2, 0, 1), (2, 1, 1), (4, 3, 2), (2, 1, 4)])
def test_oracle_context_parallel(cpw, rank, il):
    qsl, pos, bt = _ragged_inputs(cpw * 10 + rank, cpw=cpw)
    n = int(qsl[-1])
    out = _run_oracle(n, n + 37, qsl, pos, bt, 16, cp_world_size=cpw, cp_rank=rank,
                      cp_kv_cache_interleave_size=il)
    want = torch_ref.slot_mapping(n, qsl, pos, bt, 16, max_num_tokens=n + 37, cp_world_size=cpw,
                                  cp_rank=rank, interleave=il)
    assert torch.equal(out, want)
    # every position is local to exactly one rank
    if cpw > 1:
        owners = torch.zeros(n, dtype=torch.int64)
        for rk in range(cpw):
            o = _run_oracle(n, n, qsl, pos, bt, 16, cp_world_size=cpw, cp_rank=rk,
                            cp_kv_cache_interleave_size=il)
            owners += (o >= 0).long()
        assert bool((owners == 1).all())


def test_oracle_reproduces_workload_slots():
    """The paged slots the c2 workload builds from its block tables are what
    slot-mapping generation computes from the same tables."""
    w = W.make_workload(2)
    m = w.meta
    qsl = torch.zeros(m["new_lens"].numel() + 1, dtype=torch.int32)
    qsl[1:] = torch.cumsum(m["new_lens"], 0)
    out = _run_oracle(w.num_tokens, w.num_tokens, qsl, w.position_ids, m["block_table"], 64)
    assert torch.equal(out, w.slot_mapping)


# ------------------------------------------------------------------- GPU ----

def _gpu(num_tokens, max_tokens, qsl, pos, bt, bs, **kw):
    import flaggems_vllm

    out = torch.full((max_tokens,), -7, dtype=torch.int64, device=DEV)
    flaggems_vllm.compute_slot_mapping_parallel(num_tokens, max_tokens, qsl.to(DEV), qsl.numel() - 1,
                                                pos.to(DEV), bt.to(DEV), out, bs, **kw)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.gpu
@pytest.mark.parametrize("case", REF_CASES)
def test_gpu_reference_cases(case):
    print(f"\n[case] slot mapping {case}", flush=True)
    nreq, tlen, maxtok, bs = case
    qsl, pos, bt = _ref_inputs(nreq, tlen, bs)
    n = nreq * tlen
    assert torch.equal(_gpu(n, maxtok, qsl, pos, bt, bs), _run_oracle(n, maxtok, qsl, pos, bt, bs))


@pytest.mark.gpu
@pytest.mark.parametrize("cpw,rank,il", [(1, 0, 1), (2, 1, 1), (4, 3, 2)])
def test_gpu_ragged_and_context_parallel(cpw, rank, il):
    print(f"\n[case] slot mapping cp {cpw} {rank} {il}", flush=True)
    qsl, pos, bt = _ragged_inputs(cpw * 10 + rank, cpw=cpw)
    n = int(qsl[-1])
    kw = dict(cp_world_size=cpw, cp_rank=rank, cp_kv_cache_interleave_size=il)
    for p in (pos, pos.to(torch.int32)):
        assert torch.equal(_gpu(n, n + 37, qsl, p, bt, 16, **kw), _run_oracle(n, n + 37, qsl, p, bt, 16, **kw))


@pytest.mark.gpu
@pytest.mark.parametrize("config", [2, 4])
def test_gpu_reproduces_workload_slots(config):
    print(f"\n[case] slot mapping workload c{config}", flush=True)
    w = W.make_workload(config)
    m = w.meta
    qsl = torch.zeros(m["new_lens"].numel() + 1, dtype=torch.int32)
    qsl[1:] = torch.cumsum(m["new_lens"], 0)
    out = _gpu(w.num_tokens, w.num_tokens + 100, qsl, w.position_ids, m["block_table"], 64)
    want = _run_oracle(w.num_tokens, w.num_tokens + 100, qsl, w.position_ids, m["block_table"], 64)
    assert torch.equal(out, want)
    keep = w.slot_mapping >= 0  # c4 pads 10% of its slots afterwards
    assert torch.equal(out[:w.num_tokens][keep], w.slot_mapping[keep])
