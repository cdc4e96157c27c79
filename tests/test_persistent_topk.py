"""persistent_topk: vLLM's decode top-k over rows of per-row lengths.

Reference: src/flaggems_vllm/ops/persistent_topk.py:2179-2342; tests
tests/test_persistent_topk.py:98-418 (STRIDE 262144, K 512, the heterogeneous,
k-value, MTP, boundary and data-distribution cases; the reference compares the
selected values with torch.topk's).  Here each row's index set is compared
with the C oracle's (values equal to the k-th largest taken lowest index
first), and the values with torch.topk's as the reference does.
"""
import pytest
import torch

import oracle

DEV = torch.device("cuda:0")
I32 = torch.int32
STRIDE, K = 262144, 512


def _hetero(lengths, seed=0, dist="random"):
    g = torch.Generator().manual_seed(seed)
    x = torch.full((len(lengths), STRIDE), float("-inf"))
    for i, n in enumerate(lengths):
        if dist == "random":
            x[i, :n] = torch.randn(n, generator=g)
        elif dist == "sorted_asc":
            x[i, :n] = torch.arange(n, dtype=torch.float32)
        elif dist == "sorted_desc":
            x[i, :n] = torch.arange(n, 0, -1, dtype=torch.float32)
        elif dist == "all_same":
            x[i, :n] = 1.0
        else:  # small_differences
            x[i, :n] = 1.0 + torch.randn(n, generator=g) * 1e-6
    return x


def _run(x, lengths, k=K, ws_bytes=2 << 20, max_seq_len=None, lengths_shape=None):
    from flaggems_vllm import persistent_topk

    lens = torch.tensor(lengths, dtype=I32)
    dl = lens.view(lengths_shape) if lengths_shape else lens
    out = torch.full((len(lengths), k), -7, dtype=I32, device=DEV)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    persistent_topk(x.to(DEV), dl.to(DEV), out, ws, k=k, max_seq_len=max_seq_len)
    torch.cuda.synchronize()
    exp = oracle.top_k_per_row(x, k, seq_lens=lens, next_n=1)
    got = out.cpu()
    short = (exp < 0).any(1)
    assert torch.equal(got[short], exp[short]), "rows of at most k values: 0..len-1 then -1"
    assert torch.equal(got[~short].sort(1).values, exp[~short]), "index sets differ from the oracle's"
    for i, n in enumerate(lengths):  # the reference's own check: the selected values equal torch.topk's
        v = got[i][got[i] >= 0].long()
        ref = x[i, :n].topk(min(k, n)).values.sort(descending=True).values
        assert torch.equal(x[i].gather(0, v).sort(descending=True).values, ref)
    return got


def test_asserts_like_the_reference():
    from flaggems_vllm import persistent_topk

    with pytest.raises(AssertionError):  # CPU tensors
        persistent_topk(torch.zeros(2, 8), torch.ones(2, dtype=I32), torch.zeros(2, 512, dtype=I32),
                        torch.empty(16, dtype=torch.uint8))


HETERO = [(1, [1, 1, 1, 1]), (1055, [1, 256, 515, 1055]), (4120, [4120]), (16390, [16383, 16384, 16385, 16390]),
          (20000, [8000, 16384, 20000]), (32772, [32767, 32768, 32769]), (32774, [32773, 32774]),
          (1048576, [262144]), (1048576, [1, 32773, 32773, 262144]), (1048576, [1, 1, 1, 262144]), (32, [1, 32])]


@pytest.mark.gpu
@pytest.mark.parametrize("max_seq_len,lengths", HETERO)
def test_gpu_heterogeneous(max_seq_len, lengths):
    """The reference's heterogeneous rows (-inf past each length)."""
    print(f"\n[case] persistent_topk {lengths}", flush=True)
    _run(_hetero(lengths, seed=len(lengths)), lengths, max_seq_len=max_seq_len)


@pytest.mark.gpu
@pytest.mark.parametrize("k", [1024, 2048])
@pytest.mark.parametrize("lengths,max_seq_len", [([262144], 1048576), ([32773, 32774], 32774)])
def test_gpu_k_values(k, lengths, max_seq_len):
    print(f"\n[case] persistent_topk k={k} {lengths}", flush=True)
    _run(_hetero(lengths, seed=k), lengths, k=k, max_seq_len=max_seq_len)


@pytest.mark.gpu
def test_gpu_mtp_lengths():
    """lengths [B, next_n] (MTP): one length per row."""
    print("\n[case] persistent_topk MTP", flush=True)
    _run(_hetero([32772, 32773], seed=3), [32772, 32773], max_seq_len=32774, lengths_shape=(1, 2))


@pytest.mark.gpu
@pytest.mark.parametrize("lengths", [[262144] * 5, [65535], [65536], [262144] * 40])
def test_gpu_boundary(lengths):
    """The reference's boundary cases, and 40 long rows (more than the split takes)."""
    print(f"\n[case] persistent_topk boundary {len(lengths)} x {lengths[0]}", flush=True)
    _run(_hetero(lengths, seed=5), lengths, max_seq_len=max(lengths))


@pytest.mark.gpu
@pytest.mark.parametrize("dist", ["sorted_asc", "sorted_desc", "all_same", "small_differences"])
def test_gpu_data_distributions(dist):
    print(f"\n[case] persistent_topk {dist}", flush=True)
    _run(_hetero([5000, 10000], seed=7, dist=dist), [5000, 10000], max_seq_len=10000)


@pytest.mark.gpu
def test_gpu_workspace_too_small_or_misaligned():
    """A workspace too small for the split (or not 16-byte aligned) leaves
    the rows streamed: the same index sets."""
    from flaggems_vllm import persistent_topk

    print("\n[case] persistent_topk workspace", flush=True)
    lengths = [262144, 200000, 262144]
    x = _hetero(lengths, seed=9)
    big = _run(x, lengths, ws_bytes=2 << 20)
    small = _run(x, lengths, ws_bytes=16)
    assert torch.equal(big.sort(1).values, small.sort(1).values)
    buf = torch.empty((2 << 20) + 8, dtype=torch.uint8, device=DEV)
    out = torch.empty(3, K, dtype=I32, device=DEV)
    persistent_topk(x.to(DEV), torch.tensor(lengths, dtype=I32, device=DEV), out, buf[8:], k=K)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().sort(1).values, big.sort(1).values)


@pytest.mark.gpu
def test_gpu_torch_op():
    """torch.ops.flaggems_vllm.persistent_topk writes the function's sets."""
    import flaggems_vllm  # noqa: F401

    lengths = [70000, 300]
    x = _hetero(lengths, seed=11).to(DEV)
    lens = torch.tensor(lengths, dtype=I32, device=DEV)
    out = torch.empty(2, K, dtype=I32, device=DEV)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    torch.ops.flaggems_vllm.persistent_topk(x, lens, out, ws, K, None)
    torch.cuda.synchronize()
    exp = oracle.top_k_per_row(x.cpu(), K, seq_lens=lens.cpu())
    assert torch.equal(out.cpu()[0].sort().values, exp[0])
    assert torch.equal(out.cpu()[1], exp[1])


@pytest.mark.gpu
def test_gpu_torch_op_split_rows_opcheck():
    """Rows long enough to split write their candidates into the workspace:
    the schema declares it written, and opcheck's schema test (which flags an
    undeclared mutation) passes on that path."""
    from flaggems_vllm import _native

    print("\n[case] persistent_topk torch.ops split path opcheck", flush=True)
    lengths = [262144, 250000, 262144, 200000]
    need = _native.lib().fgv_top_k_per_row_workspace_bytes(len(lengths), STRIDE, K)
    assert need > 0, "the rows must take the split path"
    x = _hetero(lengths, seed=13).to(DEV)
    lens = torch.tensor(lengths, dtype=I32, device=DEV)
    out = torch.empty(len(lengths), K, dtype=I32, device=DEV)
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    torch.ops.flaggems_vllm.persistent_topk(x, lens, out, ws, K, None)
    torch.cuda.synchronize()
    assert bool(ws.any()), "the split path leaves candidates in the workspace"
    exp = oracle.top_k_per_row(x.cpu(), K, seq_lens=lens.cpu())
    assert torch.equal(out.cpu().sort(1).values, exp)
    torch.library.opcheck(torch.ops.flaggems_vllm.persistent_topk.default, (x, lens, out, ws, K, None),
                          test_utils=("test_schema", "test_faketensor"))
