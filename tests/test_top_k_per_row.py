"""top_k_per_row_decode / top_k_per_row_prefill: the sparse indexer's top-k.

Reference: src/flaggems_vllm/ops/top_k_per_row_decode.py:877-1043, 1263-1399;
src/flaggems_vllm/ops/top_k_per_row_prefill.py:1232-1331; tests
tests/test_top_k_per_row_decode.py:98-260 and tests/test_top_k_per_row_prefill.py:79-260
(their torch.topk references and shapes), benchmark shapes
benchmark/test_top_k_per_row_decode.py:70-83, benchmark/test_top_k_per_row_prefill.py:122-132.

The reference's own check is value-based (the selected values, sorted, equal
torch.topk's).  Here the bar is stronger: equal values are taken lowest index
first, so each row's selected index set is exact; it is compared, sorted,
with the oracle's (a sort of the whole row), and the values with torch.topk's.
"""
import pytest
import torch

import oracle

DEV = torch.device("cuda:0")
I32 = torch.int32


# ------------------------------------------------------------- oracle ----

def test_oracle_small_known_answers():
    x = torch.tensor([[3., 1., 4., 1., 5., 9., 2., 6.]])
    n = torch.tensor([8], dtype=I32)
    assert oracle.top_k_per_row(x, 3, seq_lens=n).tolist() == [[4, 5, 7]]          # 5, 9, 6
    assert oracle.top_k_per_row(x, 2, seq_lens=torch.tensor([4], dtype=I32)).tolist() == [[0, 2]]  # of 3 1 4 1
    # ties at the k-th value: lowest index first
    assert oracle.top_k_per_row(torch.ones(1, 6), 2, seq_lens=torch.tensor([6], dtype=I32)).tolist() == [[0, 1]]
    y = torch.tensor([[1., 7., 7., 2., 7., 7.]])
    assert oracle.top_k_per_row(y, 3, seq_lens=torch.tensor([6], dtype=I32)).tolist() == [[1, 2, 4]]
    # NaN above +inf, -inf below everything, -0 == +0 (index order)
    z = torch.tensor([[float("-inf"), float("inf"), float("nan"), -0.0, 0.0, -1.0]])
    assert oracle.top_k_per_row(z, 2, seq_lens=torch.tensor([6], dtype=I32)).tolist() == [[1, 2]]
    assert oracle.top_k_per_row(z, 4, seq_lens=torch.tensor([6], dtype=I32)).tolist() == [[1, 2, 3, 4]]
    # short rows: 0..len-1 then -1; prefill indices relative to the row start
    assert oracle.top_k_per_row(x, 5, seq_lens=torch.tensor([3], dtype=I32)).tolist() == [[0, 1, 2, -1, -1]]
    s, e = torch.tensor([2], dtype=I32), torch.tensor([7], dtype=I32)
    assert oracle.top_k_per_row(x, 2, row_starts=s, row_ends=e).tolist() == [[2, 3]]   # 5, 9 of 4 1 5 9 2


def test_oracle_against_torch_topk_values():
    """The oracle's selected values equal torch.topk's (the reference test's
    check), over decode rows with next_n = 2 and prefill rows with ragged
    ranges, ties and infinities included."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(12, 3000, generator=g)
    x[3] = torch.randint(0, 3, (3000,), generator=g).float()  # heavy ties
    x[5, ::3] = float("-inf")
    seq = torch.tensor([3000, 700, 64, 1500, 2999, 100], dtype=I32)
    k = 100
    o = oracle.top_k_per_row(x, k, seq_lens=seq, next_n=2)
    for r in range(12):
        n = int(seq[r // 2]) - 2 + r % 2 + 1
        row = x[r, :n]
        if n <= k:
            assert o[r].tolist() == list(range(n)) + [-1] * (k - n)
            continue
        assert torch.equal(row[o[r].long()].sort().values, row.topk(k).values.sort().values)
    st = torch.randint(0, 1500, (12,), generator=g, dtype=I32)
    en = st + torch.randint(0, 1500, (12,), generator=g, dtype=I32)
    o = oracle.top_k_per_row(x, k, row_starts=st, row_ends=en)
    for r in range(12):
        row = x[r, int(st[r]):int(en[r])]
        if row.numel() <= k:
            continue
        assert torch.equal(row[o[r].long()].sort().values, row.topk(k).values.sort().values)


def test_c_abi_rejects_bad_arguments():
    from flaggems_vllm import _native

    L = _native.lib()
    p = 1 << 12  # never dereferenced
    d = L.fgv_top_k_per_row_decode
    assert d(p, 64, 1, 4, 64, 0, p, p, 8, 1, 8, None, 0, None) == -2        # next_n 0
    assert d(p, 64, 1, -1, 64, 1, p, p, 8, 1, 8, None, 0, None) == -2       # negative rows
    assert d(None, 64, 1, 4, 64, 1, p, p, 8, 1, 8, None, 0, None) == -1
    assert d(p + 2, 64, 1, 4, 64, 1, p, p, 8, 1, 8, None, 0, None) == -3
    assert d(p, 64, 1, 4, 64, 1, None, p, 8, 1, 8, None, 0, None) == -1     # no seq_lens
    assert d(p, 64, 1, 4, 64, 1, p, p, 8, 1, 0, None, 0, None) == 0         # top_k 0: nothing to do
    w = L.fgv_top_k_per_row_workspace_bytes
    assert w(32, 262144, 512) == 32 * 16 * 512 * 8      # 16 parts of 16384, 512 part workgroups
    assert w(1, 200000, 512) == 13 * 512 * 8
    assert w(33, 262144, 512) == 0 and w(496, 262144, 512) == 0   # more than two part workgroups per CU (256)
    assert w(1, 180224, 512) == 0 and w(64, 129280, 1024) == 0    # under 12 parts: streamed
    assert w(1, 16384, 1024) == 0 and w(4, 262144, 1024) == 0     # one part; 16 x 1024 over the merge's 8192
    f = L.fgv_top_k_per_row_prefill
    assert f(p, 64, 1, 4, 64, None, p, p, 8, 1, 8, None, 0, None) == -1
    assert f(p, 64, 1, 0, 64, p, p, p, 8, 1, 8, None, 0, None) == 0


def test_wrapper_asserts_like_the_reference():
    import flaggems_vllm

    x = torch.zeros(4, 16)
    with pytest.raises(AssertionError):  # num_rows must equal logits.shape[0]
        flaggems_vllm.top_k_per_row_decode(x, 1, torch.full((4,), 16, dtype=I32), torch.zeros(4, 8, dtype=I32),
                                           3, 16, 1, 8)


# ---------------------------------------------------------------- GPU ----

def _check_rows(got, logits_cpu, k, rows, exp):
    """got: GPU indices [R, k]; exp: the oracle's sorted sets for `rows`."""
    g = got.cpu()[rows]
    short = (exp < 0).any(1)
    # rows of at most top_k values are positional (0..len-1 then -1); others are sets
    assert torch.equal(g[short], exp[short]), "short rows differ from 0..len-1, -1..."
    assert torch.equal(g[~short].sort(1).values, exp[~short]), "selected index sets differ from the oracle's"


def _decode_case(B, V, k, next_n=1, seq=None, seed=42, fill=None, stride0=None, stride1=1):
    g = torch.Generator().manual_seed(seed)
    rows = B * next_n
    s0 = stride0 or V
    buf = torch.randn((rows - 1) * s0 + (V - 1) * stride1 + 1, generator=g)
    if fill is not None:
        buf = fill(buf, g)
    logits = torch.as_strided(buf, (rows, V), (s0, stride1))
    seq_lens = torch.full((B,), V, dtype=I32) if seq is None else torch.as_tensor(seq, dtype=I32)
    return buf, logits, seq_lens


def _run_decode(buf, logits, seq_lens, k, next_n, rows_checked):
    import flaggems_vllm

    R = logits.shape[0]
    dbuf = buf.to(DEV)
    dl = torch.as_strided(dbuf, logits.shape, logits.stride())
    idx = torch.full((R, k), -7, dtype=I32, device=DEV)
    flaggems_vllm.top_k_per_row_decode(dl, next_n, seq_lens.to(DEV), idx, R, dl.stride(0), dl.stride(1), k)
    torch.cuda.synchronize()
    exp = oracle.top_k_per_row(logits, k, seq_lens=seq_lens, next_n=next_n, rows=rows_checked)
    _check_rows(idx, logits, k, rows_checked, exp)
    return idx


DECODE_SHAPES = [(1, 4096, 64), (1, 8192, 128), (1, 16384, 256), (1, 32768, 512), (1, 129280, 1024),
                 (1, 262144, 512), (496, 262144, 512), (56, 262144, 512)]


@pytest.mark.gpu
@pytest.mark.parametrize("B,V,k", DECODE_SHAPES)
def test_gpu_decode_reference_shapes(B, V, k):
    """The reference test's and benchmark's shapes (full rows); the oracle
    checks up to 64 rows of each, torch.topk's values every row."""
    print(f"\n[case] top-k decode B={B} V={V} k={k}", flush=True)
    buf, logits, seq = _decode_case(B, V, k)
    rows = list(range(min(B, 48))) + ([B - 1] if B > 48 else [])
    idx = _run_decode(buf, logits, seq, k, 1, rows)
    vals = torch.gather(logits.to(DEV), 1, idx.long()).sort(1).values
    assert torch.equal(vals, logits.to(DEV).topk(k, dim=1).values.sort(1).values)


@pytest.mark.gpu
@pytest.mark.parametrize("V,k,s", [(129280, 1024, 100000), (32768, 256, 16384), (8192, 64, 4096),
                                   (262144, 512, 496), (262144, 512, 512), (262144, 512, 513)])
def test_gpu_decode_partial_rows(V, k, s):
    """seq_len below the vocabulary (reference :144-170), and a row of at most
    top_k values (:174-194): 0..len-1 then -1."""
    print(f"\n[case] top-k decode partial V={V} k={k} seq={s}", flush=True)
    buf, logits, seq = _decode_case(1, V, k, seq=[s], seed=123)
    _run_decode(buf, logits, seq, k, 1, [0])


@pytest.mark.gpu
def test_gpu_decode_next_n_and_ragged():
    """next_n = 3: each batch's rows end one position apart; ragged seq_lens."""
    print("\n[case] top-k decode next_n=3 ragged", flush=True)
    seq = [50000, 700, 3, 262144, 1025, 999]
    buf, logits, seq_t = _decode_case(6, 262144, 512, next_n=3, seq=seq, seed=9)
    _run_decode(buf, logits, seq_t, 512, 3, list(range(18)))


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["lsb8", "few_values", "all_equal", "neg_inf_tail", "nan"])
def test_gpu_decode_ties_and_specials(kind):
    """Rows whose values share their upper bits (the reference's 8-LSB test,
    :198-222: every value in one first-level bin, more than LDS holds), few
    distinct values and all equal (ties at the k-th value, lowest index
    first), -inf tails, NaN."""
    print(f"\n[case] top-k decode {kind}", flush=True)

    def fill(buf, g):
        n = buf.numel()
        if kind == "lsb8":
            bits = 0x3F900000 | torch.randint(0, 256, (n,), generator=g, dtype=torch.int32)
            return bits.view(torch.float32)
        if kind == "few_values":
            return torch.randint(0, 5, (n,), generator=g).float()
        if kind == "all_equal":
            return torch.full((n,), 0.5)
        if kind == "neg_inf_tail":
            buf = buf.clone()
            buf.view(4, -1)[:, 3000:] = float("-inf")
            return buf
        buf = buf.clone()
        buf[torch.randperm(n, generator=g)[:300]] = float("nan")
        return buf

    buf, logits, seq = _decode_case(4, 65536, 512, seed=5, fill=fill)
    _run_decode(buf, logits, seq, 512, 1, [0, 1, 2, 3])
    buf, logits, seq = _decode_case(2, 5000, 256, seed=6, fill=fill)  # rows held in LDS
    _run_decode(buf, logits, seq, 256, 1, [0, 1])


@pytest.mark.gpu
@pytest.mark.parametrize("s1", [1, 3])
def test_gpu_decode_strided(s1):
    """stride0 above the row (the benchmark passes explicit strides) and a
    column stride."""
    print(f"\n[case] top-k decode strided s1={s1}", flush=True)
    buf, logits, seq = _decode_case(5, 20000, 512, stride0=20000 * s1 + 37, stride1=s1, seed=11)
    _run_decode(buf, logits, seq, 512, 1, list(range(5)))


def _run_prefill(logits, starts, ends, k, rows_checked):
    import flaggems_vllm

    R = logits.shape[0]
    dl = logits.to(DEV)
    idx = torch.full((R, k), -7, dtype=I32, device=DEV)
    flaggems_vllm.top_k_per_row_prefill(dl, starts.to(DEV), ends.to(DEV), idx, R, dl.stride(0), dl.stride(1), k)
    torch.cuda.synchronize()
    exp = oracle.top_k_per_row(logits, k, row_starts=starts, row_ends=ends, rows=rows_checked)
    _check_rows(idx, logits, k, rows_checked, exp)


PREFILL_SHAPES = [(64, 129280, 1024), (4, 8193, 512), (2000, 4095, 512), (4, 16385, 512), (1300, 4100, 512),
                  (1600, 5115, 512), (4100, 1025, 512)]


@pytest.mark.gpu
@pytest.mark.parametrize("R,V,k", PREFILL_SHAPES)
def test_gpu_prefill_reference_shapes(R, V, k):
    """The benchmark's shapes (full rows; its 16383- and 12961-row cases with
    fewer rows), oracle on up to 64 rows."""
    print(f"\n[case] top-k prefill R={R} V={V} k={k}", flush=True)
    g = torch.Generator().manual_seed(42)
    logits = torch.randn(R, V, generator=g)
    starts = torch.zeros(R, dtype=I32)
    ends = torch.full((R,), V, dtype=I32)
    _run_prefill(logits, starts, ends, k, list(range(min(R, 63))) + [R - 1])


@pytest.mark.gpu
def test_gpu_prefill_ragged_ranges():
    """Nonzero row starts (reference :210-240), ragged and empty rows, rows
    past the width, rows of at most top_k values."""
    print("\n[case] top-k prefill ragged", flush=True)
    g = torch.Generator().manual_seed(321)
    R, V, k = 40, 65536, 1024
    logits = torch.randn(R, V, generator=g)
    starts = torch.randint(0, 30000, (R,), generator=g, dtype=I32)
    ends = starts + torch.randint(0, 36000, (R,), generator=g, dtype=I32)
    starts[:2] = torch.tensor([128, 4096], dtype=I32)
    ends[:2] = torch.tensor([4096, 8192], dtype=I32)
    ends[5], ends[6], starts[7] = starts[5], starts[6] + 100, 70000
    _run_prefill(logits, starts, ends, k, list(range(R)))


def _sampled_positions(n):
    """Positions of the sample a workgroup takes from a row longer than its
    LDS cache before streaming it: chunks of 256 contiguous values, one every
    n // chunks values, chunks = max((n // 32) rounded down to 256, 2048) /
    256 (the cache's size caps it, 8192 or 12288 values: not reached below
    262144-value rows)."""
    ns = max((n // 32) & ~255, 2048)
    nch = ns // 256
    stride = n // nch
    return (torch.arange(nch)[:, None] * stride + torch.arange(256)[None, :]).reshape(-1)


@pytest.mark.gpu
@pytest.mark.parametrize("reps", [1, 50])
@pytest.mark.parametrize("kind", ["random", "lsb8", "few_values", "sample_high", "sample_low", "sorted"])
def test_gpu_long_rows_without_workspace(kind, reps):
    """Rows wider than 16384 values with no workspace: one workgroup per row
    streams it instead of the split into parts and merge (1024 threads for 6
    rows, 512 for 300); same index sets.  A sample of the row sets the
    threshold of a single read; rows whose sampled values lie above the rest
    (fewer than top_k values reach the threshold) or below it (more than LDS
    holds reach it) are read again, twice (or four times for a threshold bin
    larger than LDS)."""
    from flaggems_vllm import _native

    print(f"\n[case] top-k long rows without workspace {kind} x{reps}", flush=True)
    g = torch.Generator().manual_seed(17)
    R, V, k = 6, 200000, 512
    seq = torch.tensor([V, 190000, 40000, 513, V, 16385], dtype=I32)
    if kind == "lsb8":
        x = (0x3F900000 | torch.randint(0, 256, (R, V), generator=g, dtype=torch.int32)).view(torch.float32)
    elif kind == "few_values":
        x = torch.randint(0, 7, (R, V), generator=g).float()
    elif kind == "sorted":
        x = torch.arange(V, dtype=torch.float32).repeat(R, 1) * (1 - 2 * (torch.arange(R) % 2))[:, None]
    else:
        x = torch.randn(R, V, generator=g)
        if kind.startswith("sample"):
            for r in range(R):
                n = int(seq[r])
                if n > 16384:
                    pos = _sampled_positions(n)
                    x[r, pos] += 50.0 if kind == "sample_high" else -50.0
    assert _native.lib().fgv_top_k_per_row_workspace_bytes(R, V, k) > 0, "the split applies to these rows"
    x, seq = x.repeat(reps, 1), seq.repeat(reps)
    R *= reps
    d = x.to(DEV)
    idx = torch.full((R, k), -7, dtype=I32, device=DEV)
    rc = _native.lib().fgv_top_k_per_row_decode(d.data_ptr(), V, 1, R, V, 1, seq.to(DEV).data_ptr(),
                                                idx.data_ptr(), k, 1, k, None, 0,
                                                torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    rows = list(range(6)) + ([R - 6 + i for i in range(6)] if reps > 1 else [])
    _check_rows(idx, x, k, rows, oracle.top_k_per_row(x, k, seq_lens=seq, rows=rows))


@pytest.mark.gpu
@pytest.mark.parametrize("R", [32, 33])
def test_gpu_split_threshold(R):
    """Either side of the row count where the split stops (its parts over
    two per CU): the wrapper allocates the workspace only up to it; both
    give the oracle's sets."""
    from flaggems_vllm import _native

    print(f"\n[case] top-k split threshold R={R}", flush=True)
    V, k = 262144, 512
    split = _native.lib().fgv_top_k_per_row_workspace_bytes(R, V, k) > 0
    assert split == (16 * R <= 2 * torch.cuda.get_device_properties(0).multi_processor_count)
    buf, logits, seq = _decode_case(R, V, k, seed=77)
    _run_decode(buf, logits, seq, k, 1, list(range(0, R, 9)) + [R - 1])


@pytest.mark.gpu
@pytest.mark.parametrize("k", [1, 100, 512, 2048])
def test_gpu_many_short_rows(k):
    """Many short rows (1100 x 4096, the LDS-cached kernel): ragged ranges
    (empty rows, rows of at most k values, rows past the width), and rows of
    ties (8 distinct low bits, 5 distinct values, all equal), NaN, -inf;
    160 rows against the oracle's sets."""
    print(f"\n[case] top-k many short rows k={k}", flush=True)
    g = torch.Generator().manual_seed(900 + k)
    R, V = 1100, 4096
    logits = torch.randn(R, V, generator=g)
    logits[1::7] = (logits[1::7] * 256).round() / 256          # 8-bit ties
    logits[2::7] = torch.randint(0, 5, (len(range(2, R, 7)), V), generator=g).float()
    logits[3::7] = 1.5                                           # all equal
    logits[4::7, ::9] = float("nan")
    logits[5::7, V // 2:] = float("-inf")
    starts = torch.randint(0, 600, (R,), generator=g, dtype=I32)
    ends = starts + torch.randint(0, V - 400, (R,), generator=g, dtype=I32)
    ends[::11] = starts[::11] + torch.randint(0, k + 1, (len(range(0, R, 11)),), generator=g, dtype=I32)
    ends[6::50] = starts[6::50]                                  # empty
    ends[8::50] = V + 5                                          # past the width
    rows = sorted(set(range(0, R, 7)) | set(range(1, 80)) | {R - 1})
    _run_prefill(logits, starts, ends, k, rows)
