"""The index rows sparse attention reads: compute_global_topk_indices_and_lens
and combine_topk_swa_indices.

Reference: src/flaggems_vllm/ops/deepseek_v4_attention_compute_global_topk_indices_and_lens.py:46-160,
src/flaggems_vllm/ops/deepseek_v4_attention_combine_topk_swa_indices.py:30-150; tests
tests/test_deepseek_v4_attention_compute_global_topk_indices_and_lens.py:42-98 and
tests/test_deepseek_v4_attention_combine_topk_swa_indices.py:49-144 (their cases are the
golden vectors below, with the expected rows worked out by hand from the
definitions); benchmark shapes benchmark/test_deepseek_v4_attention_compute_global_topk_indices_and_lens.py:49-81
and benchmark/test_deepseek_v4_attention_combine_topk_swa_indices.py:108-140.
Integer work: the bar is bit-exact.
"""
import pytest
import torch

import oracle

DEV = torch.device("cuda:0")
I32 = torch.int32


def _t(x):
    return torch.tensor(x, dtype=I32)


# ------------------------------------------------------------- golden ----

# (topk_indices, token_to_req, block_table, is_valid, block_size) -> (indices, lens)
GLOBAL_CASES = [
    (([[0, 3, -1, 7], [2, -1, 4, 5], [1, 0, -1, -1]], [0, 1, 0], [[5, 6], [9, 10]], [1, 1, 0], 4),
     # token 0 (request 0): 0 -> 5*4+0, 3 -> 5*4+3, 7 -> block 1: 6*4+3; three valid
     # token 1 (request 1): 2 -> 9*4+2, 4 -> 10*4+0, 5 -> 10*4+1; three valid
     # token 2 (request 0, marked invalid): 1 -> 21, 0 -> 20; length 0
     ([[20, 23, -1, 27], [38, -1, 40, 41], [21, 20, -1, -1]], [3, 3, 0])),
    (([[0, 63, 64, 127], [128, -1, 191, 255], [7, 8, -1, -1]], [0, 1, 1], [[11, 12, 13, 14], [21, 22, 23, 24]],
      [1, 1, 0], 64),
     # token 0: 0 -> 11*64, 63 -> 11*64+63, 64 -> 12*64, 127 -> 12*64+63
     # token 1 (request 1): 128 -> block 2: 23*64, 191 -> 23*64+63, 255 -> block 3: 24*64+63
     # token 2 (request 1, invalid): 7 -> 21*64+7, 8 -> 21*64+8
     ([[704, 767, 768, 831], [1472, -1, 1535, 1599], [1351, 1352, -1, -1]], [4, 3, 0])),
]

# (topk_indices, query_start_loc, seq_lens, gather_lens, window, ratio, topk, M, N) -> (rows, lens)
COMBINE_CASES = [
    (([[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]], [0, 2, 3], [8, 10], [8, 10], 4, 2, 4, 64, 16),
     # request 0: tokens 0, 1 at positions 6, 7 (query length 2, gather start 0)
     #   pos 6: topk_len min(7/2, 4) = 3, swa_len 4: window rows 16 + 6 - 4 + 1 + j = 19..22
     #   pos 7: topk_len 4, swa 4: 20..23
     # request 1 (offset M = 64): token 2 at position 9: topk_len 4 -> 73..76; swa 64+16+9-4+1 = 86..89
     ([[1, 2, 3, 19, 20, 21, 22], [5, 6, 7, 8, 20, 21, 22, 23], [73, 74, 75, 76, 86, 87, 88, 89]], [7, 8, 8])),
    (([[100, 101, 102, 103], [110, 111, 112, 113], [120, 121, 122, 123], [130, 131, 132, 133],
       [140, 141, 142, 143]], [0, 3, 5], [6, 4], [4, 3], 3, 2, 4, 20, 8),
     # request 0: tokens 0..2 at positions 3..5, gather start 6 - 4 = 2, window 3
     #   pos 3: topk_len 2, swa rows 8 + 3 - 3 + 1 - 2 + j = 7..9
     #   pos 4: topk_len 2, 8..10;  pos 5: topk_len 3, 9..11
     # request 1 (offset 20): tokens 3, 4 at positions 2, 3, gather start 4 - 3 = 1
     #   pos 2: topk_len 1 -> 150; swa 20 + 8 + 2 - 3 + 1 - 1 = 27..29
     #   pos 3: topk_len 2 -> 160, 161; swa 28..30
     ([[100, 101, 7, 8, 9], [110, 111, 8, 9, 10], [120, 121, 122, 9, 10, 11], [150, 27, 28, 29],
       [160, 161, 28, 29, 30]], [5, 5, 6, 4, 5])),
]


def _pad_rows(rows, width):
    out = torch.full((len(rows), width), -1, dtype=I32)
    for i, r in enumerate(rows):
        out[i, :len(r)] = _t(r)
    return out


@pytest.mark.parametrize("case", range(len(GLOBAL_CASES)))
def test_global_oracle_golden(case):
    (topk, req, bt, valid, bs), (exp, exp_lens) = GLOBAL_CASES[case]
    idx, lens = oracle.compute_global_topk_indices_and_lens(_t(topk), _t(req), _t(bt), bs, _t(valid))
    assert torch.equal(idx, _t(exp)) and torch.equal(lens, _t(exp_lens))
    # without is_valid_token every token counts
    _, lens_all = oracle.compute_global_topk_indices_and_lens(_t(topk), _t(req), _t(bt), bs)
    assert torch.equal(lens_all, (_t(topk) >= 0).sum(1).to(I32))


@pytest.mark.parametrize("case", range(len(COMBINE_CASES)))
def test_combine_oracle_golden(case):
    args, (rows, exp_lens) = COMBINE_CASES[case]
    topk, qsl, seq, gat, window, ratio, k, M, N = args
    out, lens = oracle.combine_topk_swa_indices(_t(topk), _t(qsl), _t(seq), _t(gat), window, ratio, k, M, N)
    width = (k + window + 127) // 128 * 128
    assert out.shape == (len(topk), width) == (len(topk), 128)
    assert torch.equal(out, _pad_rows(rows, width)) and torch.equal(lens, _t(exp_lens))


def _vectorised_global(local, req, bt, bs, valid):
    """The same map in vectorised torch form (int64, then wrapped to int32)."""
    local = local.long()
    ok = local >= 0
    blk = torch.where(ok, local // bs, 0)
    f = req.long()[:, None] * bt.stride(0) + blk
    span = (bt.shape[0] - 1) * bt.stride(0) + bt.shape[1]
    inb = ok & (f >= 0) & (f < span)
    flat = bt.as_strided((span,), (1,)).long()  # the table's storage, row stride included
    slot = flat[torch.where(inb, f, 0)] * bs + local % bs
    slot = ((slot + 2 ** 31) % 2 ** 32 - 2 ** 31)
    out = torch.where(inb, slot, -1).to(I32)
    lens = torch.where(valid != 0, ok.sum(1), 0).to(I32)
    return out, lens


def _vectorised_combine(topk_idx, qsl, seq, gat, window, ratio, k, M, N):
    """Row-parallel form (the reference benchmark's torch baseline,
    benchmark/test_deepseek_v4_attention_combine_topk_swa_indices.py:49-99, written again)."""
    T = topk_idx.shape[0]
    width = (k + window + 127) // 128 * 128
    starts, ends = (qsl[:-1] - qsl[0]).long(), (qsl[1:] - qsl[0]).long()
    b = torch.repeat_interleave(torch.arange(len(seq)), ends - starts)
    tok = torch.arange(int(ends[-1]))
    pos = (seq.long()[b] - (ends - starts)[b]) + (tok - starts[b])
    tl = torch.clamp(torch.div(pos + 1, ratio, rounding_mode="trunc"), max=k)
    sl = torch.clamp(pos + 1, max=window)
    col = torch.arange(width)[None, :]
    off = col - tl[:, None]
    base = M * b + N + pos - sl + 1 - (seq.long()[b] - gat.long()[b])
    vals = torch.full((len(tok), width), -1, dtype=torch.long)
    src = torch.zeros((len(tok), width), dtype=torch.long)
    src[:, :topk_idx.shape[1]] = topk_idx[:len(tok)].long()
    vals = torch.where(col < tl[:, None], src + (M * b)[:, None], vals)
    vals = torch.where((off >= 0) & (off < sl[:, None]), base[:, None] + off, vals)
    return vals.to(I32), (tl + sl).to(I32)


def test_global_oracle_against_vectorised():
    g = torch.Generator().manual_seed(5)
    T, K, R, bpr, bs = 300, 96, 5, 12, 16
    local = torch.randint(-3, bpr * bs + 20, (T, K), generator=g, dtype=I32)  # some past the table
    req = torch.randint(0, R, (T,), generator=g, dtype=I32)
    bt = torch.randint(0, 1 << 20, (R, bpr + 3), generator=g, dtype=I32)[:, :bpr]  # row stride > row
    valid = torch.randint(0, 2, (T,), generator=g, dtype=I32)
    got = oracle.compute_global_topk_indices_and_lens(local, req, bt, bs, valid)
    exp = _vectorised_global(local, req, bt, bs, valid)
    assert torch.equal(got[0], exp[0]) and torch.equal(got[1], exp[1])


def test_combine_oracle_against_vectorised():
    g = torch.Generator().manual_seed(6)
    qlens = [5, 1, 17, 3]
    qsl = torch.tensor([7] + [7 + sum(qlens[:i + 1]) for i in range(len(qlens))], dtype=I32)
    seq = torch.tensor([40, 9, 17, 300], dtype=I32)
    gat = torch.tensor([20, 9, 10, 100], dtype=I32)
    T = sum(qlens)
    topk_idx = torch.randint(0, 1000, (T, 48), generator=g, dtype=I32)
    for window, ratio, k in ((8, 4, 32), (3, 1, 48), (16, 3, 5)):
        got = oracle.combine_topk_swa_indices(topk_idx, qsl, seq, gat, window, ratio, k, 333, 77)
        exp = _vectorised_combine(topk_idx, qsl, seq, gat, window, ratio, k, 333, 77)
        assert torch.equal(got[0], exp[0]) and torch.equal(got[1], exp[1])
        # the window rows end on the token's own row of the gathered buffer
        for t in range(T):
            n = int(got[1][t])
            b = int(torch.searchsorted(qsl[1:] - qsl[0], torch.tensor(t), right=True))
            pos = int(seq[b]) - qlens[b] + (t - int(qsl[b] - qsl[0]))
            assert int(got[0][t, n - 1]) == 333 * b + 77 + pos - (int(seq[b]) - int(gat[b]))


# ------------------------------------------------------------ boundary ----

def test_wrappers_reject_like_the_reference():
    import flaggems_vllm

    with pytest.raises(AssertionError):
        flaggems_vllm.compute_global_topk_indices_and_lens(torch.zeros(4, dtype=I32), _t([0]), _t([[0]]), 4)
    with pytest.raises(AssertionError):
        flaggems_vllm.combine_topk_swa_indices(torch.zeros(4, dtype=I32), _t([0, 1]), _t([1]), _t([1]),
                                               4, 2, 4, 64, 16)


def test_c_abi_rejects_bad_arguments():
    from flaggems_vllm import _native

    L = _native.lib()
    assert L.fgv_combine_topk_swa_width(4, 4) == 128 and L.fgv_combine_topk_swa_width(128, 256) == 384
    assert L.fgv_combine_topk_swa_width(-1, 4) == -1
    p = 1 << 12  # never dereferenced: each call fails its checks before launching
    g = L.fgv_compute_global_topk_indices_and_lens
    assert g(p, 4, 1, 1, 4, p, p, 2, 1, 2, 0, None, p, 4, 1, p, None) == -2   # block_size 0
    assert g(p, 4, 1, -1, 4, p, p, 2, 1, 2, 4, None, p, 4, 1, p, None) == -2  # negative tokens
    assert g(None, 4, 1, 1, 4, p, p, 2, 1, 2, 4, None, p, 4, 1, p, None) == -1
    assert g(p + 2, 4, 1, 1, 4, p, p, 2, 1, 2, 4, None, p, 4, 1, p, None) == -3
    assert g(p, 4, 1, 0, 4, p, p, 2, 1, 2, 4, None, p, 4, 1, p, None) == 0    # nothing to do
    c = L.fgv_combine_topk_swa_indices
    assert c(p, 4, 1, 3, 4, p, p, p, 2, 4, 2, 5, 64, 16, p, 128, 1, p, None) == -2  # topk > columns
    assert c(p, 4, 1, 3, 4, p, p, p, 2, 4, 0, 4, 64, 16, p, 128, 1, p, None) == -2  # ratio 0
    assert c(p, 4, 1, 3, 4, None, p, p, 2, 4, 2, 4, 64, 16, p, 128, 1, p, None) == -1
    assert c(p, 4, 1, 3, 4, p, p, p, 0, 4, 2, 4, 64, 16, p, 128, 1, p, None) == 0   # no requests


# ----------------------------------------------------------------- GPU ----

@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(GLOBAL_CASES)))
def test_gpu_global_golden(case):
    import flaggems_vllm

    print(f"\n[case] global top-k indices golden {case}", flush=True)
    (topk, req, bt, valid, bs), (exp, exp_lens) = GLOBAL_CASES[case]
    idx, lens = flaggems_vllm.compute_global_topk_indices_and_lens(
        _t(topk).to(DEV), _t(req).to(DEV), _t(bt).to(DEV), bs, _t(valid).to(DEV))
    assert torch.equal(idx.cpu(), _t(exp)) and torch.equal(lens.cpu(), _t(exp_lens))


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(len(COMBINE_CASES)))
def test_gpu_combine_golden(case):
    import flaggems_vllm

    print(f"\n[case] combine top-k + window golden {case}", flush=True)
    args, (rows, exp_lens) = COMBINE_CASES[case]
    topk, qsl, seq, gat, window, ratio, k, M, N = args
    out, lens = flaggems_vllm.combine_topk_swa_indices(_t(topk).to(DEV), _t(qsl).to(DEV), _t(seq).to(DEV),
                                                       _t(gat).to(DEV), window, ratio, k, M, N)
    assert torch.equal(out.cpu(), _pad_rows(rows, 128)) and torch.equal(lens.cpu(), _t(exp_lens))


# the reference benchmark's shapes (num_tokens, topk, num_reqs, blocks_per_req, block_size), plus ragged ones
GLOBAL_SHAPES = [(5, 4, 2, 4, 64), (512, 64, 2, 128, 64), (4096, 128, 4, 640, 64), (8192, 128, 8, 1280, 64),
                 (8192, 2048, 3, 300, 64), (777, 100, 5, 17, 16)]


@pytest.mark.gpu
@pytest.mark.parametrize("shape", GLOBAL_SHAPES)
def test_gpu_global_against_oracle(shape):
    import flaggems_vllm

    print(f"\n[case] global top-k indices {shape}", flush=True)
    T, K, R, bpr, bs = shape
    g = torch.Generator().manual_seed(T + K)
    local = torch.randint(-1, bpr * bs, (T, K), generator=g, dtype=I32)
    local.view(-1)[torch.randperm(T * K, generator=g)[:max(1, T * K // 50)]] = bpr * bs + 5  # past the table
    req = torch.randint(0, R, (T,), generator=g, dtype=I32)
    # a block table with row stride bpr + 8, the same layout on both sides: a
    # block past a row reads the padding after it (the reference's flat read)
    bt_full = torch.randint(0, 1 << 16, (R, bpr + 8), generator=g, dtype=I32)
    bt, bt_d = bt_full[:, :bpr], bt_full.to(DEV)[:, :bpr]
    valid = torch.randint(0, 2, (T,), generator=g, dtype=I32)
    for v in (valid, None):
        exp = oracle.compute_global_topk_indices_and_lens(local, req, bt, bs, v)
        got = flaggems_vllm.compute_global_topk_indices_and_lens(
            local.to(DEV), req.to(DEV), bt_d, bs, v.to(DEV) if v is not None else None)
        assert torch.equal(got[0].cpu(), exp[0]) and torch.equal(got[1].cpu(), exp[1])
    # a column slice (row stride above the row): empty_like gives a dense output
    big = torch.randint(-1, bpr * bs, (T, K + 7), generator=g, dtype=I32)
    view = big.to(DEV)[:, 3:3 + K]
    exp = oracle.compute_global_topk_indices_and_lens(big[:, 3:3 + K], req, bt, bs, valid)
    got = flaggems_vllm.compute_global_topk_indices_and_lens(view, req.to(DEV), bt_d, bs, valid.to(DEV))
    assert torch.equal(got[0].cpu(), exp[0]) and torch.equal(got[1].cpu(), exp[1])


# (query lengths, seq_lens, gather_lens, topk, window, ratio, M, N): the reference benchmark's shapes
COMBINE_SHAPES = [([3, 2], [6, 4], [4, 3], 4, 4, 2, 20, 8),
                  ([128], [512], [256], 32, 128, 4, 42240, 40960),
                  ([512, 256], [2048, 1024], [1024, 512], 64, 256, 4, 45056, 40960),
                  ([4096], [4096], [4096], 128, 256, 4, 45056, 40960),
                  ([1024, 1024], [8192, 4096], [2048, 1024], 128, 256, 4, 45056, 40960),
                  ([1] * 300 + [70], [5000] * 300 + [600], [300] * 300 + [200], 512, 128, 4, 800, 700)]


@pytest.mark.gpu
@pytest.mark.parametrize("shape", range(len(COMBINE_SHAPES)))
def test_gpu_combine_against_oracle(shape):
    import flaggems_vllm

    qlens, seq, gat, k, window, ratio, M, N = COMBINE_SHAPES[shape]
    print(f"\n[case] combine top-k + window shape {shape}", flush=True)
    g = torch.Generator().manual_seed(shape)
    T = sum(qlens) + 3  # three padding tokens outside every request
    topk_idx = torch.randint(0, 40000, (T, k + 5), generator=g, dtype=I32)
    qsl = torch.tensor([11] + [11 + sum(qlens[:i + 1]) for i in range(len(qlens))], dtype=I32)
    args = (_t(seq), _t(gat), window, ratio, k, M, N)
    exp, exp_lens = oracle.combine_topk_swa_indices(topk_idx, qsl, *args)
    out, lens = flaggems_vllm.combine_topk_swa_indices(topk_idx.to(DEV), qsl.to(DEV), _t(seq).to(DEV),
                                                       _t(gat).to(DEV), window, ratio, k, M, N)
    n = sum(qlens)
    assert out.shape == exp.shape
    assert torch.equal(out.cpu()[:n], exp[:n]) and torch.equal(lens.cpu()[:n], exp_lens[:n])


def test_combine_oracle_skips_rows_past_the_tensor():
    """query_start_loc running past topk_indices' rows: the rows inside are the
    in-bounds result, nothing past them is read or written."""
    g = torch.Generator().manual_seed(5)
    T = 20
    topk_idx = torch.randint(0, 1000, (T, 8), generator=g, dtype=I32)
    qsl, seq, gat = _t([0, 12, 31]), _t([40, 50]), _t([30, 25])
    out, lens = oracle.combine_topk_swa_indices(topk_idx, qsl, seq, gat, 16, 4, 8, 64, 32)
    # the first request lies inside; rows 12..19 of the second are the same
    # rows as a call whose tensors hold all 31 tokens
    big = torch.cat([topk_idx, torch.zeros(11, 8, dtype=I32)])
    eo, el = oracle.combine_topk_swa_indices(big, qsl, seq, gat, 16, 4, 8, 64, 32)
    assert torch.equal(out, eo[:T]) and torch.equal(lens, el[:T])


@pytest.mark.gpu
def test_gpu_combine_rows_past_the_tensor_untouched():
    """query_start_loc whose last request runs 11 tokens past topk_indices'
    rows (and a first entry of 0): the kernel writes the rows inside, as the
    oracle does, and leaves guard rows after combined and lens untouched."""
    from flaggems_vllm import _native

    print("\n[case] combine top-k + window, query_start_loc past the rows", flush=True)
    g = torch.Generator().manual_seed(5)
    T, guard = 20, 16
    topk_idx = torch.randint(0, 1000, (T, 8), generator=g, dtype=I32)
    qsl, seq, gat = _t([0, 12, 31]), _t([40, 50]), _t([30, 25])
    k, window, ratio, M, N = 8, 16, 4, 64, 32
    width = _native.lib().fgv_combine_topk_swa_width(k, window)
    exp, exp_lens = oracle.combine_topk_swa_indices(topk_idx, qsl, seq, gat, window, ratio, k, M, N)
    comb = torch.full((T + guard, width), -7, dtype=I32, device=DEV)
    lens = torch.full((T + guard,), -7, dtype=I32, device=DEV)
    # topk_indices also sits in front of guard rows, so every access the
    # kernel could make stays inside allocated memory
    d = torch.cat([topk_idx, torch.zeros(guard, 8, dtype=I32)]).to(DEV)[:T]
    q, s, ga = qsl.to(DEV), seq.to(DEV), gat.to(DEV)
    rc = _native.lib().fgv_combine_topk_swa_indices(
        d.data_ptr(), d.stride(0), d.stride(1), T, k, q.data_ptr(), s.data_ptr(), ga.data_ptr(), 2,
        window, ratio, k, M, N, comb.data_ptr(), comb.stride(0), comb.stride(1), lens.data_ptr(),
        torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(comb.cpu()[:T], exp) and torch.equal(lens.cpu()[:T], exp_lens)
    assert bool((comb.cpu()[T:] == -7).all()) and bool((lens.cpu()[T:] == -7).all())
