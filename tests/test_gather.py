"""dequantize_and_gather_k_cache: CPU pins of its oracle and GPU parity.

Reference: src/flaggems_vllm/ops/deepseek_v4_attention_dequantize_and_gather_k_cache.py:38-172,
tests/test_deepseek_v4_attention_dequantize_and_gather_k_cache.py:42-119 (the
fill pattern with scale byte 127 and the two shapes below are that test's).
"""
import pytest
import torch

import oracle
from flaggems_vllm import testing as W
from oracle import torch_ref

DEV = torch.device("cuda:0")


def _ref_fixture(batch, seq_len, gather_len, block_size, nope_dim, rope_dim):
    """The reference test's cache fill and expected rows (scale byte 127 = 1.0)."""
    scale_slots = (nope_dim + 63) // 64 + (1 if nope_dim % 64 == 0 else 0)
    tb = nope_dim + rope_dim * 2
    stride = block_size * tb + block_size * scale_slots
    bps = (seq_len + block_size - 1) // block_size
    cache = torch.zeros(batch * bps, stride, dtype=torch.uint8)
    expected = torch.zeros(batch, gather_len, nope_dim + rope_dim, dtype=torch.bfloat16)
    for req in range(batch):
        for i in range(gather_len):
            pos = seq_len - gather_len + i
            blk = req * bps + pos // block_size
            slot = blk * block_size + pos % block_size
            p = slot % block_size
            x = (torch.arange(nope_dim, dtype=torch.float32) / 32.0 + slot / 8.0).to(torch.float8_e4m3fn)
            rope = (torch.arange(rope_dim, dtype=torch.float32) / 16.0 + slot).to(torch.bfloat16)
            cache[blk, p * tb:p * tb + nope_dim] = x.view(torch.uint8)
            cache[blk, p * tb + nope_dim:p * tb + tb] = rope.view(torch.uint8)
            sb = block_size * tb + p * scale_slots
            cache[blk, sb:sb + scale_slots] = 127
            expected[req, i, :nope_dim] = x.float().to(torch.bfloat16)
            expected[req, i, nope_dim:] = rope
    seq_lens = torch.full((batch,), seq_len, dtype=torch.int32)
    gather_lens = torch.full((batch,), gather_len, dtype=torch.int32)
    bt = torch.arange(batch * bps, dtype=torch.int32).view(batch, bps)
    return cache, expected, seq_lens, gather_lens, bt, scale_slots


REF_SHAPES = [(1, 6, 3, 4, 64, 16), (2, 12, 5, 64, 448, 64)]


def test_e4m3_decode_exhaustive():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = oracle.e4m3fn_decode(codes)
    want = codes.view(torch.float8_e4m3fn).float()
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    m = ~torch.isnan(want)
    assert torch.equal(got[m].view(torch.int32), want[m].view(torch.int32))  # signed zeros too


@pytest.mark.parametrize("shape", REF_SHAPES)
def test_oracle_matches_reference_fixture(shape):
    batch, seq_len, gl, bs, nope, rope = shape
    cache, expected, seq_lens, gather_lens, bt, slots = _ref_fixture(*shape)
    for impl in (oracle.dequantize_and_gather_k_cache, torch_ref.dequantize_and_gather_k_cache):
        out = torch.zeros_like(expected)
        impl(out, cache, seq_lens, gather_lens, bt, bs, rope_dim=rope, nope_dim=nope,
             scale_slots=slots)
        assert torch.equal(out, expected)


def _inserted(config=0):
    w = W.make_workload(config)
    r = w.clone()
    oracle.qnorm_rope_kv_insert(*r.args())
    return w, r


def test_oracle_round_trip_and_torch_ref():
    """insert -> gather returns kv's nope within e4m3 error, the rope bytes
    exactly, and the C oracle agrees with the torch restatement bit for bit."""
    w, r = _inserted(0)
    slots = w.slot_mapping
    keep = torch.nonzero(slots >= 0).flatten()
    # one "request" per inserted token: seq_len = slot + 1 over an identity block table
    nblk = w.k_cache.shape[0]
    bt = torch.arange(nblk, dtype=torch.int32).repeat(keep.numel(), 1)
    seq_lens = (slots[keep] + 1).to(torch.int32)
    gl = torch.ones_like(seq_lens)
    out = torch.zeros(keep.numel(), 1, 512, dtype=torch.bfloat16)
    oracle.dequantize_and_gather_k_cache(out, r.k_cache, seq_lens, gl, bt, 64)
    out2 = torch.zeros_like(out)
    torch_ref.dequantize_and_gather_k_cache(out2, r.k_cache, seq_lens, gl, bt, 64)
    assert torch.equal(out, out2)
    x = w.kv[keep, :448].float()
    got = out[:, 0, :448].float()
    amax = x.view(-1, 7, 64).abs().amax(-1, keepdim=True).clamp(min=1e-4)
    tol = torch.maximum(x.view(-1, 7, 64).abs() * 2.0 ** -4, amax * 2.0 ** -18).view(-1, 448)
    assert bool(((got - x).abs() <= tol).all())
    rope_cache = r.k_cache.view(nblk, -1)[:, :64 * 576].reshape(-1, 576)[slots[keep], 448:]
    assert torch.equal(out[:, 0, 448:].contiguous().view(torch.uint8), rope_cache.contiguous())


def test_oracle_skips_out_of_range_blocks():
    cache, expected, seq_lens, gather_lens, bt, slots = _ref_fixture(2, 12, 5, 64, 448, 64)
    bt[1, 0] = 99  # no such block
    out = torch.full_like(expected, 7.0)
    oracle.dequantize_and_gather_k_cache(out, cache, seq_lens, gather_lens, bt, 64)
    assert torch.equal(out[0], expected[0])
    assert bool((out[1] == 7.0).all())


# ------------------------------------------------------------------- GPU ----

def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def _gpu_gather(out_like, cache, seq_lens, gather_lens, bt, bs, **kw):
    import flaggems_vllm

    out = out_like.clone().to(DEV)
    flaggems_vllm.dequantize_and_gather_k_cache(
        out, cache.to(DEV), seq_lens.to(DEV), None if gather_lens is None else gather_lens.to(DEV),
        bt.to(DEV), bs, **kw)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.gpu
@pytest.mark.parametrize("shape", REF_SHAPES)
def test_gpu_reference_fixture(shape):
    _say(f"gather reference fixture {shape}")
    batch, seq_len, gl, bs, nope, rope = shape
    cache, expected, seq_lens, gather_lens, bt, slots = _ref_fixture(*shape)
    out = _gpu_gather(torch.zeros_like(expected), cache, seq_lens, gather_lens, bt, bs,
                      rope_dim=rope, nope_dim=nope, scale_slots=slots)
    assert torch.equal(out, expected)


@pytest.mark.gpu
@pytest.mark.parametrize("config", [2, 4])
def test_gpu_insert_then_gather_round_trip(config):
    """GPU insert of a whole workload, then GPU gather of every sequence's new
    tokens: bit-exact vs the oracle's insert + gather."""
    import flaggems_vllm

    _say(f"insert -> gather round trip c{config}")
    w = W.make_workload(config)
    g = w.to(DEV)
    flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(*g.args())
    m = w.meta
    bt, seq_lens, new_lens = m["block_table"], m["seq_lens"], m["new_lens"]
    rows = int(new_lens.max())
    out = torch.zeros(bt.shape[0], rows, 512, dtype=torch.bfloat16, device=DEV)
    flaggems_vllm.dequantize_and_gather_k_cache(out, g.k_cache, seq_lens.to(DEV), new_lens.to(DEV),
                                                bt.to(DEV), w.block_size)
    torch.cuda.synchronize()
    # oracle insert restricted to the kv path (q plays no part in the cache)
    r = W.Workload(w.name, torch.zeros(w.num_tokens, 0, 512, dtype=torch.bfloat16), w.kv,
                   torch.zeros_like(w.k_cache), w.slot_mapping, w.position_ids,
                   w.cos_sin_cache, w.eps, w.block_size)
    oracle.qnorm_rope_kv_insert(*r.args())
    ref = torch.zeros(bt.shape[0], rows, 512, dtype=torch.bfloat16)
    oracle.dequantize_and_gather_k_cache(ref, r.k_cache, seq_lens, new_lens, bt, w.block_size)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.gpu
def test_gpu_whole_sequences_offset_and_bounds():
    """gather_lens=None (whole sequences), a non-zero offset, out rows that cut
    the gather short, and an out-of-range block-table entry."""
    _say("gather whole sequences with offset")
    w, r = _inserted(0)
    nblk = w.k_cache.shape[0]
    bt = torch.tensor([[0, 1, 2, 3], [3, 2, 1, 0], [1, 0, 99, 2]], dtype=torch.int32)
    seq_lens = torch.tensor([200, 256, 150], dtype=torch.int32)
    for gl, offset, rows in ((None, 0, 256), (torch.tensor([50, 256, 70], dtype=torch.int32), 3, 100)):
        ref = torch.full((3, rows, 520), 3.0, dtype=torch.bfloat16)
        oracle.dequantize_and_gather_k_cache(ref, r.k_cache, seq_lens, gl, bt, 64, offset=offset,
                                             nope_dim=448)
        got = _gpu_gather(torch.full((3, rows, 520), 3.0, dtype=torch.bfloat16), r.k_cache, seq_lens,
                          gl, bt, 64, offset=offset, nope_dim=448)
        assert torch.equal(got, ref)
    assert nblk == 4
