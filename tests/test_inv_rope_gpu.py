"""GPU parity of fused_inv_rope_fp8_quant against the CPU oracle (codes and
scales bit for bit) plus the reference's own invariants.

Reference tests mirrored: tests/test_fused_inv_rope_fp8_quant.py
  test_fused_inv_rope_fp8_quant :324-361, test_output_layout :364-391,
  test_per_group_contiguity :394-408, test_scales_are_power_of_two :411-430,
  test_large_values :433-448, test_nope_dims_unchanged :451-496,
  test_zero_positions :499-515, test_dequant_numerical_accuracy :518-545,
  test_with_real_deepseek_v4_rope :586-620;
  shapes from tests/accuracy_utils.py:104-115.
"""
import pytest
import torch

import flaggems_vllm
import oracle
from flaggems_vllm import testing as W

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _say(msg):
    print(f"\n[case] {msg}", flush=True)


def run_case(w: W.InvRopeWorkload, tma):
    d = w.to(DEV)
    out, scale = flaggems_vllm.fused_inv_rope_fp8_quant(
        d.o, d.positions, d.cos_sin_cache, d.n_groups, d.heads_per_group,
        tma_aligned_scales=tma)
    torch.cuda.synchronize()
    r8, rs = oracle.inv_rope_fp8_quant(w.o, w.positions, w.cos_sin_cache, w.n_groups,
                                       w.heads_per_group, tma_aligned_scales=tma)
    return out, scale, r8, rs


def unpack_ue8m0(packed):
    shifts = torch.arange(4, device=packed.device, dtype=torch.int32) * 8
    b = (packed.unsqueeze(-1) >> shifts) & 0xFF
    return (b << 23).view(torch.float32).flatten(-2)


def dequant(out, scale, hpg):
    if scale.dtype == torch.int32:
        scale = unpack_ue8m0(scale)
    return out.float() * scale.repeat_interleave(128, dim=-1)


@pytest.mark.parametrize("seed", [0, 42])
@pytest.mark.parametrize("tma", [False, True])
@pytest.mark.parametrize("H,G", [(32, 4), (64, 8), (128, 8)])
@pytest.mark.parametrize("T", [1, 7, 32, 128])
def test_matches_oracle(T, H, G, tma, seed):
    _say(f"inv rope T={T} H={H} G={G} tma={tma} seed={seed}")
    w = W.make_inv_rope_workload(T, H, G, seed=seed, max_pos=max(4096, 2 * T))
    out, scale, r8, rs = run_case(w, tma)
    assert out.dtype == torch.float8_e4m3fn
    assert torch.equal(out.cpu().view(torch.uint8), r8)
    assert torch.equal(scale.cpu(), rs)
    # the padded scale storage beyond T is zero (ops/fused_inv_rope_fp8_quant.py:69-88)
    tpad = (T + 3) // 4 * 4
    store = scale.transpose(0, 1)
    full = torch.as_strided(store, (G, store.shape[2], tpad), (store.stride(0), store.stride(2), 1))
    assert int(torch.count_nonzero(full[..., T:])) == 0


@pytest.mark.parametrize("tma", [False, True])
def test_prefill_size(tma):
    """T=8192, H=64, G=8 (the sibling's bench point), bit-exact."""
    _say(f"inv rope T=8192 H=64 G=8 tma={tma}")
    w = W.make_inv_rope_workload(8192, 64, 8, seed=7)
    out, scale, r8, rs = run_case(w, tma)
    assert torch.equal(out.cpu().view(torch.uint8), r8)
    assert torch.equal(scale.cpu(), rs)


@pytest.mark.parametrize("T,H,G", [(1, 64, 8), (7, 64, 8), (32, 128, 8), (128, 64, 8)])
def test_output_layout(T, H, G):
    _say(f"layout T={T} H={H} G={G}")
    d = (H // G) * 512
    w = W.make_inv_rope_workload(T, H, G, seed=0, max_pos=4096).to(DEV)
    out, scale = flaggems_vllm.fused_inv_rope_fp8_quant(w.o, w.positions, w.cos_sin_cache, G, H // G)
    assert out.shape == (T, G, d) and out.stride() == (d, T * d, 1)
    assert scale.shape == (T, G, d // 128) and (scale.permute(1, 0, 2).stride(1) == 1 or T == 1)
    for g in range(G):
        assert out[:, g, :].is_contiguous()
    out, scale = flaggems_vllm.fused_inv_rope_fp8_quant(w.o, w.positions, w.cos_sin_cache, G, H // G,
                                                        tma_aligned_scales=True)
    assert scale.dtype == torch.int32 and scale.shape[-1] == (d // 128 + 3) // 4
    assert scale.permute(1, 0, 2).stride(1) == 1 or T == 1


@pytest.mark.parametrize("tma", [False, True])
def test_scales_power_of_two(tma):
    _say(f"pow2 tma={tma}")
    w = W.make_inv_rope_workload(32, 64, 8, seed=0, max_pos=4096)
    _, scale, _, _ = run_case(w, tma)
    s = unpack_ue8m0(scale) if tma else scale
    res = (torch.log2(s) - torch.log2(s).round()).abs()
    if tma:
        assert float(res.max()) < 1e-5
    else:
        assert float(res.max()) > 1e-5


@pytest.mark.parametrize("tma", [False, True])
@pytest.mark.parametrize("mag", [1000.0, 1e-12])
def test_extreme_magnitudes(tma, mag):
    """x1000 (reference saturation case) and 1e-12 (amax below eps)."""
    _say(f"magnitude {mag} tma={tma}")
    w = W.make_inv_rope_workload(8, 64, 8, seed=0, scale=mag, max_pos=4096)
    out, scale, r8, rs = run_case(w, tma)
    assert torch.equal(out.cpu().view(torch.uint8), r8)
    assert torch.equal(scale.cpu(), rs)


@pytest.mark.parametrize("tma", [False, True])
def test_nope_unchanged_by_identity_rope(tma):
    """With cos=1, sin=0 the rotation is the identity, so every chunk equals the
    one produced with the real cache except the rope chunk."""
    _say(f"identity rope tma={tma}")
    w = W.make_inv_rope_workload(16, 64, 8, seed=0, max_pos=4096)
    ident = torch.zeros_like(w.cos_sin_cache)
    ident[:, :32] = 1.0
    w2 = W.InvRopeWorkload(w.o, w.positions, ident, w.n_groups, w.heads_per_group)
    o1, s1, _, _ = run_case(w, tma)
    o2, s2, r8, rs = run_case(w2, tma)
    assert torch.equal(o2.cpu().view(torch.uint8), r8) and torch.equal(s2.cpu(), rs)
    # identity rope: codes are the plain quantisation of o itself
    s1u = unpack_ue8m0(s1) if tma else s1
    s2u = unpack_ue8m0(s2) if tma else s2
    for h in range(8):
        for c in range(3):
            qb = h * 4 + c
            sl = slice(qb * 128, qb * 128 + 128)
            assert torch.equal(o1[:, :, sl].view(torch.uint8), o2[:, :, sl].view(torch.uint8))
            assert torch.equal(s1u[:, :, qb], s2u[:, :, qb])


@pytest.mark.parametrize("tma", [False, True])
def test_zero_positions_and_accuracy(tma):
    _say(f"zero positions tma={tma}")
    w = W.make_inv_rope_workload(32, 64, 8, seed=0, max_pos=4096)
    w = W.InvRopeWorkload(w.o, torch.zeros_like(w.positions), w.cos_sin_cache, 8, 8)
    out, scale, r8, rs = run_case(w, tma)
    assert torch.equal(out.cpu().view(torch.uint8), r8) and torch.equal(scale.cpu(), rs)
    # position 0: cos=1, sin=0, so dequantised output approximates o itself
    deq = dequant(out, scale, 8).cpu()
    x = w.o.float().view(32, 8, 4096)
    rel = (deq - x).abs() / x.abs().clamp(min=1e-6)
    assert float(rel.mean()) < 0.15


@pytest.mark.parametrize("tma", [False, True])
@pytest.mark.parametrize("T", [1, 32, 256])
def test_real_deepseek_v4_rope(T, tma):
    """DeepSeek-V4's YaRN-scaled cos/sin table (scaling 16, 65536 original
    positions; the first 65536 of its rows) at positions in [0, 4096), H=64,
    G=8: codes and scales bit for bit, and the reference's dequantised check."""
    _say(f"real DeepSeek-V4 rope T={T} tma={tma}")
    w = W.make_inv_rope_workload(T, 64, 8, seed=0, max_pos=4096)
    w = W.InvRopeWorkload(w.o, w.positions, W.make_yarn_cos_sin_cache(65536, rows=65536), 8, 8)
    out, scale, r8, rs = run_case(w, tma)
    assert torch.equal(out.cpu().view(torch.uint8), r8) and torch.equal(scale.cpu(), rs)
    # the dequantised output against the rotated input, as the reference compares them
    deq = dequant(out, scale, 8).cpu().reshape(T, 64, 512)
    x = w.o.float().view(T, 64, 512).clone()
    cs = w.cos_sin_cache[w.positions]
    c, s_ = cs[:, None, :32], cs[:, None, 32:]
    e, o = x[..., 448::2].clone(), x[..., 449::2].clone()
    x[..., 448::2], x[..., 449::2] = e * c + o * s_, o * c - e * s_
    cos = torch.nn.functional.cosine_similarity(deq.flatten(), x.flatten(), dim=0)
    assert float(1 - cos) < 1e-3


# ------------------------------------------------- other geometries ----

from .test_oracle_pins import SIBLING_GEOMETRIES, _packed_ok  # noqa: E402


@pytest.mark.parametrize("tma", [False, True])
@pytest.mark.parametrize("nope,rope,group", SIBLING_GEOMETRIES)
def test_other_geometries_match_oracle(nope, rope, group, tma):
    """Every geometry the reference accepts (head_dim 64..512, groups 32..512,
    rope 2..128 dims, rope starting inside a 16-byte piece), codes and scales
    bit for bit against the oracle; ragged token counts (pad tokens' scales
    zero); o a strided view (head and token strides beyond head_dim)."""
    D = nope + rope
    for T, H, G in ((5, 8, 2), (37, 4, 4), (64, 16, 16)):
        hpg = H // G
        if tma and not _packed_ok(nope, rope, group, hpg):
            continue
        _say(f"inv rope geometry nope={nope} rope={rope} group={group} T={T} H={H} G={G} tma={tma}")
        w = W.make_inv_rope_workload(T, H, G, seed=D + group + T, max_pos=1024, head_dim=D, rope_dim=rope)
        # o inside a wider buffer: head stride D + 8, token stride H * (D + 8) + 16
        buf = torch.zeros(T, H * (D + 8) + 16, dtype=torch.bfloat16)
        view = buf[:, :H * (D + 8)].view(T, H, D + 8)[..., :D]
        view.copy_(w.o)
        dbuf = buf.to(DEV)
        do = dbuf[:, :H * (D + 8)].view(T, H, D + 8)[..., :D]
        kw = dict(nope_dim=nope, rope_dim=rope, quant_group_size=group, tma_aligned_scales=tma)
        out, scale = flaggems_vllm.fused_inv_rope_fp8_quant(do, w.positions.to(DEV), w.cos_sin_cache.to(DEV),
                                                            G, hpg, **kw)
        torch.cuda.synchronize()
        r8, rs = oracle.inv_rope_fp8_quant(w.o, w.positions, w.cos_sin_cache, G, hpg, **kw)
        assert out.shape == (T, G, hpg * D) and out.stride() == r8.stride()
        assert torch.equal(out.cpu().view(torch.uint8), r8)
        assert scale.shape == rs.shape and scale.stride() == rs.stride()
        assert torch.equal(scale.cpu(), rs)
        tpad = (T + 3) // 4 * 4
        if tpad > T:  # the pad tokens' scales are zero, as the reference writes them
            store = torch.as_strided(scale, (G, scale.shape[-1], tpad), (scale.stride(1), scale.stride(2), 1))
            assert int(store[..., T:].cpu().view(torch.int32).abs().sum()) == 0
