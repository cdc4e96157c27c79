"""fused_q_kv_rmsnorm: CPU pins of its oracle and GPU parity.

Reference: src/flaggems_vllm/ops/deepseek_v4_attention_fused_q_kv_rmsnorm.py:24-103,
tests/test_deepseek_v4_attention_fused_q_kv_rmsnorm.py:40-76 (shapes
(4, 256, 128) and (8, 1536, 512); torch reference ``_rmsnorm_ref``).
"""
import decimal
import struct
from fractions import Fraction

import pytest
import torch

import oracle
from flaggems_vllm import testing as W
from oracle import torch_ref

from ._helpers import bf16_ulp_distance

DEV = torch.device("cuda:0")


def _f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def _inputs(T, qdim, kvdim, seed, wdtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    qr = W.randn_bf16((T, qdim), g)
    kv = W.randn_bf16((T, kvdim), g)
    qw = W.randn_bf16((qdim,), g).to(wdtype)
    kw = W.randn_bf16((kvdim,), g).to(wdtype)
    return qr, kv, qw, kw


def test_oracle_row_is_exactly_rounded():
    """y_i = bf16(fl32(fl32(x_i * r) * w_i)) with r from the exact sum of
    squares and a correctly rounded rsqrt, for both row sizes."""
    decimal.getcontext().prec = 60
    qr, kv, qw, kw = _inputs(3, 1536, 512, 1)
    qo, ko = oracle.fused_q_kv_rmsnorm(qr, kv, qw, kw, 1e-6)
    for x, w, y in ((qr, qw, qo), (kv, kw, ko)):
        for t in range(x.shape[0]):
            xs = x[t].float().tolist()
            var = sum(Fraction(v) ** 2 for v in xs) / len(xs)
            r = _f32(float(1 / decimal.Decimal(_f32(_f32(float(var)) + _f32(1e-6))).sqrt()))
            ws = w.float().tolist()
            want = torch.tensor([_f32(_f32(v * r) * wi) for v, wi in zip(xs, ws)]).to(torch.bfloat16)
            assert torch.equal(y[t], want)


@pytest.mark.parametrize("T,qdim,kvdim", [(4, 256, 128), (8, 1536, 512), (64, 1536, 512)])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_oracle_vs_torch_ref(T, qdim, kvdim, wdtype):
    qr, kv, qw, kw = _inputs(T, qdim, kvdim, 2, wdtype)
    qo, ko = oracle.fused_q_kv_rmsnorm(qr, kv, qw, kw, 1e-6)
    tq, tk = torch_ref.fused_q_kv_rmsnorm(qr, kv, qw, kw, 1e-6)
    assert int(bf16_ulp_distance(qo, tq).max()) <= 1
    assert int(bf16_ulp_distance(ko, tk).max()) <= 1


# ------------------------------------------------------------------- GPU ----

def _gpu(qr, kv, qw, kw, eps):
    import flaggems_vllm

    qo, ko = flaggems_vllm.fused_q_kv_rmsnorm(qr.to(DEV), kv.to(DEV), qw.to(DEV), kw.to(DEV), eps)
    torch.cuda.synchronize()
    return qo.cpu(), ko.cpu()


@pytest.mark.gpu
@pytest.mark.parametrize("T,qdim,kvdim", [(4, 256, 128), (8, 1536, 512), (1, 1536, 512),
                                          (8192, 1536, 512), (33, 4096, 64),
                                          # either side of each row-shape boundary (512, 1536, 2048)
                                          (17, 520, 1536), (9, 1544, 1024), (5, 2048, 2056),
                                          # a workgroup per row past 4096; the reference benchmark's
                                          # 64 x 576-wide q rows (benchmark/test_deepseek_v4_attention_fused_q_kv_rmsnorm.py:64)
                                          (32, 36864, 576), (3, 4104, 520), (2, 512, 8200), (1, 4096, 4104),
                                          # 16384 / 16392: 8 or 24 pieces per thread; 49160: a second chunk
                                          (3, 16384, 16392), (2, 49160, 520),
                                          # hoisted weight loads up to two workgroups per CU, then not
                                          (4096, 1536, 512), (700, 4104, 512),
                                          # grids beyond one round: launched with the LDS reservation
                                          (16384, 1536, 512), (8192, 4096, 512)])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_gpu_matches_oracle(T, qdim, kvdim, wdtype):
    print(f"\n[case] rmsnorm T={T} q={qdim} kv={kvdim} w={wdtype}", flush=True)
    qr, kv, qw, kw = _inputs(T, qdim, kvdim, 3, wdtype)
    qo, ko = _gpu(qr, kv, qw, kw, 1e-6)
    rq, rk = oracle.fused_q_kv_rmsnorm(qr, kv, qw, kw, 1e-6)
    assert torch.equal(qo, rq) and torch.equal(ko, rk)
    tq, tk = torch_ref.fused_q_kv_rmsnorm(qr, kv, qw, kw, 1e-6)
    assert int(bf16_ulp_distance(qo, tq).max()) <= 1 and int(bf16_ulp_distance(ko, tk).max()) <= 1


@pytest.mark.gpu
def test_gpu_strided_rows():
    """qr and kv as column slices of one fused projection buffer."""
    print("\n[case] rmsnorm strided", flush=True)
    g = torch.Generator().manual_seed(4)
    buf = W.randn_bf16((100, 1536 + 512 + 64), g)
    qr, kv = buf[:, :1536], buf[:, 1536:2048]
    qw, kw = W.randn_bf16((1536,), g), W.randn_bf16((512,), g)
    d = buf.to(DEV)
    import flaggems_vllm

    qo, ko = flaggems_vllm.fused_q_kv_rmsnorm(d[:, :1536], d[:, 1536:2048], qw.to(DEV), kw.to(DEV), 1e-6)
    torch.cuda.synchronize()
    rq, rk = oracle.fused_q_kv_rmsnorm(qr, kv, qw, kw, 1e-6)
    assert torch.equal(qo.cpu(), rq) and torch.equal(ko.cpu(), rk)
