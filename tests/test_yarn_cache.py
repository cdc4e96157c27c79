"""Pins of the YaRN-scaled rotary table builder used as test input
(flaggems_vllm.testing.make_yarn_cos_sin_cache; reference builder
tests/test_fused_inv_rope_fp8_quant.py:36-64, 246-264)."""
import math

import torch

from flaggems_vllm import testing as W


def test_correction_range_known_answers():
    # d(r) = 64 ln(P / (2 pi r)) / (2 ln 1e4), worked by hand:
    # P = 65536: d(32) = 20.10 -> 20, d(1) = 32.15 -> 33
    # P = 4096:  d(32) = 10.47 -> 10, d(1) = 22.52 -> 23
    assert W.yarn_correction_range(32, 1, 64, 10000.0, 65536) == (20, 33)
    assert W.yarn_correction_range(32, 1, 64, 10000.0, 4096) == (10, 23)
    # clipping at both ends
    assert W.yarn_correction_range(1e9, 1e-9, 64, 10000.0, 4096) == (0, 63)


def test_frequencies_outside_the_band_are_exact():
    t = W.make_yarn_cos_sin_cache(4096, rows=2)  # band (10, 23)
    theta = torch.atan2(t[1, 32:], t[1, :32]).double()  # row 1: angle = theta itself
    extra = 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64)
    for j in range(32):
        if j <= 10:
            want = extra[j]
        elif j >= 23:
            want = extra[j] / 16
        else:
            r = (j - 10) / 13
            want = extra[j] / 16 * r + extra[j] * (1 - r)
        assert math.isclose(float(theta[j]), float(want), rel_tol=1e-6), j


def test_rows_and_identity():
    t = W.make_yarn_cos_sin_cache(256)
    assert t.shape == (256 * 16, 64) and t.dtype == torch.float32
    assert torch.equal(t[0], torch.cat([torch.ones(32), torch.zeros(32)]))
    # a prefix of rows equals the full table's first rows
    assert torch.equal(W.make_yarn_cos_sin_cache(256, rows=100), t[:100])
    # scaling factor 1 leaves the plain table, up to the blend's rounding of
    # theta: one binary32 ulp of theta < 0.1 in the band, times p < 4096, moves
    # the angle by at most 4096 * 0.1 * 2^-23 < 5e-5
    torch.testing.assert_close(W.make_yarn_cos_sin_cache(4096, scaling_factor=1, rows=4096),
                               W.make_cos_sin_cache(4096), rtol=0, atol=5e-5)
    # cos^2 + sin^2 = 1 on every row
    torch.testing.assert_close(t[:, :32] ** 2 + t[:, 32:] ** 2, torch.ones(4096, 32), rtol=0, atol=1e-6)
