"""bench.py's contract on the CPU: one GPU only, and the input rotation that
keeps small calls from running out of the 256 MB MALL."""
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_mall_sets_cover_twice_the_mall():
    mall = 256 << 20
    for nbytes in (34_014_808, 67_112_960, 185_326_804, 206_635_008, 86_625_120):
        k = bench.mall_sets(nbytes)
        assert k * nbytes > 2 * mall and (k - 1) * nbytes <= 2 * mall
    assert bench.mall_sets(1_089_142_784) == 1   # c2 alone exceeds it
    assert bench.mall_sets(1000) == 16           # capped


def test_rotating_cycles_through_every_set():
    calls = []
    step, k = bench.rotating(lambda i: (lambda: calls.append(i)), 100_000_000)
    assert k == 6
    for _ in range(13):
        step()
    assert calls == [i % 6 for i in range(13)]
