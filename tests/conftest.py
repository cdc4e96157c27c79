import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "flaggems-vllm_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session", autouse=True)
def _oracle_built():
    """The CPU oracle is built by __graft_entry__.build(); build it here only
    if nothing is built yet (gcc, a second or two)."""
    import oracle

    if not os.path.exists(oracle._LIB_PATH):
        oracle.build()
    yield


def gpu_available():
    import torch

    return torch.cuda.is_available()
