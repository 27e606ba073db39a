import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a visible MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def ext(cuda_device):
    from texelator_amd import runtime

    return runtime.extension()


@pytest.fixture(scope="session")
def oracle_threads():
    from oracle import clib

    n = min(16, len(os.sched_getaffinity(0)))
    clib.set_threads(n)
    return n
