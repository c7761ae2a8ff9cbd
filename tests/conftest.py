import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for sub in ("glacier.serve_amd", "oracle", "tests/golden"):
    p = str(ROOT / sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X); run with -m gpu")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def torch_mod():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    return torch


@pytest.fixture(scope="session")
def gsp(torch_mod):
    """The product binding; a missing library is an error, never a skip."""
    import glacier_paged

    glacier_paged.load()
    return glacier_paged


@pytest.fixture(scope="session")
def ctx(gsp):
    c = gsp.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="session")
def oracle():
    import glacier_oracle

    glacier_oracle.load()
    return glacier_oracle


def threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except Exception:
        n = os.cpu_count() or 1
    return max(1, min(16, n))
