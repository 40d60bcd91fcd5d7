"""Test configuration: markers, import paths, shared fixtures.

CPU tests (-m "not gpu") cover the oracle against golden vectors and
closed-form/independent checks, the host logic and the C-ABI library surface.
GPU tests (-m gpu) run the HIP path through the engine C ABI and compare it
with the oracle on the same seeded inputs.
"""
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "netra-kernel_amd", REPO / "oracle", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle
    oracle.build()
    return oracle
