"""Shared test setup.

Markers: ``gpu`` -- needs an MI355X (run with ``-m gpu`` on the GPU box);
everything else runs on the CPU.  Tests import the oracle (``oracle/``) only
as the checker."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle

    oracle.lib()  # fail loudly if the oracle library is not built
    return oracle


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    """The GPU device; GPU tests fail (not skip) when none is present, so a
    round-end run on a GPU box can never pass on a silent CPU path."""
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    name = torch.cuda.get_device_properties(0).gcnArchName
    assert name.startswith("gfx950"), f"expected gfx950, got {name}"
    return torch.device("cuda:0")
