import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libcoopt_amd.so")


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with the library loaded; skips only when the machine has no GPU at all."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU on this machine")
    from iitj_llm_coopt_amd import _lib

    _lib.load()  # raises if the library is missing or bound to another HIP runtime
    return torch.device("cuda:0")
