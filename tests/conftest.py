import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The torch device for GPU tests.  No GPU -> skip (these tests only run under -m gpu on the box)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from cuda_tempiler_amd import capi

    capi.lib()  # raises loudly if the HIP library is missing: no fallback path exists
    return torch.device("cuda:0")
