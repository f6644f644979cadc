import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The GPU the HIP library runs on; GPU tests fail (not skip) when the
    library is missing, so a silent fallback can never pass them."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import relux_amd
    relux_amd.load()
    from relux_amd import _lib
    _lib.init(0)
    return torch.device("cuda", 0)
