import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs HIP kernels on an MI355X (gfx950)")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests are skipped only where no GPU exists at all."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this environment")
    from torch2iron_amd import _lib
    _lib.load()   # fails loudly if the HIP library is missing
    return torch.device("cuda:0")
