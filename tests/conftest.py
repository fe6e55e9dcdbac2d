import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The GPU tests run only where a GPU is expected; a missing device is an error, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected but torch.cuda.is_available() is False")
    from logitfill_amd import _native

    _native.load()  # raises NativeLibraryMissing when the HIP library is not built
    return torch.device("cuda", 0)


def pytest_collection_modifyitems(config, items):
    # Print the test name before each GPU test so a fault names its case.
    if os.environ.get("LF_TRACE_TESTS"):
        for item in items:
            item.add_marker(pytest.mark.usefixtures())
