import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libxgen_amd.so")


@pytest.fixture(scope="session")
def built_library():
    """Path of libxgen_amd.so, building it (hipcc cross-compiles) if absent."""
    from xgen_amd import _native
    path = _native.library_path()
    if not path.is_file():
        from xgen_amd import _build
        _build.build()
    return path


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a HIP device")
    return torch.device("cuda:0")
