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


@pytest.fixture(scope="session")
def kernel_gelu(cuda):
    """x -> the GPU's dtype(gelu_tanh(x)) elementwise (on the CPU, bf16 or f16 x), from a table of
    every 16-bit pattern read out of the FP8 GEMM's GELU epilogue: with zero weights the GEMM's y
    is its bias exactly, so an output row is dtype(gelu_tanh(bias)) with every pattern as the bias.
    The row quantizer's GELU is the same device function.  -0 is set by hand: the epilogue's
    0 * scale + (-0) is +0, while gelu_tanh(-0) = -0 * 0.5 = -0."""
    import torch
    from xgen_amd import _native as N
    ops = torch.ops.xgen_amd
    one = torch.ones(1, device=cuda)
    qa = torch.zeros((16, 16), dtype=torch.float8_e4m3fn, device=cuda)
    qw = torch.zeros((1 << 16, 16), dtype=torch.float8_e4m3fn, device=cuda)
    tables = {}
    for dt in (torch.bfloat16, torch.float16):
        bias = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(dt).to(cuda)
        y, _ = ops.scaled_mm(qa, qw, one, one, bias, dt, N.ACT_GELU_TANH, False)
        t = y[0].cpu().clone()
        t[0x8000] = -0.0
        tables[dt] = t

    def gelu(x):
        return tables[x.dtype][x.detach().cpu().contiguous().view(torch.int16).long() & 0xFFFF]
    return gelu
