"""The C ABI from a C program (tests/c_abi/drop_in.c): no torch and no Python in the process that
drives the kernels, the quantizers' bytes and scales bit-exact against the oracle's C restatement,
INT8 accumulators exact, FP8 accumulators within each kind's bound, and the error contract.  Built
by __graft_entry__.build() (tests/c_abi/build.py)."""
import subprocess
from pathlib import Path

import pytest

BINARY = Path(__file__).resolve().parent / "c_abi" / "_build" / "drop_in"


def run_binary():
    if not BINARY.is_file():
        pytest.fail(f"{BINARY} is not built: run __graft_entry__.build()")
    return subprocess.run([str(BINARY)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)


def test_program_loads_and_reports_no_device(built_library):
    """On a host without a HIP device the program loads its libraries and exits 77 (built here, with
    the oracle's library, when absent: gcc takes seconds)."""
    import importlib.util

    import torch
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present: the GPU test runs the program")
    if not BINARY.is_file():
        from oracle import build as oracle_build
        oracle_build.build()
        spec = importlib.util.spec_from_file_location("xgen_c_abi_build", BINARY.parents[1] / "build.py")
        builder = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(builder)
        builder.build()
    proc = run_binary()
    assert proc.returncode == 77, proc.stdout
    assert "no HIP device" in proc.stdout


@pytest.mark.gpu
def test_c_program_drives_the_path(cuda):
    proc = run_binary()
    print(proc.stdout, flush=True)
    assert proc.returncode == 0, proc.stdout
    assert "c abi ok" in proc.stdout
