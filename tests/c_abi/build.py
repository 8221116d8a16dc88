"""Builds tests/c_abi/drop_in.c (a C program that drives the C ABI with no torch) into
tests/c_abi/_build/drop_in with gcc, linked against the built libxgen_amd.so, the oracle's
liboracle_quant.so and the HIP runtime; run paths relative to the binary, so the tree can move.
Test infrastructure, called by __graft_entry__.build() after both libraries are built."""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
OUT = HERE / "_build" / "drop_in"


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    cc = shutil.which("gcc") or "cc"
    tmp = OUT.with_name(OUT.name + ".tmp")
    cmd = [cc, "-O2", "-std=c11", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}", f"-I{ROCM / 'include'}",
           str(HERE / "drop_in.c"), "-o", str(tmp),
           f"-L{ROOT / 'xgen_amd' / '_lib'}", "-lxgen_amd", f"-L{ROOT / 'oracle' / '_lib'}", "-loracle_quant",
           f"-L{ROCM / 'lib'}", "-lamdhip64", "-lm",
           "-Wl,-rpath,$ORIGIN/../../../xgen_amd/_lib:$ORIGIN/../../../oracle/_lib:" + str(ROCM / "lib")]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"C ABI test program build failed:\n{proc.stdout}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
