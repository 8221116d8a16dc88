"""Builds the oracle's C code (oracle/quant_ref.c, the quantizer restatement,
and oracle/mfma_model.c, the model of gfx950's FP8 matrix sum) with gcc into
oracle/_lib/liboracle_quant.so — test infrastructure only.

No reference source is compiled: the reference's path is Python/Triton plus
Ascend C kernels that need the CANN toolchain (absent), so there is no
oracle/_ref build."""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCES = (HERE / "quant_ref.c", HERE / "mfma_model.c")
OUT = HERE / "_lib" / "liboracle_quant.so"


def build(verbose: bool = False) -> Path:
    OUT.parent.mkdir(parents=True, exist_ok=True)
    cc = shutil.which("gcc") or "cc"
    tmp = OUT.with_suffix(".so.tmp")
    # -O2 without fast-math: IEEE float division, correctly rounded fmaf, no FTZ.
    cmd = [cc, "-O2", "-std=c11", "-fPIC", "-shared", "-fno-fast-math", "-ffp-contract=off",
           *map(str, SOURCES), "-o", str(tmp), "-lm"]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stdout}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
