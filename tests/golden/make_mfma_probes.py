"""Writes tests/golden/mfma_fp8_probes.npz: inputs and the GPU's outputs of
single-instruction probes of gfx950's FP8 matrix arithmetic, the fixture that
pins oracle/mfma_model.c (tests/test_oracle_mfma.py).  Runs on an MI355X:

    python tests/golden/make_mfma_probes.py

It builds tests/golden/mfma_probe.hip with hipcc (a test tool, not part of
xgen_amd) and uses libxgen_amd's xgen_scaled_mm_fp8 for one full-K GEMM.

Contents (all bytes are e4m3fn codes; one row per problem where every row of
the problem is the same):
  group_a/_b [4096,64], group_d [4096]   product 256*256 at K index q and 1*1 at r
                                         (q*64 + r), zeros elsewhere: which K
                                         share a truncation group
  width_a/_b [68,64], width_d [68]       2^E (E = 0..16) at K 0 against 1.875^2
                                         at K 1 or 9, either sign: window width
                                         and truncation direction
  cacc_a/_b [16,64], cacc_c [16], cacc_d [16]  a large accumulator input against
                                         small products (all 64, or 63)
  rand_a/_b [32,32,64], rand_d [32,32,32]     uniformly random finite codes
  rowq_a/_b [32,32,64], rowq_d [32,32,32]     rows of the per-row FP8 quantizer
                                         (N(0,1) activations with a x50 channel,
                                         N(0,0.02) weights)
  gemm_a [16,3072], gemm_w [64,3072], gemm_acc [16,64]  a K = 3,072 GEMM through
                                         xgen_scaled_mm_fp8 (48 chained instructions)
  decode [512]                           bf16 bits of codes 0..255 by
                                         v_cvt_scalef32_pk_bf16_fp8 (scale 1), low
                                         then high word
"""
from __future__ import annotations

import ctypes
import subprocess
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

FP8 = torch.float8_e4m3fn


def _code(v: float) -> int:
    return int(torch.tensor([v], dtype=torch.float32).to(FP8).view(torch.uint8)[0])


def _lib() -> ctypes.CDLL:
    so = HERE / "_mfma_probe.so"
    subprocess.run(["hipcc", "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                    str(HERE / "mfma_probe.hip"), "-o", str(so)], check=True)
    L = ctypes.CDLL(str(so))
    L.probe.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                        ctypes.c_int, ctypes.c_void_p]
    L.decode_all.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    return L


def _run(L, A: np.ndarray, B: np.ndarray, C: np.ndarray | None = None) -> np.ndarray:
    """A, B [n,32,64] uint8 -> D [n,32,32] float32 by v_mfma_f32_32x32x64_f8f6f4."""
    dev = torch.device("cuda:0")
    n = A.shape[0]
    tA, tB = torch.from_numpy(np.ascontiguousarray(A)).to(dev), torch.from_numpy(np.ascontiguousarray(B)).to(dev)
    tC = torch.zeros((n, 32, 32), device=dev) if C is None else torch.from_numpy(np.ascontiguousarray(C)).to(dev)
    tD = torch.empty((n, 32, 32), device=dev)
    assert L.probe(0, tA.data_ptr(), tB.data_ptr(), tC.data_ptr(), tD.data_ptr(), n,
                   torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    return tD.cpu().numpy()


def _rows(row_a: np.ndarray, row_b: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[n,64] rows -> [n,32,64] problems whose rows are all the same."""
    return (np.repeat(row_a[:, None, :], 32, axis=1), np.repeat(row_b[:, None, :], 32, axis=1))


def main() -> None:
    import oracle.ref as R
    import xgen_amd  # noqa: F401
    xops = torch.ops.xgen_amd
    L = _lib()
    out = {}
    big, one = _code(256.0), _code(1.0)
    ga = np.zeros((4096, 64), np.uint8)
    gb = np.zeros_like(ga)
    for q in range(64):
        for r in range(64):
            i = q * 64 + r
            ga[i, q] = gb[i, q] = big
            if r != q:
                ga[i, r] = gb[i, r] = one
    out["group_a"], out["group_b"] = ga, gb
    out["group_d"] = _run(L, *_rows(ga, gb))[:, 0, 0]

    wa = np.zeros((68, 64), np.uint8)
    wb = np.zeros_like(wa)
    for E in range(17):
        for u, (r, sb, ss) in enumerate(((1, 1, 1), (9, 1, 1), (1, 1, -1), (1, -1, 1))):
            i = E * 4 + u
            wa[i, 0], wb[i, 0] = _code(sb * 2.0 ** (E // 2)), _code(2.0 ** (E - E // 2))
            wa[i, r], wb[i, r] = _code(ss * 1.875), _code(1.875)
    out["width_a"], out["width_b"] = wa, wb
    out["width_d"] = _run(L, *_rows(wa, wb))[:, 0, 0]

    cases = [(2.0 ** 20, 2.0 ** -6, 1.0), (2.0 ** 20, 2.0 ** -9, 1.0), (2.0 ** 24, 1.0, 1.0), (2.0 ** 24 + 2, 1.0, 1.0),
             (65536.0, 1.0, 1.0), (-65536.0, 1.0, 1.0), (1.0, 2.0 ** -9, 2.0 ** -9), (1e6, 3.0, 1.875)]
    ca = np.zeros((16, 64), np.uint8)
    cb = np.zeros_like(ca)
    cc = np.zeros(16, np.float32)
    for t, (c, a, b) in enumerate(cases):
        for u, width in enumerate((64, 63)):
            ca[2 * t + u, :width], cb[2 * t + u, :width], cc[2 * t + u] = _code(a), _code(b), c
    out["cacc_a"], out["cacc_b"], out["cacc_c"] = ca, cb, cc
    A, B = _rows(ca, cb)
    out["cacc_d"] = _run(L, A, B, np.repeat(cc, 32 * 32).reshape(16, 32, 32))[:, 0, 0]

    rng = np.random.default_rng(0)
    ra = rng.integers(0, 256, (32, 32, 64), dtype=np.uint8)
    rb = rng.integers(0, 256, (32, 32, 64), dtype=np.uint8)
    ra[(ra & 0x7F) == 0x7F] = 0
    rb[(rb & 0x7F) == 0x7F] = 0
    out["rand_a"], out["rand_b"], out["rand_d"] = ra, rb, _run(L, ra, rb)

    x = rng.standard_normal((32 * 32, 64)).astype(np.float32)
    x[:, 5] *= 50
    w = (rng.standard_normal((32 * 32, 64)) * 0.02).astype(np.float32)
    qa = R.quantize_rows_fp8(torch.from_numpy(x).to(torch.bfloat16))[0].view(torch.uint8).numpy()
    qb = R.quantize_rows_fp8(torch.from_numpy(w).to(torch.bfloat16))[0].view(torch.uint8).numpy()
    qa, qb = qa.reshape(32, 32, 64), qb.reshape(32, 32, 64)
    out["rowq_a"], out["rowq_b"], out["rowq_d"] = qa, qb, _run(L, qa, qb)

    from xgen_amd import workloads
    dev = torch.device("cuda:0")
    inp = workloads.linear_inputs(16, 3072, 64, seed=7)
    qx, sx = xops.quantize_rows(inp.x.to(dev), FP8)
    qw, sw = xops.quantize_rows(inp.weight.to(dev), FP8)
    _, acc = xops.scaled_mm(qx, qw, sx, sw, None, torch.bfloat16, 0, True)
    out["gemm_a"], out["gemm_w"] = qx.cpu().view(torch.uint8).numpy(), qw.cpu().view(torch.uint8).numpy()
    out["gemm_acc"] = acc.cpu().numpy()

    dec = torch.empty(512, dtype=torch.int16, device=dev)
    assert L.decode_all(dec.data_ptr(), torch.cuda.current_stream().cuda_stream) == 0
    out["decode"] = dec.cpu().numpy().view(np.uint16)
    np.savez_compressed(HERE / "mfma_fp8_probes.npz", **out)
    print("wrote", HERE / "mfma_fp8_probes.npz")


if __name__ == "__main__":
    main()
