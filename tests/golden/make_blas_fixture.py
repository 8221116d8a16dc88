"""Writes tests/golden/fp8_blas_gemm.npz: FP8 GEMMs computed by torch._scaled_mm on an
MI355X (hipBLASLt, a library independent of this build), the call the reference makes
(x_base/x_base/operator/h3_fp8.py:63-66, use_fast_accum=False), with unit per-tensor
scales and float32 output, so its outputs are the raw K sums.  They pin the oracle's
model of gfx950's FP8 matrix sum (oracle/mfma_model.c) to an implementation that shares
no code with xgen_amd (tests/test_oracle_mfma.py).  Runs on an MI355X:

    python tests/golden/make_blas_fixture.py

Contents (e4m3fn codes as uint8, sums as float32):
  rowq_a [16,3072], rowq_w [32,3072], rowq_acc [16,32]   operands from the per-row FP8
      quantizer's arithmetic (N(0,1) activations with a x50 outlier channel, N(0,0.02)
      weights; quantized on the CPU by the oracle)
  gelu_a [8,12288], gelu_w [16,12288], gelu_acc [8,16]    FFN-down-like operands: the
      quantized GELU-tanh of N(0,1) activations against N(0,0.02) weights, K = 12,288
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle.ref as R  # noqa: E402

FP8 = torch.float8_e4m3fn


def blas(qa: torch.Tensor, qw: torch.Tensor) -> np.ndarray:
    dev = torch.device("cuda:0")
    one = torch.ones((), device=dev)
    out = torch._scaled_mm(qa.to(dev), qw.to(dev).t(), scale_a=one, scale_b=one, out_dtype=torch.float32,
                           use_fast_accum=False)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def main() -> None:
    g = torch.Generator().manual_seed(2026)
    x = torch.randn((16, 3072), generator=g)
    x[:, 1234] *= 50
    qa, _ = R.quantize_rows_fp8(x.to(torch.bfloat16))
    qw, _ = R.quantize_rows_fp8((torch.randn((32, 3072), generator=g) * 0.02).to(torch.bfloat16))
    h = torch.nn.functional.gelu(torch.randn((8, 12288), generator=g), approximate="tanh")
    qh, _ = R.quantize_rows_fp8(h.to(torch.bfloat16))
    qd, _ = R.quantize_rows_fp8((torch.randn((16, 12288), generator=g) * 0.02).to(torch.bfloat16))
    u8 = lambda t: t.view(torch.uint8).numpy()  # noqa: E731
    np.savez_compressed(HERE / "fp8_blas_gemm.npz",
                        rowq_a=u8(qa), rowq_w=u8(qw), rowq_acc=blas(qa, qw),
                        gelu_a=u8(qh), gelu_w=u8(qd), gelu_acc=blas(qh, qd))
    print("wrote", HERE / "fp8_blas_gemm.npz")


if __name__ == "__main__":
    main()
