"""Writes the golden fixtures of the W8A8 linear path (tests/golden/*.safetensors).

The reference repository holds no golden-vector files, so these are small
seeded cases whose expected outputs come from the CPU oracle (oracle/ref.py),
itself pinned by the closed-form, exhaustive and brute-force checks under
tests/test_oracle_*.py.  Committed fixtures freeze those outputs: the CPU
suite checks that the oracle still reproduces them bit for bit, the GPU suite
checks the HIP kernels against them without running the oracle.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import oracle.ref as R  # noqa: E402


def special_rows(K: int, dtype) -> torch.Tensor:
    """Rows that exercise the quantizers' edge cases: zeros, NaN, +-inf, -0,
    subnormals, exact e4m3 rounding midpoints, the 448 / 464 boundaries."""
    rows = torch.zeros(8, K)
    rows[1, 5] = float("nan")
    rows[2, :] = torch.linspace(-3, 3, K)
    rows[2, 7] = float("inf")
    rows[3, :] = -0.0
    rows[3, 1] = 2.0 ** -130 if dtype == torch.bfloat16 else 2.0 ** -20
    rows[4, :] = torch.linspace(-448, 448, K)
    rows[4, 0], rows[4, 1] = 464.0, -464.0
    # amax exactly 448 (scale 1): e4m3 rounding midpoints, ties to even
    mids = torch.tensor([1.0625, 1.1875, 2.125, 17.0, 272.0, 1.5 * 2.0 ** -9, 0.5 * 2.0 ** -9])
    rows[5, :] = torch.cat([mids, -mids]).repeat(K // 14 + 1)[:K]
    rows[5, 0] = 448.0
    rows[6, :] = 1.0
    rows[6, 3] = 500.0
    rows[7, :] = torch.arange(K) % 17 - 8.0
    return rows.to(dtype)


def quantizer_cases():
    g = torch.Generator().manual_seed(11)
    out = {}
    for tag, dtype in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        K = 520
        x = torch.cat([special_rows(K, dtype), (torch.randn(29, K, generator=g) * 3).to(dtype)])
        x[9:, 17] = (x[9:, 17].float() * 50).to(dtype)  # an outlier channel
        q8, s8 = R.quantize_rows_fp8(x)
        qi, si = R.quantize_rows_int8(x)
        out[f"rows_{tag}_x"] = x
        out[f"rows_{tag}_fp8_q"] = q8.view(torch.uint8)
        out[f"rows_{tag}_fp8_s"] = s8
        out[f"rows_{tag}_int8_q"] = qi
        out[f"rows_{tag}_int8_s"] = si
        xt = (torch.randn(32, 128, generator=g) * 2).to(dtype)
        qt, st = R.quantize_per_tensor(xt)
        out[f"tensor_{tag}_x"] = xt
        out[f"tensor_{tag}_q"] = qt.view(torch.uint8)
        out[f"tensor_{tag}_s"] = st.reshape(1)
    return out


def front_end_cases():
    g = torch.Generator().manual_seed(12)
    B, S, H, T = 2, 37, 256, 5
    x = torch.randn(B, S, H, generator=g)
    x[..., 3] *= 50
    x = x.to(torch.bfloat16)
    scale = (torch.randn(T, H, generator=g) * 0.1).to(torch.bfloat16)
    shift = (torch.randn(T, H, generator=g) * 0.1).to(torch.bfloat16)
    idx = torch.randint(T, (S,), generator=g)
    w = (torch.randn(H, generator=g) * 0.5 + 1).to(torch.bfloat16)
    out = {"fe_x": x, "fe_scale": scale, "fe_shift": shift, "fe_idx": idx, "fe_w": w}
    for norm, out_t, weight, eps in (("layer", "fp8", None, 1e-6), ("rms", "int8", w, 1e-5), ("rms", "fp8", w, 1e-5)):
        q, s, m = R.norm_affine_quant(x, weight, scale, shift, idx, eps, norm, out_t)
        key = f"fe_{norm}_{out_t}"
        out[key + "_q"] = q.view(torch.uint8) if out_t == "fp8" else q
        out[key + "_s"] = s
        out[key + "_m"] = m
    return out


def gemm_cases():
    g = torch.Generator().manual_seed(13)
    M, K, N = 48, 256, 96
    x = torch.randn(M, K, generator=g)
    x[:, 9] *= 50
    x = x.to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(N, generator=g) * 0.01).to(torch.bfloat16)
    out = {"mm_x": x, "mm_w": w, "mm_b": b}
    qa, sa = R.quantize_rows_fp8(x)
    qw, sw = R.quantize_rows_fp8(w)
    out.update(mm_fp8_qa=qa.view(torch.uint8), mm_fp8_sa=sa, mm_fp8_qw=qw.view(torch.uint8), mm_fp8_sw=sw,
               mm_fp8_acc=R.fp8_accumulate_exact(qa, qw),
               mm_fp8_out=R.w8a8_linear_fp8(qa, sa, qw, sw, b),
               mm_fp8_out_gelu=R.w8a8_linear_fp8(qa, sa, qw, sw, b, torch.bfloat16, "gelu_tanh"))
    qa, sa = R.quantize_rows_int8(x)
    qw, sw = R.quantize_rows_int8(w)
    out.update(mm_int8_qa=qa, mm_int8_sa=sa, mm_int8_qw=qw, mm_int8_sw=sw,
               mm_int8_acc=R.int8_accumulate_exact(qa, qw).to(torch.int32),
               mm_int8_out=R.w8a8_linear_int8(qa, sa, qw, sw, b))
    return out


def build() -> dict:
    tensors = {}
    for part in (quantizer_cases(), front_end_cases(), gemm_cases()):
        tensors.update(part)
    return {k: v.contiguous() for k, v in tensors.items()}


if __name__ == "__main__":
    t = build()
    path = HERE / "w8a8_path.safetensors"
    save_file(t, str(path))
    print(f"wrote {path} ({path.stat().st_size} bytes, {len(t)} tensors)")
