"""Pins the oracle's INT8 per-row quantizer (f2bc_kernel.asc:89-107) by a second
restatement and by the closed-form properties the arithmetic fixes."""
import numpy as np
import pytest
import torch

import oracle.ref as R


def rows(dtype):
    torch.manual_seed(0)
    x = torch.randn(96, 320)
    x[:8] *= torch.logspace(-20, 20, 8)[:, None]
    x[8] = 0
    x[9] = -0.0
    x[10, 5] = float("inf")
    x[11, 9] = float("nan")
    x[12] = torch.linspace(-127, 127, 320)
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_torch_restatement_equals_c(dtype):
    x = rows(dtype)
    q_t, s_t = R.quantize_rows_int8(x)
    q_c, s_c = R.quantize_rows_c(x, "int8")
    assert torch.equal(q_t, q_c)
    assert torch.equal(s_t.view(torch.int32), s_c.view(torch.int32))


def test_range_and_extremes():
    x = rows(torch.bfloat16)[:8].float()
    x = torch.cat([x, torch.randn(64, 320)]).to(torch.bfloat16)
    q, s = R.quantize_rows_int8(x)
    assert q.abs().max() <= 127
    am = x.float().abs().argmax(dim=-1)
    picked = q.gather(1, am[:, None]).squeeze(1)
    assert (picked.abs() == 127).all()
    # |x - q * s| <= s/2 (+ a few float32 ulps of the dequantized value)
    err = (x.float() - q.float() * s[:, None]).abs()
    bound = s[:, None] * 0.5 + x.float().abs() * 2e-6 + 1e-30
    assert (err <= bound).all()


def test_round_half_to_even_ties():
    # amax = 127 -> alpha = 127/127 = 1 exactly, so x*alpha = x: bf16 halves are exact ties
    vals = torch.tensor([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5, -126.5, 0.25, 64.5])
    q, s = R.quantize_rows_int8(vals[None].to(torch.bfloat16))
    assert q[0].tolist() == [127, 0, 2, 2, 0, -2, -2, 4, 126, -126, 0, 64]
    assert s[0].item() == np.float32(127.0) * np.float32(np.float32(1.0) / np.float32(127.0))


def test_zero_row_gives_zero_scale_and_bytes():
    # npu_fusion/f1b/op_kernel/swiglu_quant_kernel.asc:72-75
    q, s = R.quantize_rows_int8(torch.zeros(3, 64, dtype=torch.bfloat16))
    assert (q == 0).all() and (s == 0).all()


def test_scale_uses_reciprocal_multiplier():
    # scale = amax * fl(1/127), not amax / 127 (f2bc_kernel.asc:97): differs on some amax
    amax = torch.tensor([3.0, 5.0, 7.0, 1e-3, 123.456], dtype=torch.float32)
    x = torch.zeros(5, 16)
    x[:, 0] = amax
    _, s = R.quantize_rows_int8(x.to(torch.bfloat16))
    a = x[:, 0].to(torch.bfloat16).float()
    assert torch.equal(s, a * (torch.tensor(1.0) / 127.0))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_subnormal_amax_row_quantizes_to_zeros(dtype):
    """127/amax overflows for a subnormal amax: every product is non-finite or
    -0 * inf = NaN, and the row comes out as zeros (the flushed-zero-row rule),
    in the torch and the C restatement alike."""
    tiny = 2.0 ** -130 if dtype == torch.bfloat16 else 2.0 ** -24
    x = torch.zeros(2, 64)
    x[0, :] = -0.0
    x[0, 3] = tiny
    x[1, 5] = -tiny
    x = x.to(dtype)
    q, s = R.quantize_rows_int8(x)
    qc, sc = R.quantize_rows_c(x, "int8")
    if dtype == torch.bfloat16:   # f16's smallest subnormal still gives a finite 127/amax
        assert (q == 0).all()
    assert torch.equal(q, qc) and torch.equal(s.view(torch.int32), sc.view(torch.int32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_symmetries(dtype):
    """Negating a row negates every byte and keeps its scale (round half to even and the max are
    symmetric); scaling a row by 2^k keeps every byte and scales the scale by exactly 2^k (the
    multiplier 127/amax moves by 2^-k, each product is unchanged); permuting a row's columns permutes
    its bytes."""
    torch.manual_seed(5)
    x = (torch.randn(40, 200) * torch.logspace(-2, 2, 40)[:, None]).to(dtype)
    q, s = R.quantize_rows_int8(x)
    qn, sn = R.quantize_rows_int8(-x)
    assert torch.equal(qn, -q) and torch.equal(sn, s)
    for k in (-3, 1, 4):
        qk, sk = R.quantize_rows_int8((x.float() * 2.0 ** k).to(dtype))
        assert torch.equal(qk, q) and torch.equal(sk, s * 2.0 ** k)
    perm = torch.randperm(200, generator=torch.Generator().manual_seed(6))
    qp, sp = R.quantize_rows_int8(x[:, perm])
    assert torch.equal(qp, q[:, perm]) and torch.equal(sp, s)
