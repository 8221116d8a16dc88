"""Pins the oracle's FP8 functions (e4m3 codec, per-tensor and per-row quantizers,
the kernels' fast division) against torch, reference known answers and brute force."""
import concurrent.futures

import numpy as np
import pytest
import torch

import oracle.ref as R


def all_bf16_values() -> np.ndarray:
    return (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)


def canon(codes: np.ndarray) -> np.ndarray:
    c = codes.copy()
    c[(c & 0x7F) == 0x7F] = 0x7F
    return c


def torch_e4m3(v: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(v)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_encoder_matches_torch_on_every_bf16_value():
    v = all_bf16_values()
    assert np.array_equal(canon(R.e4m3_encode(v)), canon(torch_e4m3(v)))


def test_encoder_matches_torch_on_random_floats():
    rng = np.random.default_rng(0)
    mag = np.exp2(rng.uniform(-14, 9.2, 1 << 20)).astype(np.float32)
    v = (mag * rng.choice([-1.0, 1.0], mag.size)).astype(np.float32)
    # also every representable midpoint and its neighbours
    table = R.e4m3_decode_table()
    finite = np.sort(np.unique(table[np.isfinite(table)]))
    mids = ((finite[1:].astype(np.float64) + finite[:-1]) / 2).astype(np.float32)
    near = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])
    v = np.concatenate([v, near]).astype(np.float32)
    assert np.array_equal(canon(R.e4m3_encode(v)), canon(torch_e4m3(v)))


@pytest.mark.parametrize("value,code", [
    (2.0 ** -9, 0x01), (1.5 * 2.0 ** -9, 0x02), (2.5 * 2.0 ** -9, 0x02), (2.0 ** -10, 0x00),
    (1.0625, 0x38), (1.1875, 0x3A), (448.0, 0x7E), (463.99, 0x7E), (464.0, 0x7E), (464.00003, 0x7F), (1e9, 0x7F),
    (-0.0, 0x80), (-448.0, 0xFE), (2.0 ** -6, 0x08), (0.0, 0x00), (float("nan"), 0x7F),
])
def test_encoder_closed_forms(value, code):
    assert int(R.e4m3_encode(np.array([value], np.float32))[0]) == code


def test_decode_table_matches_torch():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    ours = R.e4m3_decode_table()
    both_nan = np.isnan(ref) & np.isnan(ours)
    assert np.array_equal(np.isnan(ref), np.isnan(ours))
    assert np.array_equal(ref[~both_nan], ours[~both_nan])


def test_zero_quantization_is_finite():
    # x_base/tests/test_h3_cuda_precision_ops.py:8-11
    packed, scale = R.quantize_per_tensor(torch.zeros(16, 32))
    assert scale.item() > 0 and torch.isfinite(packed.float()).all()
    assert torch.equal(packed.float(), torch.zeros(16, 32))


def brute_force_e4m3(v: np.ndarray) -> np.ndarray:
    """Nearest finite e4m3 value by search over all codes; ties to the even code."""
    table = R.e4m3_decode_table().astype(np.float64)
    codes = np.arange(256)
    finite = np.isfinite(table)
    t, c = table[finite], codes[finite]
    out = np.empty(v.shape, np.uint8)
    for i, x in enumerate(v.astype(np.float64).ravel()):
        d = np.abs(t - x)
        cand = c[d == d.min()]
        # prefer the code with matching sign for zero, then the even mantissa
        if len(cand) > 1:
            cand = [k for k in cand if (k & 0x80) == (0x80 if np.signbit(x) else 0)] or list(cand)
            cand = [k for k in cand if k % 2 == 0] or cand
        out.flat[i] = cand[0]
    return out


def test_linspace_weight_bytes_against_brute_force():
    # the weight of x_diffusers/tests/test_h3_tp_cp.py:42-66
    w = torch.linspace(-2, 3, 192 * 64).reshape(192, 64).to(torch.bfloat16)
    packed, scale = R.quantize_per_tensor(w)
    expected_scale = (w.float().abs().amax() / 448).clamp_min(torch.finfo(torch.float32).tiny)
    assert torch.equal(scale, expected_scale)
    q = (w.float() / scale).clamp(-448, 448).numpy()
    assert np.array_equal(packed.view(torch.uint8).numpy(), brute_force_e4m3(q))


def edge_rows(K, dtype):
    rows = [torch.zeros(K), torch.full((K,), -0.0), torch.randn(K), torch.randn(K) * 1e-30,
            torch.randn(K) * 3e4, torch.linspace(-448, 448, K)]
    r = torch.randn(K); r[K // 3] = float("inf"); rows.append(r)
    r = torch.randn(K); r[K // 5] = float("nan"); rows.append(r)
    r = torch.randn(K); r[1] = -float("inf"); r[2] = float("inf"); rows.append(r)
    return torch.stack(rows).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_row_quantizer_torch_equals_c(dtype):
    torch.manual_seed(0)
    x = torch.cat([torch.randn(64, 384).to(dtype), edge_rows(384, dtype)])
    x[:, 7] = x[:, 7] * 50
    q_t, s_t = R.quantize_rows_fp8(x)
    q_c, s_c = R.quantize_rows_c(x, "fp8")
    assert torch.equal(q_t.view(torch.uint8), q_c.view(torch.uint8))
    assert torch.equal(s_t.view(torch.int32), s_c.view(torch.int32))


def test_row_quantizer_is_per_tensor_on_each_row():
    torch.manual_seed(1)
    x = torch.randn(12, 96, dtype=torch.bfloat16) * torch.logspace(-3, 3, 12)[:, None].to(torch.bfloat16)
    q, s = R.quantize_rows_fp8(x)
    for r in range(x.shape[0]):
        qr, sr = R.quantize_per_tensor(x[r:r + 1])
        assert torch.equal(q[r:r + 1].view(torch.uint8), qr.view(torch.uint8))
        assert torch.equal(s[r], sr)


def test_nan_rows_are_canonical_nan():
    x = torch.randn(2, 64, dtype=torch.bfloat16)
    x[0, 3] = float("nan")
    q, s = R.quantize_rows_fp8(x)
    assert torch.isnan(s[0]) and not torch.isnan(s[1])
    assert (q[0].view(torch.uint8) == 0x7F).all()


@pytest.mark.parametrize("fmt,hi", [(0, 0x7F7F), (1, 0x7BFF)])
def test_fast_division_exhaustive(fmt, hi):
    """Every (x, amax) pair of 16-bit inputs: the kernels' division gives IEEE's e4m3 byte."""
    L = R.clib()
    # work per amax grows with amax (every x <= amax is checked): equal-work slices
    bounds = np.concatenate([[1], (np.sqrt(np.linspace(0, 1, 9)[1:]) * hi).astype(np.int64) + 1])
    with concurrent.futures.ThreadPoolExecutor(8) as pool:
        bad = sum(pool.map(lambda i: L.oracle_check_fast_division(fmt, int(bounds[i]), int(bounds[i + 1] - 1)),
                           range(8)))
    assert bad == 0


@pytest.mark.parametrize("fmt", [0, 1])
def test_row_scale_two_operation_division_exhaustive(fmt):
    """The kernels' row scale max(amax / 448, FLT_MIN) (fp8_row_scale in xgen_common.h): the
    quotient as amax * r_hi + RN(amax * r_lo) with the constants of 1/448 (IEEE division below
    2^-90) equals IEEE division + clamp for every 16-bit amax (bf16 and f16, both signs, zeros,
    subnormals, infinities, NaN); and the kernel's constants are the oracle's."""
    import ctypes
    import re
    from tests.conftest import ROOT
    L = R.clib()
    r_hi, r_lo = ctypes.c_float(), ctypes.c_float()
    assert L.oracle_check_scale_division(fmt, ctypes.byref(r_hi), ctypes.byref(r_lo)) == 0
    header = (ROOT / "xgen_amd" / "csrc" / "xgen_common.h").read_text()
    m = re.search(r"kInv448Hi = (0x[0-9a-fp.+-]+)f, kInv448Lo = (0x[0-9a-fp.+-]+)f", header)
    assert m and float.fromhex(m.group(1)) == r_hi.value and float.fromhex(m.group(2)) == r_lo.value
    # the constants are 1/448 split: r_hi rounded toward zero, r_hi + r_lo within 2^-45 relative
    assert r_hi.value <= 1 / 448 and abs((r_hi.value + r_lo.value) * 448 - 1) < 2.0 ** -45


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_row_quantizer_symmetries(dtype):
    """Properties the arithmetic fixes, on random rows of both input types: negating a row flips
    exactly the sign bit of every byte (round to nearest even commutes with negation; -0 -> 0x80)
    and keeps its scale; scaling a row by 2^k (no under- or overflow of the values or the scale)
    keeps every byte and scales the scale by exactly 2^k; permuting a row's columns permutes its
    bytes.  A mistaken sign, index or scale would break one of them."""
    torch.manual_seed(3)
    x = (torch.randn(40, 200) * torch.logspace(-2, 2, 40)[:, None]).to(dtype)
    q, s = R.quantize_rows_fp8(x)
    qn, sn = R.quantize_rows_fp8(-x)
    assert torch.equal(qn.view(torch.uint8), q.view(torch.uint8) ^ 0x80)
    assert torch.equal(sn, s)
    for k in (-3, 1, 4):
        qk, sk = R.quantize_rows_fp8((x.float() * 2.0 ** k).to(dtype))
        assert torch.equal(qk.view(torch.uint8), q.view(torch.uint8))
        assert torch.equal(sk, s * 2.0 ** k)
    perm = torch.randperm(200, generator=torch.Generator().manual_seed(4))
    qp, sp = R.quantize_rows_fp8(x[:, perm])
    assert torch.equal(qp.view(torch.uint8), q.view(torch.uint8)[:, perm]) and torch.equal(sp, s)
