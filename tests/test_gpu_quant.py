"""GPU parity of the quantizers: bytes and scales bit-exact against the oracle."""
import math

import numpy as np
import pytest
import torch

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd import _native as N
from xgen_amd import workloads
from xgen_amd.operator.h3_abs_peak import activation_abs_peak
from xgen_amd.operator.h3_fp8_quant import quantize_activation

pytestmark = pytest.mark.gpu
xops = torch.ops.xgen_amd


def u8(q):
    return q.detach().cpu().view(torch.uint8)


def assert_same_quant(q_gpu, s_gpu, q_ref, s_ref):
    assert torch.equal(u8(q_gpu) if q_gpu.dtype == torch.float8_e4m3fn else q_gpu.cpu(),
                       u8(q_ref) if q_ref.dtype == torch.float8_e4m3fn else q_ref)
    assert torch.equal(s_gpu.cpu().view(torch.int32), s_ref.view(torch.int32))


def test_hardware_e4m3_conversion_on_every_bf16_value(cuda):
    """Rows holding +-448 have scale 1, so the bytes are the e4m3 conversion of
    every finite bf16 value in [-448, 448]."""
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    v = bits.view(np.float32)
    v = v[np.isfinite(v) & (np.abs(v) <= 448)]
    pad = (-len(v)) % 511
    v = np.concatenate([v, np.zeros(pad, np.float32)]).reshape(-1, 511)
    rows = np.concatenate([np.full((v.shape[0], 1), 448.0, np.float32), v], axis=1)
    x = torch.from_numpy(rows).to(torch.bfloat16)
    q, s = xops.quantize_rows(x.to(cuda), torch.float8_e4m3fn)
    assert (s.cpu() == 1.0).all()
    expected = R.e4m3_encode(rows)
    got = u8(q).numpy()
    bad = np.nonzero(got != expected)
    detail = [(float(rows[i, j]), hex(got[i, j]), hex(expected[i, j])) for i, j in zip(*bad)][:16]
    assert len(bad[0]) == 0, f"{len(bad[0])} mismatches (value, gpu, oracle): {detail}"


def rows_with_edges(M, K, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((M, K), generator=g)
    x[:, K // 7] *= 50
    x[0] = 0
    x[1] = -0.0
    x[2] *= 1e-30
    x[3] *= 1e-36  # amax below the fast-division gate
    x[4, K // 2] = float("inf")
    x[5, K // 3] = float("nan")
    x[6] *= 3e4
    if dtype == torch.float16:
        x[6] /= 3e4  # keep the row finite in f16
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K", [16, 13, 64, 1000, 3072, 5376, 12288, 16384, 20000])
@pytest.mark.parametrize("out", ["fp8", "int8"])
def test_row_quantizers_match_oracle(cuda, dtype, K, out):
    x = rows_with_edges(67, K, dtype, seed=K)
    q, s = xops.quantize_rows(x.to(cuda), torch.float8_e4m3fn if out == "fp8" else torch.int8)
    q_ref, s_ref = R.quantize_rows_c(x, out)
    assert_same_quant(q, s, q_ref, s_ref)


def test_every_bf16_amax_quotient(cuda):
    """For every positive finite bf16 amax, the row's largest quotient amax / RN(amax / 448) may exceed
    448 by an ulp or two; the quantizer does not clamp it and relies on the conversion rounding it to
    448: bytes and scales equal the oracle's (which clamps) on rows [amax, -amax, 0.3 amax, ...]."""
    bits = np.arange(1, 0x7F80, dtype=np.int32) << 16
    a = torch.from_numpy(bits).view(torch.float32).to(torch.bfloat16)
    x = torch.zeros(len(a), 16, dtype=torch.bfloat16)
    x[:, 0], x[:, 1] = a, -a
    x[:, 2:] = (a.float()[:, None] * torch.linspace(-0.99, 0.99, 14)).to(torch.bfloat16)
    q, s = xops.quantize_rows(x.to(cuda), torch.float8_e4m3fn)
    q_ref, s_ref = R.quantize_rows_c(x, "fp8")
    assert_same_quant(q, s, q_ref, s_ref)
    fast = a.float() >= 2.0 ** -100
    assert (u8(q)[fast, 0] == 0x7E).all() and (u8(q)[fast, 1] == 0xFE).all()


def test_row_quantizer_on_strided_rows(cuda):
    x = rows_with_edges(40, 1024, torch.bfloat16).to(cuda)
    view = x[:, 128:128 + 768]  # leading dimension 1024
    q, s = xops.quantize_rows(view, torch.float8_e4m3fn)
    q_ref, s_ref = R.quantize_rows_c(view.cpu().contiguous(), "fp8")
    assert_same_quant(q, s, q_ref, s_ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(32, 128), (997, 5376), (2048, 14336)])
def test_per_tensor_packing_matches_reference_quantizer(cuda, dtype, shape):
    # x_base/tests/test_h3_cuda_precision_ops.py:35-58 (Triton pack == torch quantizer)
    value = torch.randn(shape, dtype=dtype, generator=torch.Generator().manual_seed(1))
    for sample in (value, torch.zeros_like(value)):
        expected, scale = R.quantize_per_tensor(sample)
        actual, actual_scale = quantize_activation(sample.to(cuda))
        assert torch.equal(actual_scale.cpu(), scale)
        assert torch.equal(u8(actual), expected.view(torch.uint8))


def test_abs_peak_propagates_nan_and_inf(cuda):
    x = torch.randn(3, 1000, dtype=torch.bfloat16)
    assert activation_abs_peak(x.to(cuda)).item() == R.abs_peak(x).item()
    x[1, 7] = -float("inf")
    assert activation_abs_peak(x.to(cuda)).item() == float("inf")
    x[2, 999] = float("nan")
    assert torch.isnan(activation_abs_peak(x.to(cuda)))
    tail = torch.randn(1001, dtype=torch.bfloat16)  # numel % 8 != 0
    tail[1000] = 77.0
    assert activation_abs_peak(tail.to(cuda)).item() == 77.0


def test_pack_with_caller_scale(cuda):
    x = torch.randn(4096, dtype=torch.bfloat16) * 10
    scale = torch.tensor(0.0173, dtype=torch.float32)  # quotients exceed 448: clamped
    q = xops.fp8_pack(x.to(cuda), scale.to(cuda))
    ref = (x.float() / scale).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert torch.equal(u8(q), R.canonical_nan_e4m3(ref).view(torch.uint8))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pack_infinity_in_chunk_without_nan(cuda, dtype):
    """+-Inf in 8-value chunks that hold no NaN, at power-of-two scales of the per-tensor
    kernel's form (1.0 from a peak of 448, and the FLT_MIN floor), where the fast division's
    low reciprocal part is 0: +Inf -> 448 (0x7e), -Inf -> -448 (0xfe), as _pack's clamp gives
    (h3_fp8_quant.py:13-14)."""
    x = torch.tensor([float("inf"), 1, 2, 3, 4, 5, 6, -float("inf"),
                      -1, float("inf"), 0.5, -0.0, 7, 8, 9, 10], dtype=dtype)
    for peak in (448.0, 0.0):
        src = torch.zeros(16, dtype=dtype)
        src[3] = peak
        scale = xops.fp8_tensor_scale(src.to(cuda))
        assert scale.item() in (1.0, torch.finfo(torch.float32).tiny)
        q = xops.fp8_pack(x.to(cuda), scale)
        want = R.canonical_nan_e4m3((x.float() / scale.cpu()).clamp(-448, 448).to(torch.float8_e4m3fn))
        assert torch.equal(u8(q), want.view(torch.uint8)), (u8(q).tolist(), want.view(torch.uint8).tolist())
        assert u8(q)[0].item() == 0x7E and u8(q)[7].item() == 0xFE


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pack_every_input_value_at_peak_form_scales(cuda, dtype):
    """fp8_pack's fast division applies to scales of the per-tensor kernel's form,
    max(RN(a / 448), FLT_MIN) for an input value a (what fp8_tensor_scale gives, and a MAX
    all-reduce of such scales): every 16-bit input value (NaN, +-Inf, -0, subnormals) against
    IEEE division + clamp, with peaks above, below and equal to most inputs (values above a
    are clamped), at the FLT_MIN floor, and for caller scales of other forms (IEEE path)."""
    x = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(dtype)
    xd = x.to(cuda)
    peaks = [1.0, 3.0, 448.0, 1344.0, 0.0173, 2.0 ** -14, 1e-30, 0.0]
    peaks.append(3.3e38 if dtype == torch.bfloat16 else 65504.0)
    scales = []
    for a in peaks:
        src = torch.zeros(16, dtype=dtype)
        src[5] = a
        scales.append(xops.fp8_tensor_scale(src.to(cuda)))
    scales.append(torch.tensor(0.0173, dtype=torch.float32, device=cuda))  # not of that form
    scales.append(torch.tensor(1.0 / 3.0, dtype=torch.float32, device=cuda))
    for scale in scales:
        q = xops.fp8_pack(xd, scale)
        ref = R.canonical_nan_e4m3((x.float() / scale.cpu()).clamp(-448, 448).to(torch.float8_e4m3fn))
        got, want = u8(q), ref.view(torch.uint8)
        bad = torch.nonzero(got != want)
        assert bad.numel() == 0, (float(scale), x[bad[:4, 0]].tolist(), got[bad[:4, 0]].tolist(),
                                  want[bad[:4, 0]].tolist())


def test_full_size_requant_k12288(cuda):
    """The FFN-down requant at C3 size (M=15,624, K=12,288): the call moves 576 MB, more than the
    256 MB last-level cache, so the quantizer takes its non-temporal-load form.  Bytes and scales
    of every row against the oracle, FP8 and INT8."""
    g = torch.Generator(device=cuda).manual_seed(12)
    h = torch.randn((workloads.M_5S, 4 * workloads.D_MODEL), generator=g, device=cuda).to(torch.bfloat16)
    h[7] *= 50
    hc = h.cpu()
    for out, dt in (("fp8", torch.float8_e4m3fn), ("int8", torch.int8)):
        q, s = xops.quantize_rows(h, dt)
        q_ref, s_ref = R.quantize_rows_c(hc, out)
        assert_same_quant(q, s, q_ref, s_ref)


def test_full_size_token_quant_c2(cuda):
    """C2 activations (M=15,624, K=3,072, outlier channels) quantized per token."""
    g = workloads.generator(0, cuda)
    x, _ = workloads.activations(workloads.M_5S, workloads.D_MODEL, g, cuda)
    q, s = xops.quantize_rows(x, torch.float8_e4m3fn)
    q_ref, s_ref = R.quantize_rows_c(x.cpu(), "fp8")
    assert_same_quant(q, s, q_ref, s_ref)
    qi, si = xops.quantize_rows(x, torch.int8)
    qi_ref, si_ref = R.quantize_rows_c(x.cpu(), "int8")
    assert_same_quant(qi, si, qi_ref, si_ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_kernel_gelu_within_ulp_of_torch(kernel_gelu, dtype):
    """The GELU-tanh shared by the GEMM epilogue and the GELU requant, on every 16-bit value:
    within 1 ulp of torch's GELU(approximate='tanh') above -3 (absolute 1e-3 at and below -3,
    where torch's float32 tanh form cancels), exact (x/2) for |x| < 2^-60, +0 -> +0, -0 -> -0,
    +inf -> +inf, NaN wherever torch gives NaN."""
    x = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(dtype)
    got = kernel_gelu(x)
    ref = torch.nn.functional.gelu(x.float(), approximate="tanh").to(dtype)
    fin = torch.isfinite(x)
    assert torch.equal(torch.isnan(got[~fin]), torch.isnan(ref[~fin]))
    assert got[x == float("inf")].item() == float("inf")
    body = fin & (x.float() > -3)
    assert R.bf16_ulp_diff(got[body], ref[body]).max() <= 1
    tiny = fin & (x.float().abs() < 2.0 ** -60)
    assert torch.equal(got[tiny].view(torch.int16), (x[tiny].float() * 0.5).to(dtype).view(torch.int16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_kernel_gelu_tail_within_ulp_of_float64(kernel_gelu, dtype):
    """The negative tail (x <= -3), where torch's float32 (and, below about -7, float64)
    0.5x(1 + tanh z) cancels: within 1 ulp of the output dtype of GELU-tanh evaluated in float64
    as x / (1 + exp(-2z)) (the identity 0.5(1 + tanh z) = 1 / (1 + exp(-2z)); that float64 form is
    first held to torch's float64 tanh form, 1e-11 relative, above -3 where the latter does not cancel).
    Exception: the five bf16 inputs in [-10.3125, -10.0625], whose GELU lies below 2^-124 — the
    kernel's float32 exp2 of 2z·log2(e) overflows there and it returns -0."""
    x = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(dtype)
    fin = torch.isfinite(x)
    xd = x[fin].double()
    z = math.sqrt(2.0 / math.pi) * (xd + 0.044715 * xd ** 3)
    exact = xd / (1.0 + torch.exp(-2.0 * z))
    plain = xd > -3
    torch_tanh = torch.nn.functional.gelu(xd[plain], approximate="tanh")
    assert ((exact[plain] - torch_tanh).abs() <= 1e-11 * torch_tanh.abs()).all()
    got = kernel_gelu(x)[fin]
    tail = xd <= -3
    want = exact.to(dtype)
    under = tail & (exact.abs() < 2.0 ** -124) & (want != 0)
    assert R.bf16_ulp_diff(got[tail & ~under], want[tail & ~under]).max() <= 1
    assert torch.equal(got[under].view(torch.int16), torch.full_like(got[under], -0.0).view(torch.int16))
    assert int(under.sum()) == (5 if dtype == torch.bfloat16 else 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K", [13, 1000, 2048, 3072, 4096, 6144, 8192, 12288, 16384, 20000])
@pytest.mark.parametrize("out", ["fp8", "int8"])
def test_gelu_row_quantizers_match_oracle(cuda, kernel_gelu, dtype, K, out):
    """quantize_rows(x, ., ACT_GELU_TANH) quantizes dtype(gelu_tanh(x)): bytes and scales bit-exact
    against the oracle's row quantizer of the GPU's GELU of x, for every launch form (2 to 32
    values per lane, 1 to 4 waves per row, the generic kernel for odd and wide rows) and the edge
    rows (zeros, -0, tiny, inf, NaN, outlier channels)."""
    x = rows_with_edges(67, K, dtype, seed=K + 1)
    q, s = xops.quantize_rows(x.to(cuda), torch.float8_e4m3fn if out == "fp8" else torch.int8, N.ACT_GELU_TANH)
    q_ref, s_ref = R.quantize_rows_c(kernel_gelu(x), out)
    assert_same_quant(q, s, q_ref, s_ref)


@pytest.mark.parametrize("kind", ["fp8", "int8"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gelu_requant_equals_epilogue_then_requant(cuda, kind, dtype):
    """The FFN's two placements of the GELU give the down-projection the same input: quantizing
    the up GEMM's plain output with the GELU requant equals quantizing its GELU-epilogue output,
    bit for bit, on row widths of every launch form (strided views of one [M, 16,400] output)."""
    dt = torch.float8_e4m3fn if kind == "fp8" else torch.int8
    g = workloads.generator(41, cuda)
    M, K, Nf = 200, 256, 16400
    qa, sa = xops.quantize_rows(torch.randn((M, K), generator=g, device=cuda).to(torch.bfloat16), dt)
    qw, sw = xops.quantize_rows((torch.randn((Nf, K), generator=g, device=cuda) * 0.05).to(torch.bfloat16), dt)
    bias = (torch.randn((Nf,), generator=g, device=cuda) * 0.1).to(dtype)
    pre, _ = xops.scaled_mm(qa, qw, sa, sw, bias, dtype, N.ACT_NONE, False)
    post, _ = xops.scaled_mm(qa, qw, sa, sw, bias, dtype, N.ACT_GELU_TANH, False)
    for width in (1000, 2048, 3072, 4096, 6144, 8192, 12288, 16384, 16400, 1003):
        q1, s1 = xops.quantize_rows(pre[:, :width], dt, N.ACT_GELU_TANH)
        q2, s2 = xops.quantize_rows(post[:, :width], dt)
        assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8)), width
        assert torch.equal(s1.view(torch.int32), s2.view(torch.int32)), width


def test_full_size_gelu_requant_k12288(cuda, kernel_gelu):
    """The GELU requant at C3 size (M=15,624, K=12,288; the non-temporal-load form): bytes and
    scales of every row against the oracle's quantizer of the GPU's GELU, FP8 and INT8."""
    g = torch.Generator(device=cuda).manual_seed(13)
    h = torch.randn((workloads.M_5S, 4 * workloads.D_MODEL), generator=g, device=cuda).to(torch.bfloat16)
    h[9] *= 50
    gh = kernel_gelu(h)
    for out, dt in (("fp8", torch.float8_e4m3fn), ("int8", torch.int8)):
        q, s = xops.quantize_rows(h, dt, N.ACT_GELU_TANH)
        q_ref, s_ref = R.quantize_rows_c(gh, out)
        assert_same_quant(q, s, q_ref, s_ref)
