"""Pins the oracle's front end (LayerNorm/RMSNorm, AdaLN modulation, fused
composite), GELU-tanh and GEMM accumulators."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.ref as R


def test_layer_norm_f64_matches_torch_within_one_ulp():
    torch.manual_seed(0)
    x = torch.randn(256, 3072, dtype=torch.bfloat16)
    x[:, :3] = (x[:, :3].float() * 50).to(torch.bfloat16)
    ours = R.layer_norm_f64(x, 1e-6)
    ref = F.layer_norm(x, (3072,), eps=1e-6)  # nn.LayerNorm(3072, elementwise_affine=False, eps=1e-6)
    ulps = R.bf16_ulp_diff(ours, ref)
    assert ulps.max() <= 1
    assert (ulps == 0).float().mean() >= 0.999


def test_layer_norm_f64_invariants():
    torch.manual_seed(1)
    x = torch.randn(64, 1024, dtype=torch.bfloat16) * 7 + 3
    v = x.double()
    n = (v - v.mean(-1, keepdim=True)) / torch.sqrt(v.var(-1, unbiased=False, keepdim=True) + 1e-6)
    assert torch.allclose(n.mean(-1), torch.zeros(64, dtype=torch.float64), atol=1e-12)
    assert torch.allclose((n * n).mean(-1), torch.ones(64, dtype=torch.float64), atol=1e-5)
    assert torch.equal(R.layer_norm_f64(x, 1e-6), n.float().to(torch.bfloat16))


@pytest.mark.parametrize("H", [512, 3072, 5376])
@pytest.mark.parametrize("eps", [1e-5, 1e-6])
@pytest.mark.parametrize("wdtype", [None, torch.bfloat16, torch.float32])
def test_rms_norm_f64_matches_torch_rms_norm(H, eps, wdtype):
    """rms_norm_f64 (the f2bc order x * rsqrt(mean(x^2) + eps) * w) against torch's own RMSNorm:
    bit for bit when torch runs in float64 too, and within 1 bf16 ulp (>= 99.9% equal) of
    torch's bf16 F.rms_norm.  Rows scaled by 2^-12 make eps dominate mean(x^2) (a dropped or
    misplaced eps fails), one row of zeros normalises to zeros.  (A float32 weight is compared
    in float64 only: torch's bf16 path takes a bf16 weight.)"""
    g = torch.Generator().manual_seed(H + int(eps * 1e7))
    x = torch.randn((48, H), generator=g)
    x[:8] *= 2.0 ** -12
    x[8] = 0
    x[9:12] *= 40
    x = x.to(torch.bfloat16)
    w = None if wdtype is None else (1 + 0.1 * torch.randn(H, generator=g)).to(wdtype)
    ours = R.rms_norm_f64(x, eps, w)
    ref64 = F.rms_norm(x.double(), (H,), None if w is None else w.double(), eps).float().to(torch.bfloat16)
    assert torch.equal(ours.view(torch.int16), ref64.view(torch.int16))
    if wdtype != torch.float32:  # torch's bf16 module form (nn.RMSNorm in bf16: bf16 weight)
        ref16 = F.rms_norm(x, (H,), w, eps)
        ulps = R.bf16_ulp_diff(ours, ref16)
        assert ulps.max() <= 1 and (ulps == 0).float().mean() >= 0.999
    # eps matters on the small rows: without it they would normalise to unit RMS
    no_eps = (x[:8].double() / torch.sqrt((x[:8].double() ** 2).mean(-1, keepdim=True)))
    assert (ours[:8].double().pow(2).mean(-1) < 0.5 * no_eps.pow(2).mean(-1)).all()


def test_rms_norm_f64_invariants():
    """Unit mean square without weight (eps negligible); invariant to scaling the row by 2^k."""
    torch.manual_seed(2)
    x = (torch.randn(32, 1024) * 3).to(torch.bfloat16)
    n = R.rms_norm_f64(x, 1e-6).double()
    assert torch.allclose(n.pow(2).mean(-1), torch.ones(32, dtype=torch.float64), atol=1e-2)
    assert torch.equal(R.rms_norm_f64(x * 8, 1e-12), R.rms_norm_f64(x, 1e-12))


def test_fp8_linear_epilogue_equals_torch_scaled_mm():
    """w8a8_linear_fp8 with per-tensor scales == CPU torch._scaled_mm(a, w.T, scale_a, scale_b,
    bias, out_dtype=bf16) bit for bit (h3_fp8.py:63-66).  Operands are e4m3 codes of exponents
    -3..3 with K = 64, so every partial sum is exact in float32 whatever the summation order: the
    comparison isolates the dequant-and-bias epilogue.  Scales are not powers of two."""
    g = torch.Generator().manual_seed(11)
    for M, N, out_dtype in ((64, 256, torch.bfloat16), (37, 80, torch.bfloat16), (16, 48, torch.float16)):
        def codes(rows):
            mag = torch.randint(0x20, 0x58, (rows, 64), generator=g, dtype=torch.int32)  # exponent field 4..10
            sign = torch.randint(0, 2, (rows, 64), generator=g, dtype=torch.int32) << 7
            return (mag | sign).to(torch.uint8).view(torch.float8_e4m3fn)
        qa, qw = codes(M), codes(N)
        sa = torch.rand((), generator=g) * 0.01 + 1e-3
        sw = torch.rand((), generator=g) * 0.01 + 1e-3
        for bias in (None, (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16)):
            ref = torch._scaled_mm(qa, qw.t(), scale_a=sa, scale_b=sw, bias=bias, out_dtype=out_dtype)
            ours = R.w8a8_linear_fp8(qa, sa, qw, sw, bias, out_dtype)
            assert torch.equal(ours, ref)


def test_fp8_linear_matches_torch_scaled_mm_general_operands():
    """General row-quantized operands (K = 3,072): CPU _scaled_mm sums in float32 in its own
    order, the oracle exactly; outputs equal on >= 99.99% of elements, all within 1 ulp."""
    g = torch.Generator().manual_seed(12)
    x = torch.randn((64, 3072), generator=g).to(torch.bfloat16)
    w = (torch.randn((512, 3072), generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(512, generator=g) * 0.01).to(torch.bfloat16)
    qa, sa = R.quantize_per_tensor(x)
    qw, sw = R.quantize_per_tensor(w)
    ref = torch._scaled_mm(qa, qw.t(), scale_a=sa, scale_b=sw, bias=b, out_dtype=torch.bfloat16)
    ulps = R.bf16_ulp_diff(R.w8a8_linear_fp8(qa, sa, qw, sw, b), ref)
    assert ulps.max() <= 1 and (ulps == 0).float().mean() >= 0.9999


def test_modulate_eager_equals_explicit_rounding():
    # the reference's own bitwise check of its fused modulation against eager bf16
    # (x_base/tests/test_h3_indexed_affine.py:7-23)
    g = torch.Generator().manual_seed(42)
    x = torch.randn((2, 37, 128), generator=g, dtype=torch.bfloat16)
    tables = torch.randn((7, 6 * 128), generator=g, dtype=torch.bfloat16)
    shift, scale, *_ = tables.chunk(6, dim=-1)
    idx = torch.randint(7, (37,), generator=g)
    eager = R.modulate(x, scale.index_select(0, idx), shift.index_select(0, idx))
    explicit = R.modulate_np(R.bf16_to_np(x), R.bf16_to_np(scale.index_select(0, idx)),
                             R.bf16_to_np(shift.index_select(0, idx)))
    assert np.array_equal(eager.float().numpy().view(np.uint32), explicit.view(np.uint32))


def test_round_bf16_np_matches_torch():
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.standard_normal(1 << 16).astype(np.float32) * 100,
                        (np.arange(1 << 16, dtype=np.uint32) << 16 | 0x8000).view(np.float32)])
    ours = R.round_bf16_np(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    fin = np.isfinite(ref)
    assert np.array_equal(ours[fin].view(np.uint32), ref[fin].view(np.uint32))


@pytest.mark.parametrize("norm,out", [("layer", "fp8"), ("rms", "int8")])
def test_norm_affine_quant_composite(norm, out):
    g = torch.Generator().manual_seed(5)
    B, S, H, T = 2, 13, 256, 5
    x = torch.randn((B, S, H), generator=g).to(torch.bfloat16)
    shift = (torch.randn((T, H), generator=g) * 0.1).to(torch.bfloat16)
    scale = (torch.randn((T, H), generator=g) * 0.1).to(torch.bfloat16)
    idx = torch.randint(T, (S,), generator=g)
    q, s, m = R.norm_affine_quant(x, None, scale, shift, idx, 1e-6, norm, out)
    assert q.shape == (B * S, H) and s.shape == (B * S,) and m.shape == (B * S, H)
    # row r = b*S + s uses table row idx[s]
    r = S + 4
    n = (R.layer_norm_f64 if norm == "layer" else R.rms_norm_f64)(x[1, 4:5], 1e-6)
    expect_m = R.modulate(n, scale[idx[4]][None], shift[idx[4]][None])
    assert torch.equal(m[r:r + 1], expect_m)
    qq, ss = (R.quantize_rows_fp8 if out == "fp8" else R.quantize_rows_int8)(m)
    assert torch.equal(q.view(torch.uint8) if out == "fp8" else q, qq.view(torch.uint8) if out == "fp8" else qq)
    assert torch.equal(s, ss)


def test_gelu_tanh_against_closed_form():
    v = torch.linspace(-12, 12, 20001).to(torch.bfloat16)
    ours = R.gelu_tanh_bf16(v)
    x = v.double()
    exact = 0.5 * x * (1 + torch.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
    # float32 evaluation of 1 + tanh(z) cancels for negative x (to 0 below ~-9):
    # ulp comparison where it does not, absolute bound in the tail
    body = x > -3
    assert R.bf16_ulp_diff(ours[body], exact[body].float().to(torch.bfloat16)).max() <= 1
    assert (ours[~body].double() - exact[~body]).abs().max() < 1e-5


def test_fp8_accumulators_exact_against_integer_brute_force():
    torch.manual_seed(7)
    a = (torch.randn(17, 96) * 30).to(torch.float8_e4m3fn)
    w = (torch.randn(23, 96) * 30).to(torch.float8_e4m3fn)
    acc = R.fp8_accumulate_exact(a, w)
    ai = (a.double() * 512).long()   # every e4m3 value is a multiple of 2^-9
    wi = (w.double() * 512).long()
    exact = (ai[:, None, :] * wi[None, :, :]).sum(-1)
    assert torch.equal((acc * (1 << 18)).long(), exact)


def test_int8_accumulators_exact():
    torch.manual_seed(8)
    a = torch.randint(-127, 128, (32, 1024), dtype=torch.int8)
    w = torch.randint(-127, 128, (48, 1024), dtype=torch.int8)
    acc = R.int8_accumulate_exact(a, w)
    brute = (a.long()[:, None, :] * w.long()[None, :, :]).sum(-1)
    assert torch.equal(acc, brute)
    assert torch.equal(acc.int(), torch._int_mm(a, w.T.contiguous()))


def test_fp8_linear_close_to_bf16_linear():
    # the reference's FP8-vs-BF16 statistic (x_base/tests/test_h3_cuda_precision_ops.py:19-32)
    torch.manual_seed(42)
    weight = torch.randn(256, 128, dtype=torch.bfloat16)
    bias = torch.randn(256, dtype=torch.bfloat16)
    x = torch.randn(38, 128, dtype=torch.bfloat16)
    qw, sw = R.quantize_per_tensor(weight)
    qa, sa = R.quantize_per_tensor(x)
    y = R.w8a8_linear_fp8(qa, sa, qw, sw, bias)
    ref = F.linear(x.float(), weight.float(), bias.float())
    rel = (y.float() - ref).square().mean().sqrt() / ref.square().mean().sqrt()
    assert rel < 0.08
    # per-token x per-channel scaling is at least as close
    qa2, sa2 = R.quantize_rows_fp8(x)
    qw2, sw2 = R.quantize_rows_fp8(weight)
    y2 = R.w8a8_linear_fp8(qa2, sa2, qw2, sw2, bias)
    assert R.rel_l2(y2, ref) <= R.rel_l2(y, ref) + 1e-3


def test_cpu_fake_quant_path_equals_oracle_linear():
    torch.manual_seed(9)
    x = torch.randn(64, 256, dtype=torch.bfloat16)
    w = (torch.randn(128, 256) * 0.02).to(torch.bfloat16)
    b = (torch.randn(128) * 0.01).to(torch.bfloat16)
    qw, sw = R.quantize_rows_fp8(w)
    qa, sa = R.quantize_rows_fp8(x)
    a = R.cpu_fake_quant_linear_fp8(x, qw, sw, b)
    ref = R.w8a8_linear_fp8(qa, sa, qw, sw, b)
    assert R.rel_l2(a, ref) < 1e-2 and R.cosine(a, ref) > 0.9999


def test_gate_residual_eager_equals_explicit_rounding():
    """The reference's bitwise check of its gated residual against eager bf16
    (x_base/tests/test_h3_indexed_affine.py:21-22): multiply, round, add, round."""
    g = torch.Generator().manual_seed(42)
    x = torch.randn((2, 37, 128), generator=g, dtype=torch.bfloat16)
    residual = torch.randn(x.shape, generator=g, dtype=torch.bfloat16)
    tables = torch.randn((7, 6 * 128), generator=g, dtype=torch.bfloat16)
    _, _, gate, *_ = tables.chunk(6, dim=-1)
    idx = torch.randint(7, (37,), generator=g)
    eager = R.gate_residual(residual, x, gate, idx)
    explicit = R.gate_residual_np(R.bf16_to_np(residual), R.bf16_to_np(x), R.bf16_to_np(gate.index_select(0, idx))[None])
    assert np.array_equal(eager.float().numpy().view(np.uint32), explicit.view(np.uint32))
    # and it is not the fused multiply-add: some elements differ from a single rounding
    fused = (residual.float() + gate.index_select(0, idx).float()[None] * x.float()).to(torch.bfloat16)
    assert not torch.equal(fused, eager)


def test_swiglu_oracle_layouts_scale_modes_and_closed_form():
    g = torch.Generator().manual_seed(8)
    F = 64
    u = (torch.randn((2, 9, 2 * F), generator=g) * 3).to(torch.bfloat16)
    q1, s1, v1 = R.swiglu_quant(u, gate_first=False, out="int8", scale_mode=1)
    # layout: [hidden | gate] vs [gate | hidden] are the same op on swapped halves
    swapped = torch.cat([u[..., F:], u[..., :F]], dim=-1)
    _, _, v2 = R.swiglu_quant(swapped, gate_first=True)
    assert torch.equal(v1, v2)
    # a = bf16(silu(gate)) against the float64 closed form; v = bf16(hidden * a)
    hidden, gate = u[..., :F].double(), u[..., F:].double()
    a64 = (gate / (1 + torch.exp(-gate))).float().to(torch.bfloat16).double()
    v64 = (hidden * a64).float().to(torch.bfloat16)
    assert (v64.reshape(-1, F) == v1).float().mean() >= 0.999
    # eager torch (the reference's fallback `hidden * F.silu(gate)` in bf16)
    eager = (u[..., :F] * torch.nn.functional.silu(u[..., F:])).reshape(-1, F)
    assert (eager == v1).float().mean() >= 0.999
    # scale modes: amax * fl(1/127) vs 1 / fl(127 / amax), same bytes
    q0, s0, _ = R.swiglu_quant(u, scale_mode=0)
    assert torch.equal(q0, q1)
    amax = v1.float().abs().amax(dim=-1)
    assert torch.equal(s1, amax * (torch.tensor(1.0) / 127.0))
    assert torch.equal(s0, torch.tensor(1.0) / (torch.tensor(127.0) / amax))
    # FP8 form: the row quantizer of v
    qf, sf, _ = R.swiglu_quant(u, out="fp8")
    qr, sr = R.quantize_rows_fp8(v1)
    assert torch.equal(qf.view(torch.uint8), qr.view(torch.uint8)) and torch.equal(sf, sr)
