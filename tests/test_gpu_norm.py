"""GPU parity of the fused norm + AdaLN modulate + quantize kernel.

Contract (the reductions of the norm are order-dependent in float32):
  * pre-quant bf16 rows m >= 99.9% bit-identical to the oracle (float64
    statistics, eager bf16 modulation) and >= 99.99% within one bf16 ulp;
    elsewhere the difference is what one bf16 ulp of the normalised value n
    can become after the modulation: it moves the exact n*f by
    |f| ulp(n) <= 2^-7 |n*f|, rounding bf16(n*f) can add one more ulp, and
    rounding m one ulp of m, so
    |dm| <= 2^-6 |n*f| + 2^-7 |m| (bf16(n*f) + shift may cancel, so ulps of
    m alone do not bound it);
  * quantized bytes and scales bit-exact given the kernel's own pre-quant rows.
"""
import pytest
import torch

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd import _native as N
from xgen_amd import workloads
from xgen_amd.operator.nq2 import norm_affine_quant

pytestmark = pytest.mark.gpu
xops = torch.ops.xgen_amd


def inputs(B, S, H, T, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((B, S, H), generator=g)
    x[..., 3] *= 50
    x = x.to(torch.bfloat16)
    shift = (torch.randn((T, H), generator=g) * 0.1).to(torch.bfloat16)
    scale = (torch.randn((T, H), generator=g) * 0.1).to(torch.bfloat16)
    idx = torch.randint(T, (S,), generator=g)
    return x.to(dev), scale.to(dev), shift.to(dev), idx.to(dev)


def check(x, weight, scale, shift, idx, eps, norm, out, q, s, m):
    w = None if weight is None else weight.cpu()
    qr, sr, mr = R.norm_affine_quant(x.cpu(), w, scale.cpu(), shift.cpu(), idx.cpu(), eps, norm, out)
    B, S, H = x.shape
    n = (R.layer_norm_f64 if norm == "layer" else R.rms_norm_f64)(x.cpu().reshape(B * S, H), eps, w)
    g = idx.cpu().long().repeat(B)
    nf = n * (1.0 + scale.cpu()[g])  # eager bf16: bf16(n * bf16(1 + scale))
    ulps = R.bf16_ulp_diff(m.cpu(), mr)
    assert (ulps == 0).float().mean() >= 0.999
    assert (ulps <= 1).float().mean() >= 0.9999
    bound = 2.0 ** -6 * nf.double().abs() + 2.0 ** -7 * mr.double().abs() + 1e-30
    assert ((m.cpu().double() - mr.double()).abs() <= bound).all()
    q2, s2 = (R.quantize_rows_fp8 if out == "fp8" else R.quantize_rows_int8)(m.cpu())
    if out == "fp8":
        assert torch.equal(q.cpu().view(torch.uint8), q2.view(torch.uint8))
    else:
        assert torch.equal(q.cpu(), q2)
    assert torch.equal(s.cpu().view(torch.int32), s2.view(torch.int32))
    same_rows = (ulps == 0).all(dim=-1)
    if out == "fp8":
        assert torch.equal(q.cpu().view(torch.uint8)[same_rows], qr.view(torch.uint8)[same_rows])
    assert torch.equal(s.cpu()[same_rows], sr[same_rows])


@pytest.mark.parametrize("norm", ["layer", "rms"])
@pytest.mark.parametrize("out", ["fp8", "int8"])
@pytest.mark.parametrize("B,S,H", [(2, 37, 128), (1, 300, 3072), (3, 20, 1000), (1, 64, 5376), (1, 33, 8192)])
def test_fused_front_end_matches_oracle(cuda, norm, out, B, S, H):
    x, scale, shift, idx = inputs(B, S, H, 20, seed=H + S, dev=cuda)
    q, s, m = xops.norm_affine_quant(x, None, scale, shift, idx, 1e-6, N.NORM_LAYER if norm == "layer" else N.NORM_RMS,
                                     torch.float8_e4m3fn if out == "fp8" else torch.int8, True)
    check(x, None, scale, shift, idx, 1e-6, norm, out, q, s, m)


@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_rms_with_weight_reference_signature(cuda, wdtype):
    # the reference op's surface: norm_affine_quant(x, weight, scale, shift, indices, eps=1e-5) -> int8
    x, scale, shift, idx = inputs(2, 17, 512, 3, seed=9, dev=cuda)
    w = (torch.randn(512, generator=torch.Generator().manual_seed(4)) * 0.5 + 1).to(wdtype).to(cuda)
    q, s = norm_affine_quant(x, w, scale, shift, idx)
    assert q.dtype == torch.int8 and q.shape == (34, 512) and s.shape == (34,)
    q, s, m = norm_affine_quant(x, w, scale, shift, idx, return_normed=True)
    check(x, w, scale, shift, idx, 1e-5, "rms", "int8", q, s, m)


def test_strided_input_and_tables(cuda):
    big, scale, shift, idx = inputs(2, 24, 1024, 6, seed=3, dev=cuda)
    x = big[:, :, 256:256 + 512]           # row stride 1024
    tab = torch.cat([scale, shift], dim=1)  # tables with row stride 2048
    sc, sh = tab[:, 256:768], tab[:, 1024 + 256:1024 + 768]
    q, s, m = xops.norm_affine_quant(x, None, sc, sh, idx, 1e-6, N.NORM_LAYER, torch.float8_e4m3fn, True)
    check(x, None, sc, sh, idx, 1e-6, "layer", "fp8", q, s, m)


def test_out_of_range_index_poisons_only_its_row(cuda):
    x, scale, shift, idx = inputs(1, 8, 256, 4, seed=1, dev=cuda)
    idx = idx.clone()
    idx[5] = 99
    q, s, _ = xops.norm_affine_quant(x, None, scale, shift, idx, 1e-6, N.NORM_LAYER, torch.float8_e4m3fn, True)
    assert torch.isnan(s[5]) and (q[5].view(torch.uint8) == 0x7F).all()
    assert torch.isfinite(s[torch.arange(8, device=cuda) != 5]).all()


@pytest.mark.parametrize("H", [1000, 3072, 5376, 8192])
def test_offset_and_constant_rows(cuda, H):
    """Rows with a large common offset (the one-pass variance E[x^2] - mean^2 would cancel) take
    the two-pass variance, next to ordinary rows in the same workgroup (one, two and four waves
    per row); constant rows normalise to exactly zero, as the eager (x - mean) * rstd does, so
    their modulated row is the shift row; every row's result is independent of its neighbours."""
    g = torch.Generator().manual_seed(H)
    S = 24
    x = torch.randn(1, S, H, generator=g)
    x[0, 1::3] += 6.0  # mean^2 ~ 36 of E[x^2] ~ 37: two-pass
    const_rows, consts = list(range(2, S, 6)), [1.5, -3.0, 100.0, 0.0]
    for r, c in zip(const_rows, consts):
        x[0, r] = c
    x = x.to(torch.bfloat16).to(cuda)
    shift = (torch.randn((5, H), generator=g) * 0.1).to(torch.bfloat16).to(cuda)
    scale = (torch.randn((5, H), generator=g) * 0.1).to(torch.bfloat16).to(cuda)
    idx = torch.randint(5, (S,), generator=g).to(cuda)
    q, s, m = xops.norm_affine_quant(x, None, scale, shift, idx, 1e-6, N.NORM_LAYER, torch.float8_e4m3fn, True)
    check(x, None, scale, shift, idx, 1e-6, "layer", "fp8", q, s, m)
    for r in const_rows:
        assert torch.equal(m[r].view(torch.int16), shift[idx[r]].view(torch.int16))
    for r in (0, 1, 2, 7):
        q1, s1, m1 = xops.norm_affine_quant(x[:, r:r + 1], None, scale, shift, idx[r:r + 1], 1e-6, N.NORM_LAYER,
                                            torch.float8_e4m3fn, True)
        assert torch.equal(m1[0].view(torch.int16), m[r].view(torch.int16))
        assert torch.equal(q1[0].view(torch.uint8), q[r].view(torch.uint8)) and torch.equal(s1[0], s[r])


@pytest.mark.parametrize("M", [workloads.M_5S, workloads.M_10S], ids=["c2_share_m15624", "c5_share_m31248"])
def test_full_size_front_end(cuda, M):
    """LayerNorm(eps 1e-6) + 20-row AdaLN table + per-token FP8 at one SP8 rank's share of the 5 s
    clip (M=15,624) and of the 10 s clip (C5, M=31,248), d=3,072."""
    H = workloads.D_MODEL
    g = workloads.generator(0, cuda)
    x, _ = workloads.activations(M, H, g, cuda)
    shift, scale = workloads.adaln_tables(20, H, g, cuda)
    idx = torch.randint(20, (M,), generator=g, device=cuda)
    q, s, m = xops.norm_affine_quant(x[None], None, scale, shift, idx, 1e-6, N.NORM_LAYER, torch.float8_e4m3fn, True)
    check(x[None], None, scale, shift, idx, 1e-6, "layer", "fp8", q, s, m)


def test_adaln_one_plus_matches_eager_bf16(cuda):
    """bf16(1 + scale) == the eager bf16 `1.0 + scale` (torch CPU), special values included."""
    from xgen_amd.operator.nq2 import adaln_one_plus
    g = torch.Generator().manual_seed(4)
    t = (torch.randn(37, 520, generator=g) * torch.logspace(-6, 3, 520)).to(torch.bfloat16)
    t[0, :6] = torch.tensor([float("nan"), float("inf"), float("-inf"), -1.0, -0.0, 2.0 ** -133])
    big = torch.zeros(37, 1024, dtype=torch.bfloat16)
    big[:, :520] = t
    got = adaln_one_plus(big.to(cuda)[:, :520]).cpu()
    ref = 1.0 + t
    assert ref.dtype == torch.bfloat16
    nan = torch.isnan(ref)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got.view(torch.int16)[~nan], ref.view(torch.int16)[~nan])


@pytest.mark.parametrize("norm", ["layer", "rms"])
@pytest.mark.parametrize("out", ["fp8", "int8"])
@pytest.mark.parametrize("H", [1000, 1024, 3072, 5376, 8192])
@pytest.mark.parametrize("wdtype", [None, torch.bfloat16, torch.float32])
def test_prepared_one_plus_scale_is_bit_identical(cuda, norm, out, H, wdtype):
    """scale_is_one_plus=True with bf16(1 + scale) gives the same bytes, scales and rows as the plain
    call, with and without a norm weight; an index outside the table poisons its row (NaN scale)
    in both forms."""
    from xgen_amd.operator.nq2 import adaln_one_plus
    x, scale, shift, idx = inputs(2, 41, H, 7, seed=H, dev=cuda)
    idx = idx.clone()
    idx[5] = 7  # outside the table
    w = None if wdtype is None else (torch.randn(H, generator=torch.Generator().manual_seed(2)) * 0.3 + 1).to(
        wdtype).to(cuda)
    dt = torch.float8_e4m3fn if out == "fp8" else torch.int8
    eps = 1e-6 if norm == "layer" else 1e-5
    q0, s0, m0 = norm_affine_quant(x, w, scale, shift, idx, eps=eps, norm=norm, out_dtype=dt, return_normed=True)
    f = adaln_one_plus(scale)
    q1, s1, m1 = norm_affine_quant(x, w, f, shift, idx, eps=eps, norm=norm, out_dtype=dt, return_normed=True,
                                   scale_is_one_plus=True)
    assert torch.equal(q0.view(torch.uint8), q1.view(torch.uint8))
    assert torch.equal(s0.view(torch.int32), s1.view(torch.int32))
    assert torch.equal(m0.view(torch.int16), m1.view(torch.int16))
    assert torch.isnan(s0[5]) and torch.isnan(s0[41 + 5]) and not torch.isnan(s0[4])


@pytest.mark.parametrize("H", [8, 1032, 2048, 2056, 3080, 4096, 4104, 6144, 6152])
@pytest.mark.parametrize("wdtype", [None, torch.float32])
def test_every_width_form(cuda, H, wdtype):
    """Each launch form of the width dispatch at and just past its boundaries (one wave per row up
    to 3,072 with 2 / 4 / 6 chunks per lane, two waves per row to 4,096, four beyond), LayerNorm and
    RMSNorm, with and without a norm weight, against the oracle."""
    x, scale, shift, idx = inputs(2, 11, H, 4, seed=H, dev=cuda)
    w = None if wdtype is None else (torch.randn(H, generator=torch.Generator().manual_seed(H)) * 0.3 + 1).to(
        wdtype).to(cuda)
    for norm, eps in (("layer", 1e-6), ("rms", 1e-5)):
        q, s, m = xops.norm_affine_quant(x, w, scale, shift, idx, eps, N.NORM_LAYER if norm == "layer" else N.NORM_RMS,
                                         torch.float8_e4m3fn, True)
        check(x, w, scale, shift, idx, eps, norm, "fp8", q, s, m)
