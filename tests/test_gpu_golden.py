"""The HIP kernels against the committed golden fixtures (tests/golden/
w8a8_path.safetensors): quantized bytes and scales bit-exact, INT8
accumulators bit-exact, FP8 accumulators within the MFMA accumulation bound,
fused front end within the pre-quant contract, bf16 GEMM outputs within
rel-L2 1e-3.  No oracle code runs here.  The fixture holds the oracle's
outputs frozen at the time it was written (tests/golden/make_golden.py;
tests/test_golden_oracle.py checks the oracle still reproduces them): this is a
regression check of the kernels against stored vectors, while parity with the
reference rests on the oracle's own pins (tests/test_oracle_*.py)."""
from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file

import xgen_amd  # noqa: F401
from xgen_amd import _native as N

pytestmark = pytest.mark.gpu
xops = torch.ops.xgen_amd
GOLDEN = Path(__file__).resolve().parent / "golden" / "w8a8_path.safetensors"
FP8 = torch.float8_e4m3fn


@pytest.fixture(scope="module")
def gold():
    return load_file(str(GOLDEN))


def u8(t):
    return t.detach().cpu().contiguous().view(torch.uint8)


def rel_l2(a, b):
    a, b = a.detach().cpu().double(), b.detach().cpu().double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("tag", ["bf16", "f16"])
def test_quantizers(cuda, gold, tag):
    x = gold[f"rows_{tag}_x"].to(cuda)
    q, s = xops.quantize_rows(x, FP8)
    assert torch.equal(u8(q), gold[f"rows_{tag}_fp8_q"])
    assert torch.equal(u8(s), u8(gold[f"rows_{tag}_fp8_s"]))
    q, s = xops.quantize_rows(x, torch.int8)
    assert torch.equal(q.cpu(), gold[f"rows_{tag}_int8_q"])
    assert torch.equal(u8(s), u8(gold[f"rows_{tag}_int8_s"]))
    xt = gold[f"tensor_{tag}_x"].to(cuda)
    st = xops.fp8_tensor_scale(xt)
    qt = xops.fp8_pack(xt, st)
    assert torch.equal(u8(qt), gold[f"tensor_{tag}_q"])
    assert torch.equal(u8(st.reshape(1)), u8(gold[f"tensor_{tag}_s"]))


def test_front_end(cuda, gold):
    x, sc, sh, idx, w = (gold[k].to(cuda) for k in ("fe_x", "fe_scale", "fe_shift", "fe_idx", "fe_w"))
    for norm, out, weight, eps in (("layer", "fp8", None, 1e-6), ("rms", "int8", w, 1e-5), ("rms", "fp8", w, 1e-5)):
        key = f"fe_{norm}_{out}"
        q, s, m = xops.norm_affine_quant(x, weight, sc, sh, idx, eps, N.NORM_LAYER if norm == "layer" else N.NORM_RMS,
                                         FP8 if out == "fp8" else torch.int8, True)
        m_ref = gold[key + "_m"]
        same = (u8(m).view(torch.int16) == u8(m_ref).view(torch.int16))
        assert same.float().mean() >= 0.999
        rows_same = same.reshape(m_ref.shape[0], -1).all(dim=1)
        # bit-exact bytes and scales wherever the pre-quant row is bit-identical
        assert torch.equal(u8(q)[rows_same], u8(gold[key + "_q"])[rows_same])
        assert torch.equal(u8(s).view(torch.int32)[rows_same], u8(gold[key + "_s"]).view(torch.int32)[rows_same])
        assert rows_same.float().mean() >= 0.5


@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_gemm(cuda, gold, kind):
    b = gold["mm_b"].to(cuda)
    if kind == "fp8":
        qa, qw = gold["mm_fp8_qa"].view(FP8).to(cuda), gold["mm_fp8_qw"].view(FP8).to(cuda)
        sa, sw = gold["mm_fp8_sa"].to(cuda), gold["mm_fp8_sw"].to(cuda)
    else:
        qa, qw = gold["mm_int8_qa"].to(cuda), gold["mm_int8_qw"].to(cuda)
        sa, sw = gold["mm_int8_sa"].to(cuda), gold["mm_int8_sw"].to(cuda)
    out, acc = xops.scaled_mm(qa, qw, sa, sw, b, torch.bfloat16, N.ACT_NONE, True)
    if kind == "fp8":
        exact = gold["mm_fp8_acc"]
        mag = qa.cpu().double().abs() @ qw.cpu().double().abs().T
        assert ((acc.cpu().double() - exact).abs() <= 2.0 ** -11 * mag + 1e-30).all()
    else:
        assert torch.equal(acc.cpu(), gold["mm_int8_acc"])
    assert rel_l2(out, gold[f"mm_{kind}_out"]) <= 1e-3
    if kind == "fp8":
        gelu, _ = xops.scaled_mm(qa, qw, sa, sw, b, torch.bfloat16, N.ACT_GELU_TANH, False)
        assert rel_l2(gelu, gold["mm_fp8_out_gelu"]) <= 1e-3
