"""The committed golden fixtures (tests/golden/w8a8_path.safetensors, written by
tests/golden/make_golden.py) against the CPU oracle: every stored output is
reproduced bit for bit from the stored inputs, and the hand-checked e4m3
rounding midpoints of the fixture hold independently of the oracle."""
from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file

import oracle.ref as R

GOLDEN = Path(__file__).resolve().parent / "golden" / "w8a8_path.safetensors"


@pytest.fixture(scope="module")
def gold():
    return load_file(str(GOLDEN))


def bits(t):
    return t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t.contiguous().view(torch.uint8)


@pytest.mark.parametrize("tag", ["bf16", "f16"])
def test_row_and_tensor_quantizers_reproduce(gold, tag):
    x = gold[f"rows_{tag}_x"]
    q8, s8 = R.quantize_rows_fp8(x)
    assert torch.equal(q8.view(torch.uint8), gold[f"rows_{tag}_fp8_q"])
    assert torch.equal(bits(s8), bits(gold[f"rows_{tag}_fp8_s"]))
    qi, si = R.quantize_rows_int8(x)
    assert torch.equal(qi, gold[f"rows_{tag}_int8_q"])
    assert torch.equal(bits(si), bits(gold[f"rows_{tag}_int8_s"]))
    qt, st = R.quantize_per_tensor(gold[f"tensor_{tag}_x"])
    assert torch.equal(qt.view(torch.uint8), gold[f"tensor_{tag}_q"])
    assert torch.equal(bits(st.reshape(1)), bits(gold[f"tensor_{tag}_s"]))


def test_midpoint_row_is_ties_to_even(gold):
    # row 5: amax 448 -> scale exactly 1; e4m3 midpoints round to the even code
    x, q = gold["rows_bf16_x"][5], gold["rows_bf16_fp8_q"][5]
    assert gold["rows_bf16_fp8_s"][5].item() == 1.0
    expect = {1.0625: 0x38, 1.1875: 0x3A, 2.125: 0x40, 17.0: 0x58, 272.0: 0x78,
              1.5 * 2.0 ** -9: 0x02, 0.5 * 2.0 ** -9: 0x00, 448.0: 0x7E}
    for v, code in expect.items():
        hits = (x.float() == v).nonzero().flatten()
        assert len(hits) > 0
        assert (q[hits] == code).all(), v
        neg = (x.float() == -v).nonzero().flatten()
        if v != 448.0:
            assert (q[neg] == (code | 0x80)).all(), -v


def test_special_rows(gold):
    q, s = gold["rows_bf16_fp8_q"], gold["rows_bf16_fp8_s"]
    assert (q[0] == 0).all() and s[0].item() == torch.finfo(torch.float32).tiny   # zero row
    assert torch.isnan(s[1]) and (q[1] == 0x7F).all()                             # NaN row
    assert torch.isinf(s[2]) and q[2, 7] == 0x7F and (q[2, :7] == 0x80).all()     # +inf: scale inf, x/inf = -0
    assert (q[3] == 0x80).sum() >= q.shape[1] - 1                                  # -0 keeps its sign


def test_front_end_reproduces(gold):
    x, sc, sh, idx, w = gold["fe_x"], gold["fe_scale"], gold["fe_shift"], gold["fe_idx"], gold["fe_w"]
    for norm, out, weight, eps in (("layer", "fp8", None, 1e-6), ("rms", "int8", w, 1e-5), ("rms", "fp8", w, 1e-5)):
        q, s, m = R.norm_affine_quant(x, weight, sc, sh, idx, eps, norm, out)
        key = f"fe_{norm}_{out}"
        assert torch.equal(bits(q), gold[key + "_q"].view(torch.uint8))
        assert torch.equal(bits(s), bits(gold[key + "_s"]))
        assert torch.equal(bits(m), bits(gold[key + "_m"]))


def test_gemm_reproduces(gold):
    b = gold["mm_b"]
    qa, qw = gold["mm_fp8_qa"].view(torch.float8_e4m3fn), gold["mm_fp8_qw"].view(torch.float8_e4m3fn)
    sa, sw = gold["mm_fp8_sa"], gold["mm_fp8_sw"]
    assert torch.equal(R.fp8_accumulate_exact(qa, qw), gold["mm_fp8_acc"])
    assert torch.equal(bits(R.w8a8_linear_fp8(qa, sa, qw, sw, b)), bits(gold["mm_fp8_out"]))
    assert torch.equal(bits(R.w8a8_linear_fp8(qa, sa, qw, sw, b, torch.bfloat16, "gelu_tanh")),
                       bits(gold["mm_fp8_out_gelu"]))
    qa, qw, sa, sw = gold["mm_int8_qa"], gold["mm_int8_qw"], gold["mm_int8_sa"], gold["mm_int8_sw"]
    assert torch.equal(R.int8_accumulate_exact(qa, qw).to(torch.int32), gold["mm_int8_acc"])
    assert torch.equal(bits(R.w8a8_linear_int8(qa, sa, qw, sw, b)), bits(gold["mm_int8_out"]))
