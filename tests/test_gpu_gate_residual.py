"""GPU parity of the gated residual: the standalone op bit-exact against the
oracle (the reference's eager-bf16 expression), and the GEMM with the gated
residual in its epilogue bit-exact against GEMM-then-op (same arithmetic),
within the GEMM contract against the oracle composite."""
import pytest
import torch

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd import _native as N
from xgen_amd import workloads
from xgen_amd.operator.gate_residual import gate_residual
from xgen_amd.operator.h3_fp8 import H3FP8Linear
from xgen_amd.operator.matmul import WeightQuantLinearModule

pytestmark = pytest.mark.gpu
xops = torch.ops.xgen_amd


def inputs(B, S, H, T, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((B, S, H), generator=g, dtype=torch.bfloat16)
    residual = torch.randn((B, S, H), generator=g, dtype=torch.bfloat16)
    tables = torch.randn((T, 6 * H), generator=g, dtype=torch.bfloat16)
    gate = tables.chunk(6, dim=-1)[2]  # a strided view, as the reference's test takes it
    idx = torch.randint(T, (S,), generator=g)
    return x, residual, gate, idx


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16)


@pytest.mark.parametrize("B,S,H", [(2, 37, 128), (1, 300, 3072), (3, 5, 5376)])
def test_op_bit_exact(cuda, B, S, H):
    x, residual, gate, idx = inputs(B, S, H, 7, seed=S + H)
    out = gate_residual(residual.to(cuda), x.to(cuda), gate.to(cuda), idx.to(cuda))
    ref = R.gate_residual(residual, x, gate, idx)
    assert out.shape == (B, S, H) and out.dtype == torch.bfloat16
    assert torch.equal(u16(out), u16(ref))


def test_op_strided_inputs_and_bad_index(cuda):
    x, residual, gate, idx = inputs(2, 24, 256, 4, seed=1)
    big = torch.cat([residual, x], dim=-1).to(cuda)         # row stride 512
    r_view, x_view = big[..., :256], big[..., 256:]
    idx = idx.clone()
    idx[3] = 9
    out = gate_residual(r_view, x_view, gate.to(cuda), idx.to(cuda))
    ok = torch.arange(24) != 3
    ref = R.gate_residual(residual[:, ok], x[:, ok], gate, idx[ok])
    assert torch.equal(u16(out[:, ok.to(cuda)]), u16(ref))
    assert torch.isnan(out[:, 3].float()).all()


def test_op_contract(cuda):
    x, residual, gate, idx = inputs(1, 4, 64, 2, seed=2)
    with pytest.raises(ValueError):
        gate_residual(residual.to(cuda).requires_grad_(), x.to(cuda), gate.to(cuda), idx.to(cuda))
    with pytest.raises(RuntimeError):
        gate_residual(residual.to(cuda), x.to(cuda), gate.to(cuda), idx.to(cuda), tile=1000)
    with pytest.raises(RuntimeError):
        gate_residual(residual.to(cuda), x[:, :, :32].to(cuda), gate.to(cuda), idx.to(cuda))


@pytest.mark.parametrize("kind", ["fp8", "int8"])
@pytest.mark.parametrize("B,S,K,Nf", [(2, 150, 512, 256), (1, 333, 768, 1024), (3, 7, 256, 96)])
def test_fused_epilogue_equals_gemm_then_op(cuda, kind, B, S, K, Nf):
    g = torch.Generator().manual_seed(K + Nf)
    x, _ = workloads.activations(B * S, K, g)
    w = (torch.randn((Nf, K), generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn((Nf,), generator=g) * 0.01).to(torch.bfloat16)
    residual = torch.randn((B, S, Nf), generator=g).to(torch.bfloat16)
    gate = (torch.randn((5, Nf), generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.randint(5, (S,), generator=g)
    dt = torch.float8_e4m3fn if kind == "fp8" else torch.int8
    qa, sa = xops.quantize_rows(x.to(cuda), dt)
    qw, sw = xops.quantize_rows(w.to(cuda), dt)
    fused = xops.scaled_mm_gate_residual(qa, qw, sa, sw, b.to(cuda), residual.reshape(-1, Nf).to(cuda),
                                         gate.to(cuda), idx.to(cuda))
    y, _ = xops.scaled_mm(qa, qw, sa, sw, b.to(cuda), torch.bfloat16, N.ACT_NONE, False)
    twostep = xops.gate_residual(residual.to(cuda), y.reshape(B, S, Nf), gate.to(cuda), idx.to(cuda))
    assert torch.equal(u16(fused), u16(twostep.reshape(-1, Nf)))
    lin = R.w8a8_linear_fp8 if kind == "fp8" else R.w8a8_linear_int8
    y_ref = lin(qa.cpu(), sa.cpu(), qw.cpu(), sw.cpu(), b)
    ref = R.gate_residual(residual, y_ref.reshape(B, S, Nf), gate, idx).reshape(-1, Nf)
    assert R.rel_l2(fused, ref) <= 1e-3 and R.cosine(fused, ref) >= 0.9999


@pytest.mark.parametrize("kind", ["fp8", "fp8_mfma", "int8"])
def test_module_forward_gate_residual(cuda, kind):
    g = torch.Generator().manual_seed(3)
    B, S, K, Nf = 2, 64, 512, 256
    x = torch.randn((B, S, K), generator=g).to(torch.bfloat16).to(cuda)
    w = (torch.randn((Nf, K), generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn((Nf,), generator=g) * 0.01).to(torch.bfloat16)
    residual = torch.randn((B, S, Nf), generator=g).to(torch.bfloat16).to(cuda)
    gate = (torch.randn((3, Nf), generator=g) * 0.5).to(torch.bfloat16).to(cuda)
    idx = torch.randint(3, (S,), generator=g).to(cuda)
    acc = "mfma" if kind == "fp8_mfma" else "exact"
    m = (H3FP8Linear(w, b, weight_scaling="channel", activation_scaling="token", accumulation=acc)
         if kind.startswith("fp8") else WeightQuantLinearModule(w, b)).to(cuda)
    fused = m.forward_gate_residual(x, residual, gate, idx)
    assert torch.equal(u16(fused), u16(gate_residual(residual, m(x), gate, idx)))


@pytest.mark.parametrize("accumulation", ["mfma", "exact"])
def test_full_size_out_projection(cuda, accumulation):
    """Out-projection [3072 x 3072] at M = 15,624 with the gated residual (fused into the FP8 MFMA
    kind's epilogue; after the GEMM for the exact kind): bit-exact against GEMM-then-op."""
    M, d = workloads.M_5S, workloads.D_MODEL
    g = workloads.generator(0, cuda)
    x, _ = workloads.activations(M, d, g, cuda)
    w, b = workloads.weight("out", g, cuda)
    residual = torch.randn((1, M, d), generator=g, device=cuda).to(torch.bfloat16)
    gate = (torch.randn((20, d), generator=g, device=cuda) * 0.1).to(torch.bfloat16)
    idx = torch.randint(20, (M,), generator=g, device=cuda)
    m = H3FP8Linear(w, b, weight_scaling="channel", activation_scaling="token", accumulation=accumulation)
    fused = m.forward_gate_residual(x[None], residual, gate, idx)
    assert torch.equal(u16(fused), u16(gate_residual(residual, m(x[None]), gate, idx)))


@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_fused_epilogue_bad_indices(cuda, kind):
    """Indices outside the gate table (negative, = T, a high word set) poison their rows in the
    fused epilogue exactly as in the standalone op (NaN rows, bit for bit); other rows unchanged."""
    B, S, K, Nf, T = 3, 100, 256, 96, 5
    g = torch.Generator().manual_seed(17)
    x, _ = workloads.activations(B * S, K, g)
    w = (torch.randn((Nf, K), generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn((Nf,), generator=g) * 0.01).to(torch.bfloat16)
    residual = torch.randn((B, S, Nf), generator=g).to(torch.bfloat16)
    gate = (torch.randn((T, Nf), generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.randint(T, (S,), generator=g)
    bad = [3, 40, 41, 99]
    idx[3], idx[40], idx[41], idx[99] = -1, T, 1 << 40, -(1 << 40)
    dt = torch.float8_e4m3fn if kind == "fp8" else torch.int8
    qa, sa = xops.quantize_rows(x.to(cuda), dt)
    qw, sw = xops.quantize_rows(w.to(cuda), dt)
    fused = xops.scaled_mm_gate_residual(qa, qw, sa, sw, b.to(cuda), residual.reshape(-1, Nf).to(cuda),
                                         gate.to(cuda), idx.to(cuda))
    y, _ = xops.scaled_mm(qa, qw, sa, sw, b.to(cuda), torch.bfloat16, N.ACT_NONE, False)
    twostep = xops.gate_residual(residual.to(cuda), y.reshape(B, S, Nf), gate.to(cuda), idx.to(cuda))
    assert torch.equal(u16(fused), u16(twostep.reshape(-1, Nf)))
    rows_bad = torch.zeros(S, dtype=torch.bool)
    rows_bad[bad] = True
    nan_rows = torch.isnan(fused.float().cpu()).reshape(B, S, Nf).all(dim=2)
    assert torch.equal(nan_rows, rows_bad.expand(B, S))
    assert not torch.isnan(fused.float().cpu()).reshape(B, S, Nf)[:, ~rows_bad].any()
