"""The fused block path reached the way the reference's H3 block reaches it:
through runtime.Kernels.get(feature, value) and the modules it returns, with the
calls and arguments of x_diffusers/x_diffusers/framework/transformer/
h3_npu_fusion.py (_h3_feed_forward :74-101 -> _h3_from_projected :33-54 ->
_h3_residual :56-72), on the HIP kernels, against the oracle composite of the
same INT8 FFN half-block."""
import pytest
import torch

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd.operator import gate_residual as gr
from xgen_amd.operator import nq2, swiglu_quant
from xgen_amd.operator.matmul import WeightQuantLinearModule
from xgen_amd.operator.runtime import Diagnostics, Kernels, quant_linear, quant_matmul, tensors_ok

pytestmark = pytest.mark.gpu


def test_ffn_half_block_through_kernels(cuda):
    g = torch.Generator().manual_seed(21)
    S, H, F, T, eps = 300, 1024, 2048, 6, 1e-5
    x = torch.randn((1, S, H), generator=g).to(torch.bfloat16)
    norm_w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    shift = (torch.randn((T, H), generator=g) * 0.1).to(torch.bfloat16)
    scale = (torch.randn((T, H), generator=g) * 0.1).to(torch.bfloat16)
    gate = (torch.randn((T, H), generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.randint(T, (S,), generator=g)
    w_up = (torch.randn((2 * F, H), generator=g) * 0.02).to(torch.bfloat16)
    b_up = (torch.randn(2 * F, generator=g) * 0.01).to(torch.bfloat16)
    w_dn = (torch.randn((H, F), generator=g) * 0.02).to(torch.bfloat16)
    b_dn = (torch.randn(H, generator=g) * 0.01).to(torch.bfloat16)
    up, down = WeightQuantLinearModule(w_up, b_up).to(cuda), WeightQuantLinearModule(w_dn, b_dn).to(cuda)
    xc, sc, sh, gt, ic, wc = (t.to(cuda) for t in (x, scale, shift, gate, idx, norm_w))

    diag = Diagnostics(prefix="H3_OPT")
    kernels = Kernels(diag)
    with torch.no_grad():
        assert tensors_ok(xc, sc, sh) and quant_linear(up, H, xc.device)
        k = kernels.get("norm_quant", xc)
        assert k is nq2
        q, s = k.norm_affine_quant(xc, wc.detach(), sc.detach(), sh.detach(), ic, eps=eps, cached=True)
        u = quant_matmul(q, s, up, xc.shape)
        diag.hit("norm_quant", f"shape={tuple(xc.shape)}")
        assert tensors_ok(u) and quant_linear(down, u.shape[-1] // 2, u.device)
        k = kernels.get("swiglu", u)
        assert k is swiglu_quant
        q2, s2 = k.swiglu_quantize_reuse(u, tile=4096, blocks=40)
        branch = quant_matmul(q2, s2, down, u.shape)
        diag.hit("swiglu", f"shape={tuple(u.shape)}")
        k = kernels.get("gate_residual", xc)
        assert k is gr
        out = k.gate_residual(xc, branch, gt.detach(), ic, tile=4096)
        diag.hit("gate_residual", f"shape={tuple(xc.shape)}")
    assert dict(diag.hits) == {"norm_quant": 1, "swiglu": 1, "gate_residual": 1} and not diag.fallbacks
    assert kernels.get("rope", xc) is None and ("rope", "not part of the W8A8 linear path built for MI355X") \
        in diag.fallbacks

    # oracle composite: RMSNorm * w -> modulate -> INT8 rows -> up -> SwiGLU + INT8 -> down -> gated residual
    qr, sr, _ = R.norm_affine_quant(x, norm_w, scale, shift, idx, eps, "rms", "int8")
    qw_up, sw_up = R.quantize_rows_int8(w_up)
    qw_dn, sw_dn = R.quantize_rows_int8(w_dn)
    u_ref = R.w8a8_linear_int8(qr, sr, qw_up, sw_up, b_up)
    q2r, s2r, _ = R.swiglu_quant(u_ref.reshape(1, S, 2 * F), False, "int8", 1)
    br_ref = R.w8a8_linear_int8(q2r, s2r, qw_dn, sw_dn, b_dn).reshape(1, S, H)
    out_ref = R.gate_residual(x, br_ref, gate, idx)
    for got, ref in ((u.reshape(S, -1), u_ref), (branch, br_ref), (out, out_ref)):
        rel, cos = R.rel_l2(got, ref), R.cosine(got, ref)
        assert rel <= 1e-2 and cos >= 0.9999, (rel, cos)
    # the front end's bytes feed the same up-projection accumulators: given them, u is exact
    assert torch.equal(quant_matmul(q, s, up, xc.shape).cpu(), u.cpu())


def test_gate_first_swiglu_matches_oracle(cuda):
    """h3_swiglu.py:31-41: bf16 activation of a gate-first [..., 2F] input, and its max |value|."""
    g = torch.Generator().manual_seed(22)
    x = (torch.randn((2, 37, 2 * 640), generator=g) * 2).to(torch.bfloat16)
    x[0, 3, 700] = float("nan")  # a NaN value propagates into amax
    out = swiglu_quant.gate_first_swiglu(x.to(cuda))
    out2, amax = swiglu_quant.gate_first_swiglu(x.to(cuda), with_amax=True)
    _, _, v = R.swiglu_quant(x, True, "fp8", 1)
    assert out.shape == (2, 37, 640) and out.dtype == torch.bfloat16
    v = v.reshape(2, 37, 640)
    same = torch.isnan(out.cpu()) == torch.isnan(v)
    assert same.all()
    fin = ~torch.isnan(v)
    assert torch.equal(out.cpu()[fin].view(torch.int16), v[fin].view(torch.int16))
    assert torch.equal(out2.cpu().view(torch.int16), out.cpu().view(torch.int16))
    assert amax.dim() == 0 and amax.dtype == torch.float32 and torch.isnan(amax.cpu())
    out3, amax3 = swiglu_quant.gate_first_swiglu(x[1:].to(cuda), with_amax=True)
    assert float(amax3) == float(v[1:].float().abs().max())


def test_attention_half_linear_path_through_kernels(cuda):
    """The block's attention half outside the attention itself, reached through Kernels.get as
    h3_npu_fusion.py reaches it: the front end's shared INT8 rows feed the Q/K/V projections
    (_h3_project_qkv :103-119), Q/K/V are packed into the exchange's send buffers
    (phaa/fused_layout.py:27-33), the returned chunks are merged and quantized into QuantizedRows
    (:44-48) for the INT8 out-projection (_h3_project_output :142-145), and the gated residual
    closes the half (:56-72).  One GPU stands in for the four owners: the 'returned' chunks are the
    V send buffer (the layout a peer's attention output comes back in), i.e. attention = identity on
    V.  Against the oracle composite of the same chain."""
    from xgen_amd.operator import merge_quant as mq
    from xgen_amd.operator import phaa_layout
    from xgen_amd.operator.quantized import QuantizedRows

    g = torch.Generator().manual_seed(23)
    S, H, W, T, eps = 64, 1024, 7168, 5, 1e-5
    x = torch.randn((1, S, H), generator=g).to(torch.bfloat16)
    norm_w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    shift, scale = ((torch.randn((T, H), generator=g) * 0.1).to(torch.bfloat16) for _ in range(2))
    gate = (torch.randn((T, H), generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.randint(T, (S,), generator=g)
    ws = [((torch.randn((n, k), generator=g) * 0.02).to(torch.bfloat16),
           (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16)) for n, k in ((W, H),) * 3 + ((H, W),)]
    to_q, to_k, to_v, to_out = (WeightQuantLinearModule(w, b).to(cuda) for w, b in ws)
    xc, sc, sh, gt, ic, wc = (t.to(cuda) for t in (x, scale, shift, gate, idx, norm_w))

    diag = Diagnostics(prefix="H3_OPT")
    kernels = Kernels(diag)
    with torch.no_grad():
        q, s = kernels.get("norm_quant", xc).norm_affine_quant(xc, wc, sc, sh, ic, eps=eps, cached=True)
        proj = [quant_matmul(q, s, lin, (1, S, H)) for lin in (to_q, to_k, to_v)]   # [1, S, 7168] each
        layout = kernels.get("phaa_layout", xc)
        sends = [torch.empty((7, 4, S, 1, 2, 128), dtype=torch.bfloat16, device=cuda) for _ in range(3)]
        layout.pack_qkv(*(p.view(1, S, 56, 128) for p in proj), *sends)
        merge = kernels.get("merge_quant", xc)
        qm, smq = merge.merge_quant(sends[2].view(7, 4, S, 1, 256))
        value = QuantizedRows(qm, smq, (1, S, W))
        branch = quant_matmul(value.q, value.scale, to_out, value.shape)
        out = kernels.get("gate_residual", xc).gate_residual(xc, branch, gt, ic)
    assert mq.merge_quant is merge.merge_quant and not diag.fallbacks

    qr, sr, _ = R.norm_affine_quant(x, norm_w, scale, shift, idx, eps, "rms", "int8")
    qws = [R.quantize_rows_int8(w) for w, _ in ws]
    v_ref = R.w8a8_linear_int8(qr, sr, *qws[2], ws[2][1])                       # [S, 7168]
    # the merged rows of V's send buffer are V's rows (pack then merge is the identity)
    assert torch.equal(R.merge_rows(R.phaa_pack_qkv(v_ref.reshape(1, S, 56, 128)).reshape(7, 4, S, 1, 256)), v_ref)
    qv, sv = R.quantize_rows_int8(proj[2].reshape(S, W))                       # from the kernel's own V
    assert torch.equal(qm.cpu(), qv) and torch.equal(smq.cpu(), sv)
    br_ref = R.w8a8_linear_int8(qv, sv, *qws[3], ws[3][1]).reshape(1, S, H)
    out_ref = R.gate_residual(x, br_ref, gate, idx)
    for got, ref in ((proj[2].reshape(S, W), v_ref), (branch, br_ref), (out, out_ref)):
        rel, cos = R.rel_l2(got, ref), R.cosine(got, ref)
        assert rel <= 1e-2 and cos >= 0.9999, (rel, cos)
