"""GPU parity of the reference module surfaces built on the HIP kernels:
H3FP8Linear (per-tensor and per-token/per-channel), WeightQuantLinearModule,
the layer swapper, shared-QKV quant_matmul, and the FFN pair (up + GELU-tanh,
per-token requant, down)."""
import pytest
import torch
import torch.nn.functional as F
from torch import nn

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd import config, workloads
from xgen_amd.operator.h3_fp8 import H3FP8Linear, quantize_per_tensor
from xgen_amd.operator.matmul import WeightQuantLinearModule, enable_weight_quant_linear
from xgen_amd.operator.runtime import quant_linear, quant_matmul

pytestmark = pytest.mark.gpu
xops = torch.ops.xgen_amd


def test_fp8_projection_bias_and_unaligned_rows(cuda):
    # x_base/tests/test_h3_cuda_precision_ops.py:19-32
    torch.manual_seed(42)
    weight = torch.randn(256, 128, dtype=torch.bfloat16)
    bias = torch.randn(256, dtype=torch.bfloat16)
    layer = H3FP8Linear(weight, bias).cuda()
    x = torch.randn(2, 19, 128, device='cuda', dtype=torch.bfloat16)
    result = layer(x)
    reference = F.linear(x, weight.cuda(), bias.cuda())
    assert result.shape == reference.shape and result.dtype == reference.dtype
    assert layer.weight.dtype == torch.float8_e4m3fn
    assert torch.isfinite(result).all()
    relative = (result.float() - reference.float()).square().mean().sqrt() / reference.float().square().mean().sqrt()
    assert relative.item() < 0.08
    assert layer.calls == 1


def test_per_tensor_module_matches_oracle(cuda):
    torch.manual_seed(1)
    weight = torch.randn(512, 256, dtype=torch.bfloat16) * 0.02
    bias = torch.randn(512, dtype=torch.bfloat16) * 0.01
    layer = H3FP8Linear(weight, bias)
    assert layer.weight.device.type == "cpu"  # buffers stay on the weight's device (h3_fp8.py:22-25)
    layer = layer.cuda()
    qw, sw = R.quantize_per_tensor(weight)
    assert torch.equal(layer.weight.cpu().view(torch.uint8), qw.view(torch.uint8))
    assert torch.equal(layer.weight_scale.cpu(), sw)
    x = torch.randn(3, 41, 256, dtype=torch.bfloat16)
    out = layer(x.cuda())
    qa, sa = R.quantize_per_tensor(x.reshape(-1, 256))
    ref = R.w8a8_linear_fp8(qa, sa, qw, sw, bias).reshape(3, 41, 512)
    assert R.rel_l2(out, ref) < 1e-3 and R.cosine(out, ref) > 0.9999
    assert out.shape == (3, 41, 512)
    assert layer(x.cuda()[:, :0]).shape == (3, 0, 512)
    # the module function itself (h3_fp8.py:9-12): bytes and scale of the oracle, on the input's device
    for src in (weight, weight.cuda()):
        q, sc = quantize_per_tensor(src)
        assert q.device == src.device and sc.device == src.device and sc.dim() == 0
        assert torch.equal(q.cpu().view(torch.uint8), qw.view(torch.uint8)) and torch.equal(sc.cpu(), sw.reshape(()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_token_channel_module_c1(cuda, dtype):
    """C1: x [256,1024], W [1024,1024] per-channel, per-token activations."""
    inp = workloads.linear_inputs(256, 1024, 1024, seed=0)
    layer = H3FP8Linear(inp.weight, inp.bias, weight_scaling="channel", activation_scaling="token").cuda()
    qw, sw = R.quantize_rows_fp8(inp.weight)
    assert torch.equal(layer.weight.cpu().view(torch.uint8), qw.view(torch.uint8))
    assert torch.equal(layer.weight_scale.cpu(), sw)
    x = inp.x.to(dtype)
    out = layer(x.cuda())
    assert out.dtype == dtype
    qa, sa = R.quantize_rows_fp8(x)
    ref = R.w8a8_linear_fp8(qa, sa, qw, sw, inp.bias, dtype)
    assert R.rel_l2(out, ref) < 1e-3 and R.cosine(out, ref) > 0.9999
    # the fake-quant CPU baseline path agrees to the north-star bar
    assert R.rel_l2(out, R.cpu_fake_quant_linear_fp8(inp.x, qw, sw, inp.bias)) <= 1e-2


def test_default_accumulation_is_exact(cuda):
    """H3FP8Linear sums exactly by default, as the reference's use_fast_accum=False asks
    (h3_fp8.py:63-66): its output equals the exact kind's bit for bit and sits at the exactly
    summed oracle's rounding; accumulation='mfma' is the FP8 MFMA's sum."""
    inp = workloads.linear_inputs(200, 1024, 512, seed=9)
    opts = dict(weight_scaling="channel", activation_scaling="token")
    default = H3FP8Linear(inp.weight, inp.bias, **opts).cuda()
    fast = H3FP8Linear(inp.weight, inp.bias, accumulation="mfma", **opts).cuda()
    assert default.accumulation == "exact" and H3FP8Linear.from_packed(default.weight, default.weight_scale).accumulation == "exact"
    x = inp.x.cuda()
    qa, sa = R.quantize_rows_fp8(inp.x)
    qw, sw = default.weight.cpu(), default.weight_scale.cpu()
    exact = R.w8a8_linear_fp8(qa, sa, qw, sw, inp.bias)
    y = default(x)
    assert R.bf16_ulp_diff(y, exact).max() <= 1 and R.rel_l2(y, exact) < 1e-4
    q, s = xops.quantize_rows(x, torch.float8_e4m3fn)
    y2, _ = xops.scaled_mm(q, default.weight, s, default.weight_scale, default.bias, torch.bfloat16, 0, False, True)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    model = R.w8a8_linear_fp8(qa, sa, qw, sw, inp.bias, accumulate=R.fp8_mfma_accumulate)
    assert R.rel_l2(fast(x), model) < 1e-4


def test_from_packed_reuses_bytes(cuda):
    inp = workloads.linear_inputs(64, 256, 128, seed=2)
    a = H3FP8Linear(inp.weight, inp.bias).cuda()
    b = H3FP8Linear.from_packed(a.weight, a.weight_scale, a.bias)
    x = inp.x.cuda()
    assert torch.equal(a(x), b(x))


def test_int8_module_matches_oracle(cuda):
    inp = workloads.linear_inputs(300, 1024, 512, seed=4)
    layer = WeightQuantLinearModule(inp.weight.cuda(), inp.bias)
    # parameters are kept on the CPU after quantization, as the reference's (matmul.py:39-48)
    assert layer.weight.device.type == "cpu" and layer.antiquant_scale.device.type == "cpu"
    layer = layer.cuda()
    qw, sw = R.quantize_rows_int8(inp.weight)
    assert torch.equal(layer.weight.cpu(), qw) and torch.equal(layer.antiquant_scale.cpu(), sw)
    assert layer.in_features == 1024 and layer.out_features == 512
    x = inp.x.reshape(3, 100, 1024)
    out = layer(x.cuda())
    qa, sa = R.quantize_rows_int8(inp.x)
    ref = R.w8a8_linear_int8(qa, sa, qw, sw, inp.bias).reshape(3, 100, 512)
    assert R.rel_l2(out, ref) < 1e-3 and R.cosine(out, ref) > 0.9999
    # fp32 input is cast to bf16 (matmul.py:57-59)
    out32 = layer(x.float().cuda())
    assert out32.dtype == torch.bfloat16 and torch.equal(out32, out)


def test_swapper_replaces_selected_linears(cuda):
    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = nn.Module()
            self.attn.to_q = nn.Linear(64, 64)
            self.ff = nn.Sequential(nn.Linear(64, 256), nn.GELU(approximate="tanh"), nn.Linear(256, 64))
            self.time_embedder = nn.Linear(64, 64)

    class HunyuanVideoTransformer3DModel(nn.Module):
        def __init__(self):
            super().__init__()
            self.transformer_blocks = nn.ModuleList([Block(), Block()])

    model = HunyuanVideoTransformer3DModel().to(torch.bfloat16)
    enable_weight_quant_linear(model, config.get_config_for_model(model))
    blk = model.transformer_blocks[1]
    assert type(blk.attn.to_q) is WeightQuantLinearModule
    assert type(blk.ff[0]) is WeightQuantLinearModule and type(blk.ff[2]) is WeightQuantLinearModule
    assert type(blk.time_embedder) is nn.Linear
    y = blk.ff.cuda()(torch.randn(5, 64, dtype=torch.bfloat16, device="cuda"))
    assert y.shape == (5, 64) and torch.isfinite(y).all()


@pytest.mark.parametrize("kind", ["fp8", "fp8_mfma", "int8"])
def test_shared_qkv_quant_matmul(cuda, kind):
    """One activation quantization shared by Q, K, V (h3_npu_fusion.py:103-119); fp8: the default
    (exact) accumulation, fp8_mfma: the FP8 MFMA sum."""
    acc_kind = "mfma" if kind == "fp8_mfma" else "exact"
    kind = "fp8" if kind.startswith("fp8") else kind
    g = workloads.generator(7)
    x, _ = workloads.activations(130, 512, g)
    layers = []
    for _ in range(3):
        w = (torch.randn(256, 512, generator=g) * 0.02).to(torch.bfloat16)
        b = (torch.randn(256, generator=g) * 0.01).to(torch.bfloat16)
        layers.append((H3FP8Linear(w, b, weight_scaling="channel", activation_scaling="token",
                                   accumulation=acc_kind) if kind == "fp8" else WeightQuantLinearModule(w, b)).cuda())
    assert all(quant_linear(m, 512, torch.device("cuda", 0)) for m in layers)
    xs = x.reshape(1, 130, 512).cuda()
    q, s = xops.quantize_rows(xs.reshape(-1, 512), torch.float8_e4m3fn if kind == "fp8" else torch.int8)
    outs = [quant_matmul(q, s, m, xs.shape) for m in layers]
    # the shared bytes and scales are the oracle's quantizer's
    q_ref, s_ref = (R.quantize_rows_fp8 if kind == "fp8" else R.quantize_rows_int8)(x)
    assert torch.equal(q.cpu().view(torch.uint8), q_ref.view(torch.uint8)) and torch.equal(s.cpu(), s_ref)
    for m, o in zip(layers, outs):
        assert o.shape == (1, 130, 256)
        assert torch.equal(o, m(xs))
        # each projection against the oracle linear on the shared (q, scale)
        if kind == "fp8":
            ref = R.w8a8_linear_fp8(q_ref, s_ref, m.weight.cpu(), m.weight_scale.cpu(), m.bias.cpu(),
                                    accumulate=R.fp8_mfma_accumulate if m.accumulation == "mfma" else None)
        else:
            ref = R.w8a8_linear_int8(q_ref, s_ref, m.weight.cpu(), m.antiquant_scale.cpu(), m.bias.cpu())
        rel, cos = R.rel_l2(o.reshape(130, 256), ref), R.cosine(o.reshape(130, 256), ref)
        assert rel <= 1e-3 and cos >= 0.9999, (rel, cos)


@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_ffn_pair_gelu_requant(cuda, kind):
    """C3 composition at reduced M: up (+GELU-tanh epilogue) -> per-token requant -> down."""
    g = workloads.generator(3)
    M, d = 200, 768
    x, _ = workloads.activations(M, d, g)
    wu = (torch.randn(4 * d, d, generator=g) * 0.02).to(torch.bfloat16)
    bu = (torch.randn(4 * d, generator=g) * 0.01).to(torch.bfloat16)
    wd = (torch.randn(d, 4 * d, generator=g) * 0.02).to(torch.bfloat16)
    bd = (torch.randn(d, generator=g) * 0.01).to(torch.bfloat16)
    if kind == "fp8":
        up = H3FP8Linear(wu, bu, weight_scaling="channel", activation_scaling="token", activation="gelu_tanh").cuda()
        down = H3FP8Linear(wd, bd, weight_scaling="channel", activation_scaling="token").cuda()
        quant, lin = R.quantize_rows_fp8, R.w8a8_linear_fp8
    else:
        up, down = WeightQuantLinearModule(wu, bu).cuda(), WeightQuantLinearModule(wd, bd).cuda()
        quant, lin = R.quantize_rows_int8, R.w8a8_linear_int8
    xc = x.cuda()
    if kind == "fp8":
        h = up(xc)
    else:
        qx, sx = xops.quantize_rows(xc, torch.int8)
        h, _ = xops.scaled_mm(qx, up.weight, sx, up.antiquant_scale, up.bias, torch.bfloat16, 1, False)
    y = down(h)
    # oracle composition (reference order: linear -> bf16 -> GELU(tanh) -> next linear's quantizer)
    qw_u, sw_u = quant(wu)
    qw_d, sw_d = quant(wd)
    qa, sa = quant(x)
    h_ref = lin(qa, sa, qw_u, sw_u, bu, torch.bfloat16, "gelu_tanh")
    assert R.rel_l2(h, h_ref) < 1e-2 and R.cosine(h, h_ref) > 0.9999
    qh, sh = quant(h_ref)
    y_ref = lin(qh, sh, qw_d, sw_d, bd)
    assert R.rel_l2(y, y_ref) < 1e-2 and R.cosine(y, y_ref) > 0.9999
    # requant bytes exact given the kernel's own GELU output
    qh_gpu, sh_gpu = xops.quantize_rows(h, torch.float8_e4m3fn if kind == "fp8" else torch.int8)
    qh2, sh2 = quant(h.cpu())
    assert torch.equal(qh_gpu.cpu().view(torch.uint8), qh2.view(torch.uint8))
    assert torch.equal(sh_gpu.cpu(), sh2)


@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_ffn_pair_gelu_in_down_requant(cuda, kind):
    """input_activation='gelu_tanh' (H3FP8Linear, WeightQuantLinearModule) applies the GELU in the
    module's input quantization: the down projection of the plain up output equals the down
    projection of the GELU-epilogue up output, bit for bit, also with the gated residual fused."""
    from xgen_amd import _native as N
    g = workloads.generator(4)
    M, d, T = 300, 512, 5
    x, _ = workloads.activations(M, d, g)
    wu = (torch.randn(4 * d, d, generator=g) * 0.02).to(torch.bfloat16)
    bu = (torch.randn(4 * d, generator=g) * 0.01).to(torch.bfloat16)
    wd = (torch.randn(d, 4 * d, generator=g) * 0.02).to(torch.bfloat16)
    bd = (torch.randn(d, generator=g) * 0.01).to(torch.bfloat16)
    xc = x.cuda()[None]
    if kind == "fp8":
        opts = dict(weight_scaling="channel", activation_scaling="token")
        h_gelu = H3FP8Linear(wu, bu, activation="gelu_tanh", **opts).cuda()(xc)
        h = H3FP8Linear(wu, bu, **opts).cuda()(xc)
        down = H3FP8Linear(wd, bd, **opts).cuda()
        down_gelu = H3FP8Linear(wd, bd, input_activation="gelu_tanh", **opts).cuda()
        assert "input_activation=gelu_tanh" in repr(down_gelu)
    else:
        up = WeightQuantLinearModule(wu, bu).cuda()
        qx, sx = xops.quantize_rows(xc[0], torch.int8)
        h_gelu = xops.scaled_mm(qx, up.weight, sx, up.antiquant_scale, up.bias, torch.bfloat16, N.ACT_GELU_TANH,
                                False)[0][None]
        h = up(xc)
        down = WeightQuantLinearModule(wd, bd).cuda()
        down_gelu = WeightQuantLinearModule(wd, bd, input_activation="gelu_tanh").cuda()
    assert torch.equal(down(h_gelu).view(torch.int16), down_gelu(h).view(torch.int16))
    res = torch.randn((1, M, d), generator=g).to(torch.bfloat16).cuda()
    gate = (torch.randn((T, d), generator=g) * 0.1).to(torch.bfloat16).cuda()
    idx = torch.randint(T, (M,), generator=g).cuda()
    r1 = down.forward_gate_residual(h_gelu, res, gate, idx)
    r2 = down_gelu.forward_gate_residual(h, res, gate, idx)
    assert torch.equal(r1.view(torch.int16), r2.view(torch.int16))
