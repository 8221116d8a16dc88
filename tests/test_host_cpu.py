"""Host logic without a GPU: module constructors' contract checks, the layer
selector, and the operators' Meta (shape/dtype) contracts — like the
reference's Meta contract suite (x_base/tests/test_npu_fusion_meta.py:12-79)."""
import pytest
import torch
from torch import nn

import xgen_amd  # noqa: F401  (registers torch.ops.xgen_amd)
from xgen_amd import config
from xgen_amd.operator.dit_chain import DiTLinearChain
from xgen_amd.operator.h3_fp8 import H3FP8Linear
from xgen_amd.operator.matmul import WeightQuantLinearModule
from xgen_amd.operator.nq2 import norm_affine_quant

xops = torch.ops.xgen_amd


def meta(*shape, dtype=torch.bfloat16):
    return torch.empty(shape, device="meta", dtype=dtype)


def test_projection_rejects_unaligned_dimensions():
    # x_base/tests/test_h3_cuda_precision_ops.py:14-16
    with pytest.raises(ValueError, match='divisible by 16'):
        H3FP8Linear(torch.randn(17, 32))


def test_input_activation_contract():
    with pytest.raises(ValueError, match="activation_scaling='token'"):
        H3FP8Linear(torch.randn(32, 32), input_activation="gelu_tanh")
    with pytest.raises(ValueError, match="unsupported input_activation"):
        H3FP8Linear(torch.randn(32, 32), activation_scaling="token", input_activation="relu")
    w = torch.zeros(32, 64, dtype=torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="activation_scaling='token'"):
        H3FP8Linear.from_packed(w, torch.ones(()), input_activation="gelu_tanh")
    with pytest.raises(ValueError, match="unsupported input_activation"):
        WeightQuantLinearModule(torch.zeros(32, 32), None, input_activation="silu")
    with pytest.raises(ValueError, match="gelu must be"):
        DiTLinearChain(*([torch.zeros(16, 16)] * 8), gelu="both")


def test_from_packed_contract():
    w = torch.zeros(32, 64, dtype=torch.float8_e4m3fn)
    with pytest.raises(ValueError, match='aligned E4M3'):
        H3FP8Linear.from_packed(torch.zeros(32, 64), torch.ones(()))
    with pytest.raises(ValueError, match='FP32 weight scale'):
        H3FP8Linear.from_packed(w, torch.ones(3))
    layer = H3FP8Linear.from_packed(w, torch.ones(()), torch.arange(32.))
    assert layer.in_features == 64 and layer.out_features == 32 and layer.calls == 0
    per_channel = H3FP8Linear.from_packed(w, torch.ones(32), activation_scaling="token")
    assert per_channel.weight_scale.shape == (32,)


def test_forward_requires_hip_bf16_input():
    layer = H3FP8Linear.from_packed(torch.zeros(32, 64, dtype=torch.float8_e4m3fn), torch.ones(()))
    with pytest.raises(ValueError, match='CUDA BF16/FP16'):
        layer(torch.randn(4, 64, dtype=torch.bfloat16))


def test_norm_affine_quant_rejects_grad():
    x = torch.randn(1, 4, 64, dtype=torch.bfloat16, requires_grad=True)
    t = torch.zeros(2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match='inference only'):
        norm_affine_quant(x, None, t, t, torch.zeros(4, dtype=torch.long))


def test_ops_have_no_cpu_kernel():
    with pytest.raises(NotImplementedError):
        xops.quantize_rows(torch.randn(4, 64, dtype=torch.bfloat16), torch.float8_e4m3fn)


# ------------------------------------------------------------------ selector
def test_h3_video_int8_keeps_adaln_projections_unquantized():
    # x_base/tests/test_h3_quant_precision.py:6-16
    class MiniMaxH3Transformer3DModel(nn.Module):
        pass

    cfg = config.get_config_for_model(MiniMaxH3Transformer3DModel())
    linear = nn.Linear(4, 4)
    assert not cfg.should_quantize("transformer_blocks.0.adaln_proj.linear", linear)
    assert not cfg.should_quantize("transformer_blocks.0.adaln_proj.linear.base_layer", linear)
    assert not cfg.should_quantize("norm_out.linear", linear)
    assert cfg.should_quantize("transformer_blocks.0.attn.to_q", linear)
    assert cfg.should_quantize("transformer_blocks.0.ff.net.0.proj", linear)


def test_hunyuan_selection_and_rules():
    class HunyuanVideoTransformer3DModel(nn.Module):
        pass

    cfg = config.get_config_for_model(HunyuanVideoTransformer3DModel())
    lin = nn.Linear(4, 4)
    assert cfg.should_quantize("transformer_blocks.3.ff.net.0.proj", lin)
    assert cfg.should_quantize("transformer_blocks.3.attn.to_q", lin)
    assert not cfg.should_quantize("time_text_embed.timestep_embedder.time_embedder.linear_1", lin)
    assert not cfg.should_quantize("transformer_blocks.3.attn.to_q.lora_A", lin)
    assert not cfg.should_quantize("transformer_blocks.3.norm2", nn.LayerNorm(4))
    # include list, glob and substring semantics, dtype lists
    c = config.QuantLayerConfig(include_patterns=["*blocks*"], exclude_patterns=["to_out"], int8_patterns=["*ff*"])
    assert c.should_quantize("blocks.0.ff.proj", lin)
    assert not c.should_quantize("blocks.0.attn.to_q", lin)          # int8 list does not match
    assert not c.should_quantize("head.ff", lin)                      # include list
    assert not c.should_quantize("blocks.0.to_out.ff", lin)           # exclude wins
    assert not config.QuantLayerConfig(int8_patterns=[]).should_quantize("a", lin)
    assert config.detect_config_name(type("MyWanThing", (nn.Module,), {})()) == "wan"


# ------------------------------------------------------------------ Meta contracts
def test_quantize_rows_meta():
    q, s = xops.quantize_rows(meta(2, 17, 96), torch.float8_e4m3fn)
    assert q.shape == (2, 17, 96) and q.dtype == torch.float8_e4m3fn and s.shape == (34,)
    q, s = xops.quantize_rows(meta(5, 64, dtype=torch.float16), torch.int8)
    assert q.dtype == torch.int8 and s.dtype == torch.float32
    with pytest.raises(RuntimeError):
        xops.quantize_rows(meta(5, 64, dtype=torch.float32), torch.int8)


def test_norm_affine_quant_meta_and_width_boundary():
    x = meta(2, 17, 64)
    table = meta(3, 64)
    idx = meta(17, dtype=torch.int64)
    q, s, n = xops.norm_affine_quant(x, meta(64), table, table, idx, 1e-6, 0, torch.float8_e4m3fn, True)
    assert q.shape == (34, 64) and s.shape == (34,) and n.shape == (34, 64)
    q, s, n = xops.norm_affine_quant(x, None, table, table, idx, 1e-6, 1, torch.int8, False)
    assert q.dtype == torch.int8 and n.numel() == 0
    with pytest.raises(RuntimeError):
        xops.norm_affine_quant(meta(1, 2, 8200), None, meta(3, 8200), meta(3, 8200),
                               meta(2, dtype=torch.int64), 1e-6, 0, torch.int8, False)
    with pytest.raises(RuntimeError):
        xops.norm_affine_quant(x, None, table, table, meta(16, dtype=torch.int64), 1e-6, 0, torch.int8, False)


def test_scaled_mm_meta():
    a = meta(300, 256, dtype=torch.float8_e4m3fn)
    w = meta(512, 256, dtype=torch.float8_e4m3fn)
    out, acc = xops.scaled_mm(a, w, meta(300, dtype=torch.float32), meta(512, dtype=torch.float32),
                              meta(512), torch.bfloat16, 1, True)
    assert out.shape == (300, 512) and out.dtype == torch.bfloat16 and acc.dtype == torch.float32
    ai = meta(300, 256, dtype=torch.int8)
    wi = meta(512, 256, dtype=torch.int8)
    out, acc = xops.scaled_mm(ai, wi, meta(300, dtype=torch.float32), meta(512, dtype=torch.float32),
                              None, torch.float16, 0, True)
    assert out.dtype == torch.float16 and acc.dtype == torch.int32
    with pytest.raises(RuntimeError):
        xops.scaled_mm(a, wi, meta(1, dtype=torch.float32), meta(1, dtype=torch.float32), None, torch.bfloat16, 0, False)
    with pytest.raises(RuntimeError):
        xops.scaled_mm(meta(4, 24, dtype=torch.int8), meta(16, 24, dtype=torch.int8), meta(1, dtype=torch.float32),
                       meta(1, dtype=torch.float32), None, torch.bfloat16, 0, False)


def test_meta_checks_leave_device_uninitialized():
    assert not torch.cuda.is_initialized()


def test_gate_residual_meta():
    m = torch.device("meta")
    r = torch.empty(2, 5, 64, dtype=torch.bfloat16, device=m)
    g = torch.empty(3, 64, dtype=torch.bfloat16, device=m)
    i = torch.empty(5, dtype=torch.int64, device=m)
    out = xops.gate_residual(r, r, g, i)
    assert out.shape == (2, 5, 64) and out.dtype == torch.bfloat16
    with pytest.raises(RuntimeError):
        xops.gate_residual(r, r, g[:, :32], i)
    with pytest.raises(RuntimeError):
        xops.gate_residual(r, r, g, i.to(torch.int32))


def test_indexed_modulate_meta():
    m = torch.device("meta")
    x = torch.empty(2, 5, 64, dtype=torch.bfloat16, device=m)
    tables = torch.empty(3, 6 * 64, dtype=torch.bfloat16, device=m)
    shift, scale = tables.chunk(6, dim=-1)[:2]
    i = torch.empty(5, dtype=torch.int64, device=m)
    out = xops.indexed_modulate(x, scale, shift, i)
    assert out.shape == (2, 5, 64) and out.dtype == torch.bfloat16
    assert xops.indexed_modulate(x, scale, shift, i, True).shape == (2, 5, 64)
    with pytest.raises(RuntimeError):
        xops.indexed_modulate(x, scale[:, :32], shift[:, :32], i)
    with pytest.raises(RuntimeError):
        xops.indexed_modulate(x, scale, shift[:2], i)
    with pytest.raises(RuntimeError):
        xops.indexed_modulate(x, scale, shift, i[:4])
    with pytest.raises(RuntimeError):
        xops.indexed_modulate(x.float(), scale, shift, i)


def test_indexed_affine_has_no_host_path():
    from xgen_amd.operator.h3_indexed_affine import _apply
    x = torch.zeros(1, 3, 16, dtype=torch.bfloat16)
    t = torch.zeros(2, 16, dtype=torch.bfloat16)
    for modulation in (True, False):
        with pytest.raises(RuntimeError, match="HIP"):
            _apply(x, t, t if modulation else x, torch.zeros(3, dtype=torch.int64), modulation=modulation)
    assert not torch.cuda.is_initialized()


def test_scaled_mm_gate_residual_meta():
    m = torch.device("meta")
    a = torch.empty(10, 64, dtype=torch.float8_e4m3fn, device=m)
    w = torch.empty(32, 64, dtype=torch.float8_e4m3fn, device=m)
    sa, sw = torch.empty(10, device=m), torch.empty(32, device=m)
    res = torch.empty(10, 32, dtype=torch.bfloat16, device=m)
    g = torch.empty(4, 32, dtype=torch.bfloat16, device=m)
    out = xops.scaled_mm_gate_residual(a, w, sa, sw, None, res, g, torch.empty(5, dtype=torch.int64, device=m))
    assert out.shape == (10, 32) and out.dtype == torch.bfloat16
    with pytest.raises(RuntimeError):   # M not a multiple of S
        xops.scaled_mm_gate_residual(a, w, sa, sw, None, res, g, torch.empty(3, dtype=torch.int64, device=m))


# --------------------------------------------------------------------------- PHAA FP8 transport (host checks)
@pytest.mark.parametrize("device", ["cpu", "meta"])
def test_non_cuda_transport_is_rejected_before_collective(monkeypatch, device):
    """test_phaa_fp8_alignment.py:9-21: non-CUDA tensors raise before any collective."""
    from unittest.mock import patch

    import torch.distributed as dist

    from xgen_amd.phaa import fp8_transport as transport

    monkeypatch.setenv("XGEN_PHAA_FP8_ALIGN16", "1")
    tensor = torch.empty((2, 128), device=device)
    with patch.object(dist, "get_world_size") as world_size, patch.object(dist, "all_to_all_single") as exchange:
        with pytest.raises(ValueError, match="requires CUDA tensors"):
            transport.fp8_all_to_all(torch.empty_like(tensor), tensor, 128, None)
    world_size.assert_not_called()
    exchange.assert_not_called()


def test_transport_rejects_bad_stream_counts():
    from xgen_amd.phaa import fp8_transport as transport

    t = torch.empty((2, 128))
    with pytest.raises(ValueError, match="one tensor or a QKV triple"):
        transport.fp8_all_to_all_many((t, t), (t, t), 128, None)
    with pytest.raises(ValueError, match="one tensor or a QKV triple"):
        transport.fp8_all_to_all_many((t,), (t, t, t), 128, None)


def test_wire_shape_contract():
    from xgen_amd.phaa.fp8_transport import wire_shape

    assert wire_shape(3, 2 * 17 * 3, 128, 2, 0) == (3 * 2 * 17 * 3, 132)
    assert wire_shape(1, 2 * 17 * 3, 128, 2, 4) == (2, 17 * 3 * 132 + 4)


def test_gemm_operand_views_are_passed_or_copied():
    """The GEMM wrappers hand a [rows, cols] view to the kernels as it is when its rows are unit-stride,
    cover the row, start 16-byte aligned and step by a multiple of the row alignment; anything else
    is copied into a fresh contiguous tensor (the kernels reject such views)."""
    from xgen_amd.ops import _kernel_rows
    big = torch.zeros(8, 96, dtype=torch.int8)
    assert big.data_ptr() % 16 == 0
    for view in (big[:, :64], big[:, 16:80], big[2:6, 32:48]):
        assert _kernel_rows(view, 16) is view
    unaligned = big[:, 1:65]                               # base 1 byte past a 16-byte boundary
    column_major = big[:, :64].t().contiguous().t()         # column stride 8
    odd_rows = big.view(-1)[:160].as_strided((4, 64), (40, 1))  # row stride 40, not a multiple of 16
    for view in (unaligned, column_major, odd_rows):
        out = _kernel_rows(view, 16)
        assert out is not view and out.is_contiguous() and out.data_ptr() % 16 == 0 and torch.equal(out, view)
    wide = torch.zeros(4, 40, dtype=torch.bfloat16)  # row stride 40 elements: a multiple of 8, not of 16
    assert _kernel_rows(wide[:, 8:24], 8).data_ptr() == wide[:, 8:24].data_ptr()
    assert _kernel_rows(wide[:, :16], 16).stride(0) == 16
