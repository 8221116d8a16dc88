"""The reference's fused operators under their own torch.ops names (xgen_amd.reference_ops): the
schemas of their TORCH_LIBRARY definitions, and the reference's Meta contract suite
(x_base/tests/test_npu_fusion_meta.py:33-48, 60-61, 63-73) run against both the op handles and this
package's wrapper modules, with no device initialized."""
import pytest
import torch

import xgen_amd  # noqa: F401  (registers torch.ops.h3_phaa_*)
from xgen_amd.operator import gate_residual, merge_quant, nq2, phaa_layout, swiglu_quant

M = torch.device("meta")


def tensor(*shape, dtype=torch.bfloat16):
    return torch.empty(shape, device=M, dtype=dtype)


@pytest.mark.parametrize("op,schema", [
    (lambda: torch.ops.h3_phaa_nq2.fused, "h3_phaa_nq2::fused(Tensor x, Tensor weight, Tensor scale, Tensor shift, "
     "Tensor indices, float eps=1.0000000000000001e-05, int blocks=40) -> (Tensor, Tensor)"),
    (lambda: torch.ops.h3_phaa_nq2_cached.fused, "h3_phaa_nq2_cached::fused(Tensor x, Tensor weight, Tensor scale, "
     "Tensor shift, Tensor indices, float eps=1.0000000000000001e-05, int blocks=40) -> (Tensor, Tensor)"),
    (lambda: torch.ops.h3_phaa_gate_residual.gate_residual, "h3_phaa_gate_residual::gate_residual(Tensor residual, "
     "Tensor branch, Tensor gate_table, Tensor indices, int tile=5376, int blocks=40) -> Tensor"),
    (lambda: torch.ops.h3_phaa_fusion_quant.swiglu_quantize, "h3_phaa_fusion_quant::swiglu_quantize(Tensor u, "
     "int tile=2048, int blocks=40, int scale_mode=1) -> (Tensor, Tensor)"),
    (lambda: torch.ops.h3_phaa_fusion_quant_vector.swiglu_quantize, "h3_phaa_fusion_quant_vector::swiglu_quantize("
     "Tensor u, int tile=2048, int blocks=40, int scale_mode=1) -> (Tensor, Tensor)"),
    (lambda: torch.ops.h3_phaa_fusion_quant_reuse.swiglu_quantize, "h3_phaa_fusion_quant_reuse::swiglu_quantize("
     "Tensor u, int tile=4096, int blocks=40, int scale_mode=1) -> (Tensor, Tensor)"),
    (lambda: torch.ops.h3_phaa_merge_quant.fused,
     "h3_phaa_merge_quant::fused(Tensor back_recv, int blocks=40) -> (Tensor, Tensor)"),
])
def test_schemas_are_the_references(op, schema):
    """nq2_queued.asc:47-51, gate_residual_queued.asc:31, swiglu_quant*_queued.asc:33,
    merge_quant_queued.asc:26."""
    assert str(op()._schemas[""]) == schema


def test_swiglu_and_width_boundary():
    """test_npu_fusion_meta.py:33-38: [B, S, 2F] -> int8 [B*S, F] + f32 [B*S]; 2F = 28,674 rejected."""
    for fn in (swiglu_quant.swiglu_quantize_reuse, torch.ops.h3_phaa_fusion_quant_reuse.swiglu_quantize):
        q, scale = fn(tensor(2, 17, 96))
        assert q.shape == (34, 48) and scale.shape == (34,) and q.dtype == torch.int8
    with pytest.raises(RuntimeError):
        torch.ops.h3_phaa_fusion_quant_reuse.swiglu_quantize(tensor(1, 2, 28674))
    with pytest.raises(RuntimeError, match="tile"):
        torch.ops.h3_phaa_fusion_quant.swiglu_quantize(tensor(2, 17, 96), 4096)


def test_gate_and_norm_contracts():
    """test_npu_fusion_meta.py:40-48: the gate keeps the residual's shape; nq2 gives int8 [B*S, H]
    and f32 [B*S]; H = 6,145 rejected."""
    value, table = tensor(2, 17, 64), tensor(3, 64)
    indices = tensor(17, dtype=torch.int64)
    for gate in (gate_residual.gate_residual, torch.ops.h3_phaa_gate_residual.gate_residual):
        assert gate(value, value, table, indices).shape == value.shape
    for norm in (lambda *a: nq2.norm_affine_quant(*a, cached=True), torch.ops.h3_phaa_nq2_cached.fused,
                 torch.ops.h3_phaa_nq2.fused):
        q, scale = norm(value, tensor(64), table, table, indices)
        assert q.shape == (34, 64) and scale.shape == (34,) and q.dtype == torch.int8
    with pytest.raises(RuntimeError):
        torch.ops.h3_phaa_nq2_cached.fused(tensor(1, 2, 6145), tensor(6145), tensor(3, 6145), tensor(3, 6145),
                                          tensor(2, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="indices"):
        torch.ops.h3_phaa_nq2.fused(value, tensor(64), table, table, tensor(16, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="gate_table"):
        torch.ops.h3_phaa_gate_residual.gate_residual(value, value, tensor(3, 32), indices)


def test_merge_contract():
    """test_npu_fusion_meta.py:60-61: [7, 4, 17, 1, 256] -> int8 [17, 7168] + f32 [17]; and the op's
    checks (merge_quant_queued.asc:10-13)."""
    for merge in (merge_quant.merge_quant, torch.ops.h3_phaa_merge_quant.fused):
        quantized, scale = merge(tensor(7, 4, 17, 1, 256))
        assert quantized.shape == (17, 7168) and scale.shape == (17,)
        assert quantized.dtype == torch.int8 and scale.dtype == torch.float32
    op = torch.ops.h3_phaa_merge_quant.fused
    with pytest.raises(RuntimeError, match=r"\[7,4,S,1,256\] required"):
        op(tensor(7, 4, 17, 2, 256))
    with pytest.raises(RuntimeError, match="contiguous BF16 required"):
        op(tensor(7, 4, 17, 1, 256, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="contiguous BF16 required"):
        op(tensor(4, 7, 17, 1, 256).transpose(0, 1))
    with pytest.raises(RuntimeError, match="DataCopy"):
        op(tensor(7, 4, (1 << 20) + 1, 1, 256))
    with pytest.raises(RuntimeError, match="blocks"):
        op(tensor(7, 4, 17, 1, 256), 41)
    with pytest.raises(ValueError, match="Inference only"):
        merge_quant.merge_quant(tensor(7, 4, 17, 1, 256).requires_grad_())
    q8, _ = merge_quant.merge_quant(tensor(7, 4, 17, 1, 256), out_dtype=torch.float8_e4m3fn)
    assert q8.dtype == torch.float8_e4m3fn
    q, s = torch.ops.xgen_amd.merge_quant(tensor(3, 2, 5, 2, 64), torch.int8)   # general geometry
    assert q.shape == (10, 384) and s.shape == (10,)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        torch.ops.xgen_amd.merge_quant(tensor(3, 2, 5, 2, 60), torch.int8)
    with pytest.raises(RuntimeError, match="16384"):
        torch.ops.xgen_amd.merge_quant(tensor(9, 8, 5, 1, 256), torch.int8)


def test_layout_and_mutation_schema():
    """test_npu_fusion_meta.py:63-71: the three layout ops accept the reference's shapes on Meta
    tensors and their schemas mark the written outputs."""
    q = tensor(1, 17, 56, 128)
    sends = [tensor(7, 4, 17, 1, 2, 128) for _ in range(3)]
    phaa_layout.pack_qkv(q, q, q, *sends)
    phaa_layout.pack_back(tensor(1, 2, 67, 128), tensor(4, 17, 1, 256), L=67, S=17)
    phaa_layout.merge_back(tensor(7, 4, 17, 1, 256), tensor(1, 17, 7168))
    schema = str(torch.ops.h3_phaa_layout.pack._schemas[""])
    assert "Tensor(a!)" in schema and "Tensor(b!)" in schema and "Tensor(c!)" in schema
    assert str(torch.ops.h3_phaa_layout.back._schemas[""]) == (
        "h3_phaa_layout::back(Tensor x, Tensor(a!) y, int S, int L, int tile=64, int blocks=40) -> ()")
    assert str(torch.ops.h3_phaa_layout.merge._schemas[""]) == (
        "h3_phaa_layout::merge(Tensor x, Tensor(a!) y, int tile=64, int blocks=40) -> ()")


def test_layout_contracts():
    """layout_queued.asc:10-49 checks and phaa_layout.py:13-28's own."""
    q = tensor(1, 17, 56, 128)
    sends = [tensor(7, 4, 17, 1, 2, 128) for _ in range(3)]
    with pytest.raises(ValueError, match="SP4/PHAA7"):
        phaa_layout.pack_qkv(q, q, q, *sends, P=8)
    with pytest.raises(ValueError, match="Inference only"):
        phaa_layout.pack_qkv(tensor(1, 17, 56, 128).requires_grad_(), q, q, *sends)
    with pytest.raises(RuntimeError, match=r"\[1,S,56,128\] required"):
        phaa_layout.pack_qkv(tensor(1, 17, 48, 128), q, q, *sends)
    with pytest.raises(RuntimeError, match="send shape mismatch"):
        phaa_layout.pack_qkv(q, q, q, tensor(7, 4, 16, 1, 2, 128), *sends[1:])
    with pytest.raises(RuntimeError, match="tile"):
        torch.ops.h3_phaa_layout.pack(q, q, q, *sends, 48)
    with pytest.raises(RuntimeError, match="single memory location"):
        phaa_layout.pack_qkv(q, q, q, sends[0], sends[0], sends[2])
    with pytest.raises(RuntimeError, match="zero/one padding"):
        phaa_layout.pack_back(tensor(1, 2, 65, 128), tensor(4, 17, 1, 256), L=65, S=17)
    with pytest.raises(RuntimeError, match="back_send shape mismatch"):
        phaa_layout.pack_back(tensor(1, 2, 68, 128), tensor(4, 17, 256), L=68, S=17)
    with pytest.raises(RuntimeError, match="contiguous"):
        phaa_layout.merge_back(tensor(7, 4, 17, 1, 256), tensor(1, 7168, 17).transpose(1, 2))
    with pytest.raises(RuntimeError, match="merged shape mismatch"):
        phaa_layout.merge_back(tensor(7, 4, 17, 1, 256), tensor(1, 16, 7168))
    with pytest.raises(RuntimeError, match="BF16"):
        phaa_layout.merge_back(tensor(7, 4, 17, 1, 256, dtype=torch.float16), tensor(1, 17, 7168))


def test_unpack_qkv_views():
    """phaa_layout.py:17-23 on the CPU (views only): position p of the attention input is peer p // S's
    position p % S."""
    S, L = 3, 11
    recv = [torch.arange(4 * S * 2 * 128, dtype=torch.float32).to(torch.bfloat16).reshape(4, S, 1, 2, 128)
            for _ in range(3)]
    views = phaa_layout.unpack_qkv(*recv, L=L)
    for x, v in zip(recv, views):
        assert v.shape == (1, 2, L, 128) and v.data_ptr() == x.data_ptr()
        for p in range(L):
            assert torch.equal(v[0, :, p], x[p // S, p % S, 0])
    with pytest.raises(ValueError, match="effective length"):
        phaa_layout.unpack_qkv(*recv, L=13)


def test_device_remains_uninitialized():
    """test_npu_fusion_meta.py:67-73."""
    assert not torch.cuda.is_initialized()


def test_register_is_idempotent():
    from xgen_amd import reference_ops
    assert reference_ops.register() == []
