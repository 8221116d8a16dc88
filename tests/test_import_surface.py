"""The names the reference's importers take from each module a maintainer aliases onto
xgen_amd (sys.modules["x_base...."] = xgen_amd....), and the installer object behind
--matmul_quant int8, on the CPU."""
import importlib
import sys

import pytest
import torch
from torch import nn

import xgen_amd.operator.matmul as matmul
from xgen_amd import config

# alias target -> {name: the reference's importers (file:line)}
IMPORTED = {
    "xgen_amd.operator.h3_fp8": {
        "H3FP8Linear": "x_diffusers/x_diffusers/adaptor/h3_input_refiner.py:53, h3_pair_parallel.py:11, "
                       "h3_cuda_precision.py:216, tools/benchmark_h3_parallel_block.py:53",
        "quantize_per_tensor": "x_base/x_base/operator/h3_fp8.py:9 (module function)",
    },
    "xgen_amd.operator.h3_fp8_quant": {
        "quantize_activation": "x_base/x_base/operator/h3_fp8.py:56",
    },
    "xgen_amd.operator.h3_abs_peak": {
        "activation_abs_peak": "x_base/x_base/operator/h3_fp8_quant.py:6, h3_nvfp4.py:76",
    },
    "xgen_amd.operator.matmul": {
        "matmul_manager": "x_base/x_base/operator/__init__.py:2 (re-exported by x_base/x_base/__init__.py:13)",
        "WeightQuantLinearModule": "x_base/x_base/operator/__init__.py:2, fsdp/fsdp.py:11, "
                                   "npu_fusion/runtime.py:74, h3_image_optimizations.py:79,117, "
                                   "x_comfyui/x_comfyui/framework/transformer/minimax_h3.py:70",
        "enable_weight_quant_linear": "x_diffusers/x_diffusers/framework/transformer/h3_image_optimizations.py:70,79",
        "MatmulManager": "x_base/x_base/operator/matmul.py:300 (class of matmul_manager)",
    },
    "xgen_amd.operator.runtime": {
        name: "x_diffusers/x_diffusers/framework/transformer/h3_npu_fusion.py:18"
        for name in ("Diagnostics", "Kernels", "no_hooks", "quant_linear", "quant_matmul", "tensors_ok")
    },
    "xgen_amd.operator.swiglu_quant": {
        "gate_first_swiglu": "x_base/x_base/operator/h3_nvfp4.py:33,99 (from .h3_swiglu)",
        "swiglu_quantize_reuse": "h3_npu_fusion.py:44 (through Kernels.get)",
        "library_path": "npu_fusion/runtime.py:125 (Kernels.get)",
    },
    "xgen_amd.operator.nq2": {
        "norm_affine_quant": "h3_npu_fusion.py:92 (through Kernels.get)",
        "library_path": "npu_fusion/runtime.py:125 (Kernels.get)",
    },
    "xgen_amd.operator.gate_residual": {
        "gate_residual": "h3_npu_fusion.py:66 (through Kernels.get)",
        "library_path": "npu_fusion/runtime.py:125 (Kernels.get)",
    },
    "xgen_amd.operator.merge_quant": {
        "merge_quant": "x_base/x_base/phaa/fused_layout.py:47 (through Kernels.get), test_npu_fusion_meta.py:60",
        "library_path": "npu_fusion/runtime.py:125 (Kernels.get)",
    },
    "xgen_amd.operator.phaa_layout": {
        "pack_qkv": "x_base/x_base/phaa/fused_layout.py:33 (through Kernels.get), test_npu_fusion_meta.py:66",
        "unpack_qkv": "x_base/x_base/operator/npu_fusion/phaa_layout.py:17 (module function)",
        "pack_back": "x_base/x_base/phaa/fused_layout.py:42, test_npu_fusion_meta.py:68",
        "merge_back": "x_base/x_base/phaa/fused_layout.py:51, test_npu_fusion_meta.py:69",
        "library_path": "npu_fusion/runtime.py:125 (Kernels.get)",
    },
    "xgen_amd.operator.quantized": {
        "QuantizedRows": "x_base/x_base/phaa/fused_layout.py:5, h3_npu_fusion.py:17",
    },
    "xgen_amd.operator.h3_indexed_affine": {
        "_apply": "x_base/x_base/operator/h3_indexed_affine.py:32, minimax_h3.py:692",
        "fused_h3_block_forward": "x_diffusers/x_diffusers/adaptor/h3_cuda.py:36",
    },
    "xgen_amd.phaa.fp8_transport": {
        "fp8_all_to_all": "x_base/x_base/phaa/phaa_attention.py:133",
        "fp8_all_to_all_many": "x_base/x_base/phaa/phaa_attention.py:133",
    },
    "xgen_amd.phaa.fp8_async_transport": {
        "AsyncFP8Options": "x_diffusers/x_diffusers/adaptor/h3_cuda.py:157, x_base/tests/test_phaa_fp8.py:77",
        "submit_fp8_exchange": "x_base/x_base/phaa/phaa_attention.py:145",
        "finish_fp8_exchange": "x_base/x_base/phaa/phaa_attention.py:145",
    },
    "xgen_amd.config": {
        "QuantLayerConfig": "x_comfyui/x_comfyui/framework/transformer/minimax_h3.py:68, "
                            "h3_image_optimizations.py:69,78",
    },
    "xgen_amd.adaln_cache": {
        "AdalnScheduleCache": "x_comfyui/x_comfyui/framework/transformer/minimax_h3.py:67, "
                              "tools/adaln_cache/prepare_cuda_adaln.py:119",
        "install_adaln_cache": "server/video/video_server.py:711, x_base/x_base/__init__.py:21",
    },
}


@pytest.mark.parametrize("module", sorted(IMPORTED))
def test_every_imported_name_exists(module):
    mod = importlib.import_module(module)
    missing = [f"{name} ({where})" for name, where in IMPORTED[module].items() if not hasattr(mod, name)]
    assert not missing, missing


def test_tensor_parallel_linear_is_not_provided():
    """H3FP8TPLinear (x_diffusers/x_diffusers/adaptor/h3_parallel.py:68, h3_cuda_precision.py:405) is
    the tensor-parallel form: outside this one-GPU path, so tensor-parallel users keep the
    reference's h3_fp8 module."""
    assert not hasattr(importlib.import_module("xgen_amd.operator.h3_fp8"), "H3FP8TPLinear")


def test_relative_import_through_alias(tmp_path, monkeypatch):
    """A package __init__ that does `from .matmul import matmul_manager, WeightQuantLinearModule`
    (the form of x_base/x_base/operator/__init__.py:2) imports through a sys.modules alias."""
    root = tmp_path / "xb_alias_probe"
    (root / "operator").mkdir(parents=True)
    (root / "__init__.py").write_text("")
    (root / "operator" / "__init__.py").write_text("from .matmul import matmul_manager, WeightQuantLinearModule\n")
    monkeypatch.syspath_prepend(str(tmp_path))
    monkeypatch.setitem(sys.modules, "xb_alias_probe.operator.matmul", matmul)
    try:
        probe = importlib.import_module("xb_alias_probe.operator")
        assert probe.matmul_manager is matmul.matmul_manager
        assert probe.WeightQuantLinearModule is matmul.WeightQuantLinearModule
    finally:
        for name in ("xb_alias_probe.operator", "xb_alias_probe"):
            sys.modules.pop(name, None)


class MiniMaxH3Transformer3DModel(nn.Module):
    def __init__(self):
        super().__init__()
        self.proj_in = nn.Linear(32, 32)
        self.block = nn.Linear(32, 32)


def test_online_dynamic_quant_detects_the_model_config(monkeypatch):
    seen = {}

    def fake(model, quant_config, dtype="w8a8"):
        seen["config"], seen["dtype"] = quant_config, dtype
        return model

    monkeypatch.setattr(matmul, "enable_weight_quant_linear", fake)
    model = MiniMaxH3Transformer3DModel()
    assert matmul.matmul_manager.enable_online_dynamic_quant(model) is model
    assert seen["dtype"] == "w8a8"
    assert seen["config"].exclude_patterns == config.get_config("minimax_h3").exclude_patterns
    assert not seen["config"].should_quantize("proj_in", model.proj_in)
    assert seen["config"].should_quantize("block", model.block)
    explicit = config.QuantLayerConfig(exclude_patterns=["block"])
    matmul.matmul_manager.enable_online_dynamic_quant(model, explicit)
    assert seen["config"] is explicit


def test_online_dynamic_quant_error_contract():
    """Failures surface as the reference's ValueError (matmul.py:339-341), the cause chained: here
    the quantizer has no HIP device, or the dtype is not W8A8."""
    if not torch.cuda.is_available():
        with pytest.raises(ValueError, match="Dynamic weight modify model failed") as info:
            matmul.matmul_manager.enable_online_dynamic_quant(nn.Sequential(nn.Linear(32, 32)))
        assert isinstance(info.value.__cause__, RuntimeError)
    with pytest.raises(ValueError, match="Dynamic weight modify model failed"):
        matmul.matmul_manager.enable_online_dynamic_quant(nn.Sequential(nn.ReLU()), dtype="w4a4")
    plain = nn.Sequential(nn.ReLU())
    assert matmul.matmul_manager.enable_online_dynamic_quant(plain) is plain  # nothing selected
    with pytest.raises(NotImplementedError):
        matmul.matmul_manager.enable_vae_conv3d_quant(nn.Identity())
