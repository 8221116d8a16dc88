"""The fused-path runtime surface (xgen_amd.operator.runtime and the modules Kernels
returns) against the contract of x_base/x_base/operator/npu_fusion/runtime.py, on
the CPU: names the block imports, Diagnostics, tensors_ok, no_hooks, quant_linear,
Kernels' fallbacks, and the signatures the block calls."""
import inspect
import logging

import pytest
import torch
from torch import nn

from xgen_amd.operator import gate_residual as gr
from xgen_amd.operator import nq2, runtime, swiglu_quant
from xgen_amd.operator.h3_fp8 import H3FP8Linear

FP8 = torch.float8_e4m3fn


def test_every_name_the_block_imports_exists():
    # x_diffusers/x_diffusers/framework/transformer/h3_npu_fusion.py:18
    for name in ("Diagnostics", "Kernels", "no_hooks", "quant_linear", "quant_matmul", "tensors_ok",
                 "configure_logging"):
        assert hasattr(runtime, name), name
    # x_base/x_base/operator/h3_nvfp4.py:33,99 import gate_first_swiglu from h3_swiglu
    assert callable(swiglu_quant.gate_first_swiglu)
    # what the block calls on the modules Kernels.get returns (h3_npu_fusion.py:44,66,92)
    assert callable(swiglu_quant.swiglu_quantize_reuse) and callable(gr.gate_residual)
    assert callable(nq2.norm_affine_quant)
    for module, args in ((nq2, (True,)), (swiglu_quant, ("reuse",)), (gr, ())):
        assert module.library_path(*args).name == "libxgen_amd.so"


def test_call_signatures_match_the_block():
    assert {"eps", "blocks", "cached"} <= set(inspect.signature(nq2.norm_affine_quant).parameters)
    assert {"tile", "blocks", "scale_mode"} <= set(inspect.signature(swiglu_quant.swiglu_quantize_reuse).parameters)
    assert {"tile", "blocks"} <= set(inspect.signature(gr.gate_residual).parameters)
    assert set(inspect.signature(swiglu_quant.gate_first_swiglu).parameters) == {"x", "with_amax"}
    assert list(inspect.signature(runtime.quant_matmul).parameters)[:4] == ["q", "scale", "linear", "shape"]


def test_diagnostics_counts_and_persistence(caplog):
    d = runtime.Diagnostics(prefix="H3_OPT")
    with caplog.at_level(logging.INFO, logger="xgen.optim"):
        d.hit("swiglu", "shape=(1, 2, 3)")
        d.hit("swiglu")
        assert d.fallback("norm_quant", "why") is False
        d.fallback("norm_quant", "why")
    assert d.hits["swiglu"] == 2
    assert d.fallbacks[("norm_quant", "why")] == 2
    assert sum("fallback=norm_quant" in r.message for r in caplog.records) == 1  # logged once
    # fallbacks outside a request persist across reset(); inside a request they do not
    d.reset()
    assert d.fallbacks[("norm_quant", "why")] == 2 and not d.hits
    d.in_request = True
    d.fallback("swiglu", "in-request")
    d.reset()
    assert ("swiglu", "in-request") not in d.fallbacks
    s = d.summary()
    assert s["phase"] == "request_end" and s["fallbacks"][0]["feature"] == "norm_quant"


def test_tensors_ok():
    t = torch.zeros(2, dtype=torch.bfloat16)
    with torch.no_grad():
        assert not runtime.tensors_ok(t)  # not on a HIP device
        assert not runtime.tensors_ok()
    meta = torch.empty(2, dtype=torch.bfloat16, device="meta")
    with torch.no_grad():
        assert not runtime.tensors_ok(meta)
    assert not runtime.tensors_ok(t)  # gradients enabled


def test_no_hooks():
    m = nn.Linear(4, 4)
    assert runtime.no_hooks(m)
    h = m.register_forward_hook(lambda *a: None)
    assert not runtime.no_hooks(m)
    h.remove()
    assert runtime.no_hooks(m)
    for attr in ("_hf_hook", "_diffusers_hook", "peft_config", "lora_A", "lora_B"):
        m2 = nn.Linear(4, 4)
        setattr(m2, attr, object())
        assert not runtime.no_hooks(m2), attr
    m3 = nn.Linear(4, 4)
    m3.forward = lambda x: x  # an instance-level forward override
    assert not runtime.no_hooks(m3)
    g = nn.modules.module.register_module_forward_hook(lambda *a: None)
    try:
        assert not runtime.no_hooks(nn.Linear(4, 4))
    finally:
        g.remove()


def test_quant_linear_gate():
    w = torch.zeros(32, 64, dtype=FP8)
    token = H3FP8Linear.from_packed(w, torch.ones(32), activation_scaling="token")
    assert runtime.quant_linear(token, 64) and not runtime.quant_linear(token, 32)
    assert not runtime.quant_linear(H3FP8Linear.from_packed(w, torch.ones(())), 64)  # per-tensor activations
    assert not runtime.quant_linear(nn.Linear(64, 32), 64)
    h = token.register_forward_pre_hook(lambda *a: None)
    assert not runtime.quant_linear(token, 64)  # hooked modules keep their forward
    h.remove()
    token.lora_A = nn.Identity()
    assert not runtime.quant_linear(token, 64)


def test_kernels_fall_back_off_device():
    d = runtime.Diagnostics()
    k = runtime.Kernels(d)
    x = torch.zeros(2, dtype=torch.bfloat16)
    for feature in runtime.Kernels.SPECS:
        assert k.get(feature, x) is None
    reasons = {f: r for (f, r) in d.fallbacks}
    assert "gfx950" in reasons["swiglu"]


def test_quant_linear_refuses_input_activation():
    """A linear whose own input quantization applies GELU-tanh cannot consume the block's shared
    plain (q, scale): quant_linear is False (the block then calls the module, and records the
    fallback) and quant_matmul refuses it instead of silently skipping the GELU."""
    w = torch.zeros(32, 64, dtype=FP8)
    gelu_in = H3FP8Linear.from_packed(w, torch.ones(32), activation_scaling="token", input_activation="gelu_tanh")
    assert not runtime.quant_linear(gelu_in, 64)
    with pytest.raises(ValueError, match="input_activation"):
        runtime.quant_matmul(torch.zeros(4, 64, dtype=FP8), torch.ones(4), gelu_in, (4, 64))
