"""Kernel capability checks, lazy loading and bounded diagnostic logging for the
fused block path, over the xgen_amd HIP library.

Same names and contracts as x_base/x_base/operator/npu_fusion/runtime.py, which
x_diffusers/x_diffusers/framework/transformer/h3_npu_fusion.py:18 imports:

  Diagnostics             runtime.py:18-52   per-request hits / fallbacks, bounded logging
  tensors_ok              runtime.py:55-60   inference-only tensors of one dtype on one
                                             device (here a HIP device: torch's "cuda")
  no_hooks                runtime.py:62-70   no global / module hooks, adapters or an
                                             overridden forward
  quant_linear            runtime.py:73-84   is this a native W8A8 linear that can take a
                                             shared (q, scale)?
  quant_matmul            runtime.py:87-91   GEMM of a pre-quantized activation
  Kernels.get             runtime.py:94-140  the module implementing a fused feature, or
                                             None (with a recorded fallback) when it
                                             cannot be loaded; errors after dispatch
                                             propagate

Kernels maps the block's features onto this package's modules: "norm_quant" ->
xgen_amd.operator.nq2, "swiglu" -> .swiglu_quant, "gate_residual" ->
.gate_residual; all three live in the one library libxgen_amd.so.  The
reference's other features (rope, PHAA layout, laser preprocessing, merge
quantization) are outside the W8A8 linear path and always fall back to the
block's native forward, with that reason recorded.
"""
from __future__ import annotations

import importlib
import json
import logging
import os
from collections import Counter

import torch

from .h3_fp8 import H3FP8Linear
from .matmul import WeightQuantLinearModule, quant_matmul_raw

LOG = logging.getLogger("xgen.optim")
ARCH = "gfx950"


def configure_logging():
    """Compatibility helper: handlers and levels belong to the application."""


class Diagnostics:
    """Counts fused-path hits and fallbacks; logs each (feature, outcome) once."""

    def __init__(self, prefix="OP_OPT"):
        self.prefix = prefix
        self.seen = set()
        self.persistent = Counter()  # fallbacks recorded outside a request survive reset()
        self.in_request = False
        self.reset()

    def reset(self):
        self.hits = Counter()
        self.fallbacks = self.persistent.copy()

    def hit(self, feature, detail=""):
        self.hits[feature] += 1
        if (feature, "enabled") not in self.seen:
            self.seen.add((feature, "enabled"))
            LOG.info("[%s] rank=%s enabled=%s %s", self.prefix, os.environ.get("RANK", "0"), feature, detail)

    def fallback(self, feature, reason):
        key = (feature, reason)
        self.fallbacks[key] += 1
        if not self.in_request:
            self.persistent[key] += 1
        if key not in self.seen:
            self.seen.add(key)
            LOG.warning("[%s] rank=%s fallback=%s reason=%s", self.prefix, os.environ.get("RANK", "0"), feature, reason)
        return False

    def summary(self, phase="request_end"):
        data = {"phase": phase, "rank": os.environ.get("RANK", "0"), "hits": dict(self.hits),
                "fallbacks": [{"feature": f, "reason": r, "count": n} for (f, r), n in sorted(self.fallbacks.items())]}
        LOG.info("[%s] summary=%s", self.prefix, json.dumps(data, ensure_ascii=False, sort_keys=True))
        return data


def tensors_ok(*values, dtype=torch.bfloat16):
    """Inference-only tensors of `dtype`, all on one HIP device."""
    if torch.is_grad_enabled() or not values:
        return False
    first = values[0]
    return all(isinstance(x, torch.Tensor) and x.dtype == dtype and not x.requires_grad and x.device.type == "cuda"
               and x.device == first.device for x in values)


_MODULE_HOOKS = ("_hf_hook", "_diffusers_hook", "_forward_hooks", "_forward_pre_hooks", "peft_config", "lora_A",
                 "lora_B")


def no_hooks(module):
    """Do not bypass offload, adapter or user hooks on a module the fused path would skip."""
    global_hooks = torch.nn.modules.module
    return (not any(getattr(global_hooks, name, None) for name in ("_global_forward_hooks",
                                                                   "_global_forward_pre_hooks"))
            and not any(getattr(module, name, None) for name in _MODULE_HOOKS)
            and "forward" not in vars(module))


def quant_linear(module, width=None, device=None):
    """The reference's gate for consuming a shared (q, scale): the INT8 module (int8 weight,
    float32 antiquant_scale [N]) or, here, also the FP8 module with per-token activation scales
    (e4m3fn weight, float32 weight_scale [1] or [N]); no hooks; shapes and devices as asked."""
    weight = getattr(module, "weight", None)
    bias = getattr(module, "bias", None)
    if type(module) is WeightQuantLinearModule:
        scale, wdtype = getattr(module, "antiquant_scale", None), torch.int8
    elif type(module) is H3FP8Linear and getattr(module, "activation_scaling", None) == "token":
        scale, wdtype = getattr(module, "weight_scale", None), torch.float8_e4m3fn
    else:
        return False
    if not isinstance(weight, torch.Tensor) or weight.ndim != 2 or weight.dtype != wdtype:
        return False
    counts = (weight.shape[0],) if wdtype == torch.int8 else (1, weight.shape[0])
    return (no_hooks(module)
            and isinstance(scale, torch.Tensor) and scale.dtype == torch.float32 and scale.numel() in counts
            and (width is None or weight.shape[1] == width)
            and (device is None or weight.device == scale.device == device)
            and (bias is None or device is None or bias.device == device))


def quant_matmul(q, scale, linear, shape, out_dtype=torch.bfloat16):
    """GEMM of a pre-quantized activation q [M,K] (+ per-token scale [M]) through `linear`,
    reshaped to [*shape[:-1], N]."""
    if type(linear) is H3FP8Linear:
        out = linear.forward_quantized(q.reshape(-1, q.shape[-1]), scale.reshape(-1), out_dtype)
    else:
        out = quant_matmul_raw(q, scale, linear, out_dtype)
    return out.reshape(*shape[:-1], linear.weight.shape[0])


def _device_arch(device: torch.device) -> str:
    props = torch.cuda.get_device_properties(device)
    return str(getattr(props, "gcnArchName", ""))


class Kernels:
    """Feature -> module implementing it, loaded once; None (and a recorded fallback) when the
    device is not a gfx950 HIP device, the feature is not built here, or the library is missing
    or fails to load."""

    SPECS = {
        "swiglu": ("swiglu_quant", "reuse"),
        "gate_residual": ("gate_residual", None),
        "norm_quant": ("nq2", True),
        "rope": None,
        "phaa_layout": None,
        "laser_preprocess": None,
        "merge_quant": None,
    }

    def __init__(self, diagnostics):
        self.diagnostics = diagnostics
        self.loaded = {}
        self.arch = {}

    def get(self, feature, value):
        """Only loading failures fall back; errors after kernel dispatch propagate."""
        device = str(value.device)
        if device not in self.arch:
            try:
                self.arch[device] = value.device.type == "cuda" and _device_arch(value.device).startswith(ARCH)
            except (AssertionError, RuntimeError):
                self.arch[device] = False
        if not self.arch[device]:
            self.diagnostics.fallback(feature, f"compiled kernel requires a {ARCH} (MI355X) HIP device")
            return None
        spec = self.SPECS[feature]
        if spec is None:
            self.diagnostics.fallback(feature, "not part of the W8A8 linear path built for MI355X")
            return None
        if feature not in self.loaded:
            module_name, argument = spec
            module = importlib.import_module("xgen_amd.operator." + module_name)
            path = module.library_path() if argument is None else module.library_path(argument)
            reason = None
            if not path.is_file():
                reason = f"library missing: {path.name}"
            else:
                try:
                    from .. import _native
                    _native.lib()
                except (OSError, RuntimeError) as error:
                    reason = f"library load failed: {type(error).__name__}: {error}"
            self.loaded[feature] = (module, reason)
        module, reason = self.loaded[feature]
        if reason:
            self.diagnostics.fallback(feature, reason)
            return None
        return module
