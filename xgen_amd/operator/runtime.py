"""Dispatch support for the fused DiT block on the xgen_amd HIP library: which
fused features may run, bookkeeping of what ran, and the shared-activation GEMM.

The block forward of the reference imports these names from
x_base/x_base/operator/npu_fusion/runtime.py
(x_diffusers/x_diffusers/framework/transformer/h3_npu_fusion.py:18) and reads
the attributes below (h3_npu_fusion.py:196-273), so they keep that contract:

  Diagnostics   runtime.py:18-52   hits[feature], fallbacks[(feature, reason)],
                                   in_request, reset(), hit(), fallback() -> False,
                                   summary(phase) with keys phase / rank / hits /
                                   fallbacks[{feature, reason, count}]
  tensors_ok    runtime.py:55-60   inference-only tensors, one dtype, one device
  no_hooks      runtime.py:62-70   the hook attributes a fused path must not skip
  quant_linear  runtime.py:73-84   may this linear consume a shared (q, scale)?
  quant_matmul  runtime.py:87-91   GEMM of that shared quantized activation
  Kernels.get   runtime.py:94-140  module of a fused feature, or None with a
                                   recorded fallback when it cannot be loaded;
                                   errors after dispatch propagate

Features map onto this package's modules: "norm_quant" -> nq2, "swiglu" ->
swiglu_quant, "gate_residual" -> gate_residual, "merge_quant" -> merge_quant,
"phaa_layout" -> phaa_layout, all in libxgen_amd.so.  The reference's other
features (rope, laser preprocessing) are attention work outside the W8A8
linear path and always fall back.
"""
from __future__ import annotations

import importlib
import json
import logging
import os
from collections import Counter
from dataclasses import dataclass

import torch

from .h3_fp8 import H3FP8Linear
from .matmul import WeightQuantLinearModule, quant_matmul_raw

LOG = logging.getLogger("xgen.optim")
ARCH = "gfx950"


def configure_logging(level=None):
    """Leaves the "xgen.optim" logger to the application's logging setup; with `level`, sets
    only that logger's level."""
    if level is not None:
        LOG.setLevel(level)


def _rank() -> str:
    return os.environ.get("RANK", "0")


class Diagnostics:
    """Tally of fused-path outcomes for one inference request.

    Every outcome is a key: (feature, "enabled") for a hit, (feature, reason) for a
    fallback.  The first occurrence of a key is logged, later ones only counted.  A
    fallback noted while no request is open (in_request False: a capability probe at
    load time) is standing: it stays in `fallbacks` across reset(), so every request's
    summary reports it.  Hits and in-request fallbacks start from zero at reset().
    """

    def __init__(self, prefix="OP_OPT"):
        self.prefix = prefix
        self.in_request = False
        self._standing = Counter()
        self._logged = set()
        self.hits = Counter()
        self.fallbacks = Counter()
        self.reset()

    def reset(self):
        self.hits = Counter()
        self.fallbacks = Counter(self._standing)

    def _log_once(self, key, level, text):
        """Log `text` ("<outcome>=<feature> ...") the first time `key` occurs."""
        if key not in self._logged:
            self._logged.add(key)
            LOG.log(level, "[%s] %s rank=%s", self.prefix, text, _rank())

    def hit(self, feature, detail=""):
        self.hits[feature] += 1
        self._log_once((feature, "enabled"), logging.INFO, f"enabled={feature} {detail}".rstrip())

    def fallback(self, feature, reason):
        key = (feature, reason)
        self.fallbacks.update((key,))
        if not self.in_request:
            self._standing.update((key,))
        self._log_once(key, logging.WARNING, f"fallback={feature} reason={reason}")
        return False

    def summary(self, phase="request_end"):
        rows = [{"feature": feature, "reason": reason, "count": count}
                for (feature, reason), count in sorted(self.fallbacks.items())]
        report = {"phase": phase, "rank": _rank(), "hits": dict(self.hits), "fallbacks": rows}
        LOG.info("[%s] summary=%s", self.prefix, json.dumps(report, ensure_ascii=False, sort_keys=True))
        return report


def tensors_ok(*values, dtype=torch.bfloat16):
    """Inference-only tensors of `dtype`, all on one HIP device (torch's "cuda" type)."""
    if not values or torch.is_grad_enabled():
        return False
    device = values[0].device if isinstance(values[0], torch.Tensor) else None
    for x in values:
        if not isinstance(x, torch.Tensor) or x.device != device or x.device.type != "cuda":
            return False
        if x.dtype != dtype or x.requires_grad:
            return False
    return True


# Attributes through which offloading (accelerate, diffusers), adapters (PEFT / LoRA) and user
# hooks attach to a module (the reference's list, runtime.py:67-69).
_MODULE_HOOKS = ("_hf_hook", "_diffusers_hook", "_forward_hooks", "_forward_pre_hooks", "peft_config", "lora_A",
                 "lora_B")
_GLOBAL_HOOKS = ("_global_forward_hooks", "_global_forward_pre_hooks")


def _hooked(module) -> bool:
    registry = torch.nn.modules.module
    if any(getattr(registry, table, None) for table in _GLOBAL_HOOKS):
        return True
    if "forward" in module.__dict__:  # an instance-level forward replaces the class's
        return True
    return any(getattr(module, attr, None) for attr in _MODULE_HOOKS)


def no_hooks(module):
    """True when a fused path may skip `module`'s own forward: nothing is attached to it (see
    _MODULE_HOOKS), no global forward hooks are registered and forward is not overridden."""
    return not _hooked(module)


def _native_operands(module):
    """(weight, scale, weight dtype, accepted scale counts) of a linear that can take a shared
    per-token quantized activation, or None."""
    if type(module) is WeightQuantLinearModule:
        weight = getattr(module, "weight", None)
        counts = (weight.shape[0],) if isinstance(weight, torch.Tensor) and weight.ndim == 2 else ()
        return weight, getattr(module, "antiquant_scale", None), torch.int8, counts
    if type(module) is H3FP8Linear and getattr(module, "activation_scaling", None) == "token":
        weight = getattr(module, "weight", None)
        counts = (1, weight.shape[0]) if isinstance(weight, torch.Tensor) and weight.ndim == 2 else ()
        return weight, getattr(module, "weight_scale", None), torch.float8_e4m3fn, counts
    return None


def quant_linear(module, width=None, device=None):
    """Whether `module` can consume a (q, scale) quantized once and shared: the INT8 module (int8
    weight, float32 antiquant_scale [N]) or, here, the FP8 module with per-token activation
    scales (e4m3fn weight, float32 weight_scale [1] or [N]); no hooks; no input_activation (its
    input quantization applies a function the shared q does not carry); width and device as
    asked."""
    operands = _native_operands(module)
    if operands is None or getattr(module, "input_activation", None) is not None:
        return False
    weight, scale, wdtype, counts = operands
    if not isinstance(weight, torch.Tensor) or weight.dtype != wdtype or not counts:
        return False
    if not isinstance(scale, torch.Tensor) or scale.dtype != torch.float32 or scale.numel() not in counts:
        return False
    if width is not None and weight.shape[1] != width:
        return False
    if device is not None:
        bias = getattr(module, "bias", None)
        if weight.device != device or scale.device != device or (bias is not None and bias.device != device):
            return False
    return no_hooks(module)


def quant_matmul(q, scale, linear, shape, out_dtype=torch.bfloat16):
    """GEMM of a pre-quantized activation q [M,K] (+ per-token scale [M]) through `linear`,
    reshaped to [*shape[:-1], N].  q is the plain quantization of the input: a linear with an
    input_activation is refused (quant_linear is False for it)."""
    if getattr(linear, "input_activation", None) is not None:
        raise ValueError("quant_matmul: the linear applies an input_activation in its own input quantization; "
                         "call the module instead of sharing a plain (q, scale)")
    if type(linear) is H3FP8Linear:
        out = linear.forward_quantized(q.reshape(-1, q.shape[-1]), scale.reshape(-1), out_dtype)
    else:
        out = quant_matmul_raw(q, scale, linear, out_dtype)
    return out.reshape(*shape[:-1], linear.weight.shape[0])


@dataclass
class _Feature:
    module: str | None       # module under xgen_amd.operator, None: not built here
    argument: object = None  # passed to that module's library_path(), as the reference's specs do


class Kernels:
    """Feature -> the module implementing it.  A feature resolves once per instance; None (and
    a recorded fallback, every time it is asked for) when the device is not a gfx950 HIP device,
    the feature is not built here, or the library is missing or does not load."""

    SPECS = {
        "swiglu": ("swiglu_quant", "reuse"),
        "gate_residual": ("gate_residual", None),
        "norm_quant": ("nq2", True),
        "rope": None,
        "phaa_layout": ("phaa_layout", None),
        "laser_preprocess": None,
        "merge_quant": ("merge_quant", None),
    }

    def __init__(self, diagnostics):
        self.diagnostics = diagnostics
        self.loaded = {}   # feature -> (module or None, reason or None)
        self.arch = {}     # str(device) -> bool

    def _device_ok(self, device: torch.device) -> bool:
        key = str(device)
        if key not in self.arch:
            ok = False
            if device.type == "cuda":
                try:
                    ok = str(getattr(torch.cuda.get_device_properties(device), "gcnArchName", "")).startswith(ARCH)
                except (AssertionError, RuntimeError):
                    ok = False
            self.arch[key] = ok
        return self.arch[key]

    @staticmethod
    def _resolve(feature):
        spec = Kernels.SPECS[feature]
        if spec is None:
            return None, "not part of the W8A8 linear path built for MI355X"
        found = _Feature(*spec)
        module = importlib.import_module(f"xgen_amd.operator.{found.module}")
        path = module.library_path() if found.argument is None else module.library_path(found.argument)
        if not path.is_file():
            return None, f"library missing: {path.name}"
        from .. import _native
        try:
            _native.lib()
        except (OSError, RuntimeError) as error:
            return None, f"library load failed: {type(error).__name__}: {error}"
        return module, None

    def get(self, feature, value):
        """Only a device or loading problem falls back; errors raised by the module's kernels
        after dispatch reach the caller."""
        if not self._device_ok(value.device):
            self.diagnostics.fallback(feature, f"compiled kernel requires a {ARCH} (MI355X) HIP device")
            return None
        if feature not in self.loaded:
            self.loaded[feature] = self._resolve(feature)
        module, reason = self.loaded[feature]
        if module is None:
            self.diagnostics.fallback(feature, reason)
        return module
