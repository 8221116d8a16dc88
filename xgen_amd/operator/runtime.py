"""Gate and GEMM helpers for pre-quantized activations.

quant_linear mirrors x_base/x_base/operator/npu_fusion/runtime.py:73-84 (is this
module a native W8A8 linear that can consume a shared (q, scale)?), quant_matmul
mirrors runtime.py:87-91.  Both accept the INT8 WeightQuantLinearModule and the
FP8 H3FP8Linear (per-token activation scaling).
"""
from __future__ import annotations

import torch

from .h3_fp8 import H3FP8Linear
from .matmul import WeightQuantLinearModule, quant_matmul_raw


def quant_linear(module, width=None, device=None):
    weight = getattr(module, "weight", None)
    bias = getattr(module, "bias", None)
    if type(module) is WeightQuantLinearModule:
        scale = getattr(module, "antiquant_scale", None)
        wdtype = torch.int8
    elif type(module) is H3FP8Linear:
        scale = getattr(module, "weight_scale", None)
        wdtype = torch.float8_e4m3fn
        if module.activation_scaling != "token":
            return False
    else:
        return False
    return (isinstance(weight, torch.Tensor) and weight.ndim == 2 and weight.dtype == wdtype
            and isinstance(scale, torch.Tensor) and scale.dtype == torch.float32
            and scale.numel() in ((weight.shape[0],) if wdtype == torch.int8 else (1, weight.shape[0]))
            and (width is None or weight.shape[1] == width)
            and (device is None or weight.device == scale.device == device)
            and (bias is None or device is None or bias.device == device)
            and not module._forward_hooks and not module._forward_pre_hooks)


def quant_matmul(q, scale, linear, shape, out_dtype=torch.bfloat16):
    """GEMM of a pre-quantized activation q [M,K] (+ per-token scale [M]) through linear,
    reshaped to [*shape[:-1], N]."""
    if type(linear) is H3FP8Linear:
        out = linear.forward_quantized(q.reshape(-1, q.shape[-1]), scale.reshape(-1), out_dtype)
    else:
        out = quant_matmul_raw(q, scale, linear, out_dtype)
    return out.reshape(*shape[:-1], linear.weight.shape[0])
