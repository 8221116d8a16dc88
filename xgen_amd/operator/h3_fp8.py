"""FP8 W8A8 projection with the reference module surface, on gfx950 MFMA.

Mirrors x_base/x_base/operator/h3_fp8.py:
  * quantize_per_tensor(value)           h3_fp8.py:9-12
  * H3FP8Linear(weight, bias=None)       h3_fp8.py:15-27  (buffers weight / weight_scale / bias, calls)
  * H3FP8Linear.from_packed(w, s, bias)  h3_fp8.py:29-43
  * H3FP8Linear.forward / _local_forward h3_fp8.py:45-68

Default scaling is the reference's: one weight scale and one activation scale
per call.  ``weight_scaling="channel"`` keeps one scale per output feature
(quantize_per_tensor's arithmetic per row) and ``activation_scaling="token"``
one scale per token: the W8A8 layout of the DiT linear path.  The GEMM and its
dequant / bias / optional GELU-tanh epilogue are one HIP kernel; rows need no
padding to 16 (the reference pads, h3_fp8.py:58-59).

``accumulation`` picks how the K sums are formed.  "exact" (default) multiplies
the e4m3fn bytes exactly on the bf16 MFMA and sums in fp32: the accumulation
the reference requests with use_fast_accum=False (h3_fp8.py:63-66), at about
twice the matrix-core time.  "mfma" is the opt-in fast sum, the counterpart of
use_fast_accum=True: gfx950's FP8 MFMA, whose sum truncates each product of a
group of 8 consecutive K to a multiple of 2^(E - 13), E the group's largest
exponent sum.  One linear's bf16 output then sits at rel-L2 ~4e-4 of the
exactly summed result; a chain of per-token requantizations amplifies that
(DiTLinearChain picks the kind per projection).
"""
from __future__ import annotations

import torch
from torch import nn

from .. import _native as N
from ..ops import xops
from .h3_fp8_quant import quantize_activation, quantize_activation_rows

_FP8_MAX = 448.0
_ACTIVATIONS = {None: N.ACT_NONE, "none": N.ACT_NONE, "gelu_tanh": N.ACT_GELU_TANH}
_ACCUMULATIONS = ("mfma", "exact")


def _device_weight(value: torch.Tensor) -> torch.Tensor:
    """The weight on a HIP device, where the quantizer kernels run (a CPU weight is copied there)."""
    if value.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("xgen_amd FP8 weight quantization requires a BF16/FP16 weight")
    if not value.is_cuda:
        if not torch.cuda.is_available():
            raise RuntimeError("xgen_amd FP8 weight quantization requires a HIP device")
        value = value.cuda()
    return value.detach().contiguous()


def _on(device, *tensors):
    return tuple(t.to(device) for t in tensors)


def quantize_per_tensor(value: torch.Tensor):
    """(e4m3fn tensor, float32 0-dim scale) with scale = max(amax/448, FLT_MIN) (h3_fp8.py:9-12),
    on the device `value` is on (quantized by the HIP kernels)."""
    return _on(value.device, *quantize_activation(_device_weight(value)))


def quantize_per_channel(value: torch.Tensor):
    """quantize_per_tensor's arithmetic applied to each row of a 2-D weight:
    (e4m3fn [N,K], float32 [N]), on the device `value` is on."""
    if value.ndim != 2:
        raise ValueError("per-channel quantization requires a 2-D weight")
    return _on(value.device, *quantize_activation_rows(_device_weight(value)))


def _check_input_activation(input_activation, activation_scaling):
    if input_activation not in (None, "gelu_tanh"):
        raise ValueError(f"unsupported input_activation {input_activation!r}")
    if input_activation is not None and activation_scaling != "token":
        raise ValueError("input_activation needs activation_scaling='token'")


class H3FP8Linear(nn.Module):
    """Keep FP8 weights; quantize activations to E4M3 and run the W8A8 GEMM (exact products summed
    in fp32 by default, or the FP8 MFMA's sum)."""

    def __init__(self, weight, bias=None, *, weight_scaling: str = "tensor",
                 activation_scaling: str = "tensor", activation: str | None = None, accumulation: str = "exact",
                 input_activation: str | None = None):
        super().__init__()
        if weight.ndim != 2 or weight.shape[0] % 16 or weight.shape[1] % 16:
            raise ValueError("H3 FP8 requires projection dimensions divisible by 16")
        if weight_scaling not in ("tensor", "channel") or activation_scaling not in ("tensor", "token"):
            raise ValueError("weight_scaling must be 'tensor'|'channel', activation_scaling 'tensor'|'token'")
        if activation not in _ACTIVATIONS:
            raise ValueError(f"unsupported activation {activation!r}")
        if accumulation not in _ACCUMULATIONS:
            raise ValueError(f"accumulation must be one of {_ACCUMULATIONS}")
        _check_input_activation(input_activation, activation_scaling)
        self.out_features, self.in_features = weight.shape
        packed, scale = (quantize_per_tensor(weight) if weight_scaling == "tensor"
                         else quantize_per_channel(weight))
        self.register_buffer('weight', packed.contiguous())
        self.register_buffer('weight_scale', scale.reshape(-1) if weight_scaling == "channel" else scale)
        # buffers stay on the weight's device, as the reference's (h3_fp8.py:22-25)
        self.register_buffer('bias', bias.detach().clone() if bias is not None else None)
        self.activation_scaling = activation_scaling
        self.activation = activation
        self.input_activation = input_activation
        self.accumulation = accumulation
        self.calls = 0

    @classmethod
    def from_packed(cls, weight, scale, bias=None, *, activation_scaling: str = "tensor",
                    activation: str | None = None, accumulation: str = "exact", input_activation: str | None = None):
        """Reuse already quantized bytes and their original scale(s) without requantization."""
        if weight.dtype != torch.float8_e4m3fn or weight.ndim != 2 or any(n % 16 for n in weight.shape):
            raise ValueError('Packed H3 FP8 projection requires an aligned E4M3 matrix')
        if scale.dtype != torch.float32 or scale.numel() not in (1, weight.shape[0]):
            raise ValueError('Packed H3 FP8 projection requires one FP32 weight scale (or one per row)')
        if activation_scaling not in ("tensor", "token") or activation not in _ACTIVATIONS \
                or accumulation not in _ACCUMULATIONS:
            raise ValueError("bad activation_scaling / activation / accumulation")
        _check_input_activation(input_activation, activation_scaling)
        result = cls.__new__(cls)
        nn.Module.__init__(result)
        result.out_features, result.in_features = weight.shape
        result.register_buffer('weight', weight.contiguous())
        result.register_buffer('weight_scale', scale.detach().clone())
        result.register_buffer('bias', bias.detach().clone() if bias is not None else None)
        result.activation_scaling = activation_scaling
        result.activation = activation
        result.input_activation = input_activation
        result.accumulation = accumulation
        result.calls = 0
        return result

    def forward(self, x):
        return self._local_forward(x, self.bias)

    def quantize_input(self, matrix):
        """(e4m3fn [M,K], float32 scale [1] or [M]) for a [M,K] activation; with
        input_activation='gelu_tanh' the rows quantized are dtype(gelu_tanh(matrix)), computed in the
        quantizer's pass (the bytes and scales of the previous linear's GELU epilogue followed by
        this quantization, hunyuan.py:358)."""
        if self.activation_scaling == "token":
            if getattr(self, 'input_activation', None) is not None:
                return xops.quantize_rows(matrix, torch.float8_e4m3fn, _ACTIVATIONS[self.input_activation])
            return quantize_activation_rows(matrix)
        group = getattr(self, 'activation_group', None)
        packed, scale = quantize_activation(matrix, group=group)
        return packed, scale.reshape(1)

    def forward_quantized(self, packed, scale, out_dtype=torch.bfloat16, activation=None):
        """GEMM on an already quantized activation (shared-QKV pattern,
        x_diffusers/x_diffusers/framework/transformer/h3_npu_fusion.py:103-119).  input_activation
        does not apply here: it acts where this module quantizes its own input (quantize_input)."""
        act = _ACTIVATIONS[activation if activation is not None else self.activation]
        out, _ = xops.scaled_mm(packed, self.weight, scale, self.weight_scale.reshape(-1), self.bias,
                                out_dtype, act, False, self.accumulation == "exact")
        self.calls += 1
        return out

    def forward_gate_residual(self, x, residual, gate_table, indices):
        """`residual + bf16(gate_table[indices] * self(x))` with the gated residual in the GEMM's
        epilogue (the out-projection / FFN-down of a DiT block followed by
        x_base/x_base/operator/h3_indexed_affine.py:58-61).  x: bf16/fp16 [B, S, K]; residual bf16
        [B, S, N]; gate_table bf16 [T, N]; indices int64 [S].  Per-token activation scaling only.
        The FP8 MFMA kind runs it as one kernel; the exact kind as its GEMM followed by the
        gated residual kernel (the same bytes as a fused form would give)."""
        if self.activation_scaling != "token" or _ACTIVATIONS[self.activation] != N.ACT_NONE:
            raise ValueError("forward_gate_residual needs activation_scaling='token' and no activation")
        if x.dim() != 3 or residual.shape != (*x.shape[:-1], self.out_features):
            raise ValueError("forward_gate_residual: x [B,S,K] and residual [B,S,N] required")
        packed, scale = self.quantize_input(x.reshape(-1, x.shape[-1]))
        if self.accumulation == "exact":
            branch, _ = xops.scaled_mm(packed, self.weight, scale, self.weight_scale.reshape(-1), self.bias,
                                       torch.bfloat16, N.ACT_NONE, False, True)
            out = xops.gate_residual(residual, branch.reshape(residual.shape), gate_table, indices)
        else:
            out = xops.scaled_mm_gate_residual(packed, self.weight, scale, self.weight_scale.reshape(-1), self.bias,
                                               residual.reshape(-1, self.out_features), gate_table, indices)
        self.calls += 1
        return out.reshape(residual.shape)

    def _local_forward(self, x, bias):
        if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("H3 FP8 Linear requires CUDA BF16/FP16 input")
        if x.shape[-1] != self.in_features:
            raise ValueError("H3 FP8 Linear input width does not match its weight")
        matrix = x.reshape(-1, self.in_features)
        if not matrix.shape[0]:
            return x.new_empty((*x.shape[:-1], self.out_features))
        packed, scale = self.quantize_input(matrix)
        output, _ = xops.scaled_mm(packed, self.weight, scale, self.weight_scale.reshape(-1), bias, x.dtype,
                                   _ACTIVATIONS[self.activation], False, self.accumulation == "exact")
        self.calls += 1
        return output.reshape(*x.shape[:-1], self.out_features)

    def extra_repr(self):
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"weight_scale={tuple(self.weight_scale.shape)}, activation_scaling={self.activation_scaling}, "
                f"activation={self.activation}, input_activation={getattr(self, 'input_activation', None)}, "
                f"accumulation={self.accumulation}")
