"""INT8 W8A8 projection with the reference module surface, on gfx950 MFMA.

Mirrors x_base/x_base/operator/matmul.py:
  * WeightQuantLinearModule(weight, bias, name=None)           matmul.py:36-50
      per-output-row symmetric int8 weight + float32 antiquant_scale [N]
  * WeightQuantLinearModule.forward(x)                         matmul.py:52-66
      fp32 input cast to bf16; per-token int8 quantization; int8 GEMM with exact
      int32 accumulation; dequant acc * pertoken_scale * antiquant_scale + bias
  * enable_weight_quant_linear(model, quant_config, dtype)     matmul.py:141-202
  * MatmulManager.enable_online_dynamic_quant / matmul_manager  matmul.py:300-348, 423
      the installer --matmul_quant int8 calls (x_diffusers/x_diffusers/adaptor/load_pipe.py:555-558)
      and the name x_base/x_base/operator/__init__.py:2 imports

Extension: ``input_activation="gelu_tanh"`` quantizes int8(gelu_tanh(x)) per row in the
quantizer's pass (the FFN-down input of a GELU FeedForward, hunyuan.py:358): the bytes and
scales of the up projection's GELU epilogue followed by the plain quantization.

The quantizer is the one the reference restates for the NPU path
(npu_fusion/f2bc/op_kernel/f2bc_kernel.asc:89-107): scale = amax * fl(1/127),
q = rint_half_even(x * fl(127/amax)); a zero row gives zeros and scale 0.
"""
from __future__ import annotations

import gc
import logging

import torch
from torch import nn

from .. import _native as N
from ..config import QuantLayerConfig, detect_config_name, get_config
from ..ops import xops

LOG = logging.getLogger(__name__)


def dynamic_quant(x: torch.Tensor):
    """Per-row symmetric int8 quantization of [..., K] -> (int8 like x, float32 [rows])
    (the role of torch_npu.npu_dynamic_quant, matmul.py:39,60)."""
    return xops.quantize_rows(x, torch.int8)


class WeightQuantLinearModule(nn.Module):
    """Parameters are quantized on the HIP device and then kept on the CPU, as the reference's
    (matmul.py:39-48: quantize on the accelerator, copy to CPU to lower its peak memory); the
    model is moved to its device afterwards."""

    def __init__(self, weight, bias, name=None, *, input_activation=None):
        super().__init__()
        if input_activation not in (None, "gelu_tanh"):
            raise ValueError(f"unsupported input_activation {input_activation!r}")
        self.input_activation = input_activation
        w = weight.detach()
        if w.ndim != 2:
            raise ValueError("WeightQuantLinearModule requires a 2-D weight")
        if w.dtype == torch.float32:
            w = w.to(torch.bfloat16)
        if not w.is_cuda:
            if not torch.cuda.is_available():
                raise RuntimeError("xgen_amd INT8 weight quantization requires a HIP device")
            w = w.cuda()
        quant_weight, weight_scale = dynamic_quant(w.contiguous())
        w_cpu, scale_cpu = quant_weight.cpu(), weight_scale.cpu()
        del quant_weight, weight_scale
        self.register_parameter('weight', nn.Parameter(w_cpu, requires_grad=False))
        self.register_parameter('antiquant_scale', nn.Parameter(scale_cpu, requires_grad=False))
        if bias is not None:
            self.register_parameter('bias', nn.Parameter(bias.detach().cpu(), requires_grad=False))
        else:
            self.register_parameter('bias', None)
        self.out_features, self.in_features = w_cpu.shape
        self.name = name

    def forward(self, x):
        ori_shape = x.shape
        ori_dtype = x.dtype
        x = x.reshape(-1, ori_shape[-1])
        # the quantizer takes BF16/FP16 (as npu_dynamic_quant): FP32 is cast to BF16
        if x.dtype == torch.float32:
            x = x.to(torch.bfloat16)
            ori_dtype = torch.bfloat16
        x_int8, pertoken_scale = self.quantize_input(x)
        out = quant_matmul_raw(x_int8, pertoken_scale, self, ori_dtype)
        return out.reshape(*ori_shape[:-1], -1)

    def quantize_input(self, matrix):
        """(int8 [M,K], float32 [M]) for a bf16/fp16 [M,K] activation; of gelu_tanh(matrix) with
        input_activation='gelu_tanh'."""
        if getattr(self, 'input_activation', None) == "gelu_tanh":
            return xops.quantize_rows(matrix, torch.int8, N.ACT_GELU_TANH)
        return dynamic_quant(matrix)

    def forward_gate_residual(self, x, residual, gate_table, indices):
        """`residual + bf16(gate_table[indices] * self(x))` with the gated residual in the INT8 GEMM's
        epilogue (x_base/x_base/operator/npu_fusion/gate_residual.py:9-14 after npu_quant_matmul).
        x: [B, S, K]; residual bf16 [B, S, N]; gate_table bf16 [T, N]; indices int64 [S]."""
        if x.dim() != 3 or residual.shape != (*x.shape[:-1], self.weight.shape[0]):
            raise ValueError("forward_gate_residual: x [B,S,K] and residual [B,S,N] required")
        m = x.reshape(-1, x.shape[-1])
        if m.dtype == torch.float32:
            m = m.to(torch.bfloat16)
        q, s = self.quantize_input(m)
        out = xops.scaled_mm_gate_residual(q, self.weight, s.reshape(-1), self.antiquant_scale.reshape(-1), self.bias,
                                           residual.reshape(-1, residual.shape[-1]), gate_table, indices)
        return out.reshape(residual.shape)


def quant_matmul_raw(q, scale, linear, out_dtype=torch.bfloat16, activation=N.ACT_NONE):
    """int8 GEMM of a pre-quantized activation against a WeightQuantLinearModule."""
    out, _ = xops.scaled_mm(q.reshape(-1, q.shape[-1]), linear.weight, scale.reshape(-1),
                            linear.antiquant_scale.reshape(-1), linear.bias, out_dtype, activation, False)
    return out


def enable_weight_quant_linear(model: nn.Module, quant_config: QuantLayerConfig, dtype: str = 'w8a8') -> nn.Module:
    """Replace every selected nn.Linear by a WeightQuantLinearModule (matmul.py:141-202).

    Selection is quant_config.should_quantize(name, layer); layers whose weight
    was released are skipped; LoRA '.base_layer' suffixes are undone in the
    replacement name.  Only W8A8 is provided (the reference's transformer path
    builds the W8A8 module for every CLI value, matmul.py:183).
    """
    if dtype != 'w8a8':
        raise ValueError("xgen_amd provides the W8A8 module only")
    for name, layer in list(model.named_modules()):
        if not quant_config.should_quantize(name, layer):
            continue
        if getattr(layer, 'weight', None) is None:
            continue
        clean_name = name.replace(".base_layer", "")
        bias = layer.bias.data if getattr(layer, 'bias', None) is not None else None
        quant_module = WeightQuantLinearModule(layer.weight.data, bias, clean_name)
        if '.' in clean_name:
            parent, leaf = clean_name.rsplit('.', 1)
            setattr(model.get_submodule(parent), leaf, quant_module)
        else:
            setattr(model, clean_name, quant_module)
    return model


def _rank() -> int:
    dist = torch.distributed
    return dist.get_rank() if dist.is_available() and dist.is_initialized() else 0


class MatmulManager:
    """The quantization installer object of the reference's pipelines (matmul.py:300-423).

    Only the transformer's W8A8 linears are this path: the VAE installers of the reference
    (Conv3D through closed NPU operators, the VAE decoder's linears) are not provided and say
    so when called."""

    def enable_online_dynamic_quant(self, transformer, quant_config: QuantLayerConfig | None = None,
                                    dtype: str = 'w8a8'):
        """Swap the selected nn.Linear layers of `transformer` for WeightQuantLinearModule in place
        and return it.  quant_config None: the model's own rule set, chosen from its class
        (xgen_amd.config.detect_config_name).  As in the reference, any failure surfaces as
        ValueError (the cause chained) after being logged."""
        rank = _rank()
        try:
            if quant_config is None:
                name = detect_config_name(transformer)
                quant_config = get_config(name)
                LOG.info("rank %d: quant config %r detected for %s", rank, name, type(transformer).__name__)
            LOG.info("rank %d: replacing linears by W8A8 modules", rank)
            model = enable_weight_quant_linear(transformer, quant_config, dtype=dtype)
            gc.collect()
            if torch.cuda.is_available():
                torch.cuda.empty_cache()
        except Exception as error:
            LOG.error("W8A8 installation failed: %s", error)
            raise ValueError("Dynamic weight modify model failed. Please try running the program again.") from error
        LOG.info("rank %d: W8A8 linears installed", rank)
        return model

    def enable_vae_conv3d_quant(self, vae):
        raise NotImplementedError("xgen_amd: VAE Conv3D quantization is outside the W8A8 DiT linear path")

    def enable_vae_linear_quant(self, vae, dtype='int8'):
        raise NotImplementedError("xgen_amd: VAE linear quantization is outside the W8A8 DiT linear path")


matmul_manager = MatmulManager()
