"""FP8 activation quantizers (x_base/x_base/operator/h3_fp8_quant.py:18-25) on the
xgen_amd HIP kernels.

quantize_activation keeps the reference's per-tensor contract:
    scale = max(abs_peak(x) / 448, FLT_MIN)      (optionally all-reduced with MAX)
    q     = e4m3fn(clamp(x / scale, -448, 448))  (correctly rounded division, RNE)
quantize_activation_rows is the per-token form the W8A8 path uses (same
arithmetic per row, one float32 scale per row).
"""
import torch

from ..ops import xops


def quantize_activation(x: torch.Tensor, group=None):
    """Per-tensor FP8 quantization -> (e4m3fn tensor shaped like x, float32 0-dim scale)."""
    scale = xops.fp8_tensor_scale(x)
    if group is not None:
        import torch.distributed as dist
        dist.all_reduce(scale, op=dist.ReduceOp.MAX, group=group)
    return xops.fp8_pack(x, scale), scale


def quantize_activation_rows(x: torch.Tensor):
    """Per-token FP8 quantization of [..., K] -> (e4m3fn like x, float32 [numel // K])."""
    return xops.quantize_rows(x, torch.float8_e4m3fn)
