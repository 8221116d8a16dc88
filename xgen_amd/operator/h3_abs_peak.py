"""Absolute peak of an activation tensor (activation_abs_peak,
x_base/x_base/operator/h3_abs_peak.py:21-25), on the xgen_amd HIP kernels."""
import torch

from ..ops import xops


def activation_abs_peak(x: torch.Tensor) -> torch.Tensor:
    """NaN-propagating max |x| over a BF16/F16 CUDA tensor, as a float32 0-dim tensor."""
    return xops.abs_peak(x)
