"""Quantized rows with their token scales and logical shape (x_base/x_base/operator/npu_fusion/quantized.py:6-9):
what merge_quant's caller hands the out-projection (x_base/x_base/phaa/fused_layout.py:47-48), consumed
by runtime.quant_matmul(value.q, value.scale, layer, value.shape)."""
from __future__ import annotations

from typing import NamedTuple

import torch


class QuantizedRows(NamedTuple):
    q: torch.Tensor
    scale: torch.Tensor
    shape: tuple
