"""Indexed gated residual, `residual + bf16(gate[indices] * branch)`, on the HIP kernels.

Mirrors x_base/x_base/operator/npu_fusion/gate_residual.py:9-14 (the
`torch.ops.h3_phaa_gate_residual.gate_residual` op of
f2a/op_extension/gate_residual_queued.asc:33-35): same arguments, BF16
[B, S, H] residual and branch, BF16 [T, H] gate table, int64 [S] indices, a
new BF16 [B, S, H] output; ValueError for tensors that require grad,
RuntimeError for contract violations.  `tile` and `blocks` are the NPU
kernel's tiling knobs, validated as the reference's schema does
(gate_residual_queued.asc:16-17) and otherwise unused: the HIP kernel sizes its
own grid.
"""
from __future__ import annotations

import torch

from .. import _native as N
from .. import ops as _ops  # noqa: F401  (registers torch.ops.xgen_amd)

xops = torch.ops.xgen_amd


def library_path():
    """The library holding the kernel (gate_residual.py:7-8; XGEN_AMD_LIBRARY overrides it)."""
    return N.library_path()


def gate_residual(residual, branch, gate_table, indices, *, tile=5376, blocks=40):
    if any(t.requires_grad for t in (residual, branch, gate_table)):
        raise ValueError("Experimental inference-only gate_residual has no backward")
    if tile not in (1024, 2048, 4096, 5376):
        raise RuntimeError("tile must be 1024/2048/4096/5376")
    if not 0 < blocks <= 40:
        raise RuntimeError("blocks must be 1..40")
    return xops.gate_residual(residual, branch, gate_table, indices)
