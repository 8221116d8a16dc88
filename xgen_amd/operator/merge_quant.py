"""Merge of the head-parallel attention's returned chunks + per-token quantization, on the HIP kernel.

Mirrors x_base/x_base/operator/npu_fusion/merge_quant.py:9-14 (the
`torch.ops.h3_phaa_merge_quant.fused` op of f4_merge_quant/op_extension/merge_quant_queued.asc:9-28):
`merge_quant(back_recv, *, blocks=40) -> (q, scale)` takes the all-to-all's returned attention
chunks, BF16 [7, 4, S, 1, 256] contiguous ([splits, owners, seq, batch, chunk]: H3's 56 heads x
128 as 4 owners x 7 chunks of 2 heads), and returns the out-projection's input rows quantized per
token: int8 [S, 7168] (owner-major, chunk-minor columns) and float32 scales [S], which
x_base/x_base/phaa/fused_layout.py:44-48 wraps as QuantizedRows for `quant_matmul`.  ValueError
for a tensor that requires grad, RuntimeError with the reference's messages for its schema
checks (merge_quant_queued.asc:10-13).  `blocks` is the NPU kernel's grid size, validated and
otherwise unused: the HIP kernel sizes its own grid.  `out_dtype=torch.float8_e4m3fn` quantizes
with the FP8 row quantizer instead (the FP8 out-projection's input), an extension.  Other
geometries (any splits / owners / batch, chunk a multiple of 8, rows up to 16,384 values) are
`torch.ops.xgen_amd.merge_quant`.
"""
from __future__ import annotations

import torch

from .. import _native as N
from .. import ops as _ops  # noqa: F401  (registers torch.ops.xgen_amd)
from .quantized import QuantizedRows  # noqa: F401  (the wrapper its callers build)

xops = torch.ops.xgen_amd

MERGE_MAX_SEQUENCE = 1 << 20  # the reference's DataCopy stride limit (capabilities.py:15)


def library_path():
    """The library holding the kernel (merge_quant.py:7-8; XGEN_AMD_LIBRARY overrides it)."""
    return N.library_path()


def check_back_recv(back_recv, blocks):
    """The reference op's schema checks, in its order and with its messages (merge_quant_queued.asc:10-13)."""
    if not (back_recv.dim() == 5 and tuple(back_recv.shape[:2]) == (7, 4) and back_recv.shape[3] == 1
            and back_recv.shape[4] == 256):
        raise RuntimeError("[7,4,S,1,256] required")
    if not (back_recv.dtype == torch.bfloat16 and back_recv.is_contiguous()):
        raise RuntimeError("contiguous BF16 required")
    if back_recv.shape[2] > MERGE_MAX_SEQUENCE:
        raise RuntimeError("S exceeds DataCopy stride contract")
    if not 0 < blocks <= 40:
        raise RuntimeError("blocks must be 1..40")


def merge_quant(back_recv, *, blocks=40, out_dtype=torch.int8):
    if back_recv.requires_grad:
        raise ValueError("Inference only; no backward")
    check_back_recv(back_recv, blocks)
    return xops.merge_quant(back_recv, out_dtype)
