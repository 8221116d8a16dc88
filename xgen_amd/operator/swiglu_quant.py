"""SwiGLU + per-row quantization (H3's FFN activation and the requant before its
down-projection) on the HIP kernel.

Mirrors x_base/x_base/operator/npu_fusion/swiglu_quant.py: `swiglu_quantize`,
`swiglu_quantize_vector` and `swiglu_quantize_reuse` (three NPU implementations
of `torch.ops.h3_phaa_fusion_quant*.swiglu_quantize`, the last registered at
f1b/op_extension/swiglu_quant_reuse_queued.asc:33-35) take u bf16 [B, S, 2F]
laid out [hidden | gate] and return (int8 [B*S, F], float32 scale [B*S]);
ValueError for an input that requires grad, RuntimeError for contract
violations (quant_meta, swiglu_quant_reuse_queued.asc:10-17).  `tile` and
`blocks` are the NPU kernels' tiling knobs, validated and otherwise unused.

`swiglu_quant` is the general form: gate-first layout ([gate | hidden], as
x_base/x_base/operator/h3_swiglu.py packs it), FP8 or INT8 output, and the
bf16 activation itself on request.
"""
from __future__ import annotations

import torch

from .. import ops as _ops  # noqa: F401

xops = torch.ops.xgen_amd


def _checked(u, tile, blocks, scale_mode, tiles):
    if u.requires_grad:
        raise ValueError("Experimental inference-only F1b has no backward")
    if tile not in tiles:
        raise RuntimeError(f"tile must be {','.join(map(str, tiles))}")
    if not 0 < blocks <= 40 or scale_mode not in (0, 1):
        raise RuntimeError("invalid blocks/scale mode")
    q, s, _ = xops.swiglu_quant(u, False, torch.int8, scale_mode, False)
    return q, s


def swiglu_quantize(u, *, tile=2048, blocks=40, scale_mode=1):
    return _checked(u, tile, blocks, scale_mode, (1024, 2048, 4096))


def swiglu_quantize_vector(u, *, tile=2048, blocks=40, scale_mode=1):
    return _checked(u, tile, blocks, scale_mode, (1024, 2048, 4096))


def swiglu_quantize_reuse(u, *, tile=4096, blocks=40, scale_mode=1):
    return _checked(u, tile, blocks, scale_mode, (1024, 2048, 4096))


def swiglu_quant(u, *, gate_first=False, out_dtype=torch.int8, scale_mode=1, return_act=False):
    """(q [B*S, F], scale [B*S]) or, with return_act, (q, scale, bf16 activation [B*S, F])."""
    if u.requires_grad:
        raise ValueError("swiglu_quant is inference-only")
    q, s, act = xops.swiglu_quant(u, gate_first, out_dtype, scale_mode, return_act)
    return (q, s, act) if return_act else (q, s)
