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
bf16 activation itself on request.  `gate_first_swiglu(x, *, with_amax)` is
h3_swiglu.py:31-41's surface: the bf16 activation of a gate-first input and,
on request, its NaN-propagating max |value| as a float32 0-dim tensor.
"""
from __future__ import annotations

import torch

from .. import _native as N
from .. import ops as _ops  # noqa: F401

xops = torch.ops.xgen_amd


def library_path(implementation='scalar'):
    """The library holding the kernels (swiglu_quant.py:11-17 resolves one per implementation;
    all three are the one HIP library here, XGEN_AMD_LIBRARY overriding its location)."""
    if implementation not in ('scalar', 'vector', 'reuse'):
        raise KeyError(implementation)
    return N.library_path()


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


def gate_first_swiglu(x, *, with_amax=False):
    """x bf16 [..., 2F] laid out [gate | value] -> bf16(bf16(gate / (1 + exp(-gate))) * value)
    [..., F] (x_base/x_base/operator/h3_swiglu.py:15-41, eager bf16 rounding of the activation);
    with_amax also returns max |result| (NaN propagates) as a float32 0-dim tensor."""
    if x.requires_grad:
        raise ValueError("gate_first_swiglu is inference-only")
    if x.dtype != torch.bfloat16 or x.shape[-1] % 2:
        raise ValueError("gate_first_swiglu: BF16 input with an even last dimension required")
    lead, F = x.shape[:-1], x.shape[-1] // 2
    u = x.reshape(1, -1, 2 * F) if x.dim() != 3 else x
    _, _, act = xops.swiglu_quant(u, True, torch.float8_e4m3fn, 1, True)
    out = act.reshape(*lead, F)
    if with_amax:
        return out, xops.abs_peak(act)
    return out
