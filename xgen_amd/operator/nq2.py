"""Fused norm + AdaLN-table modulation + per-token quantization.

Reference surface: norm_affine_quant(x, weight, scale, shift, indices, *, eps=1e-5,
blocks=40, cached=False) -> (q, token_scale)  (x_base/x_base/operator/npu_fusion/nq2.py:18-26),
op torch.ops.h3_phaa_nq2.fused (npu_fusion/f2_nq2/op_extension/nq2_queued.asc:53-61).

Extensions for the DiT linear path: ``norm="layer"`` (LayerNorm without
affine, hunyuan.py:359) besides the reference's RMSNorm, ``out_dtype``
float8_e4m3fn besides int8, ``weight=None`` for a norm without affine, and
``return_normed`` to also return the pre-quantization bf16 rows (the
reference kernel's debug output, f2bc_kernel.asc:86).  ``blocks`` and
``cached`` are accepted for signature compatibility; the HIP kernel sizes its
own grid (one wave per row) and reads table rows through L2.
"""
from __future__ import annotations

import torch

from .. import _native as N
from ..ops import xops

_NORMS = {"rms": N.NORM_RMS, "layer": N.NORM_LAYER}


def norm_affine_quant(x, weight, scale, shift, indices, *, eps=1e-5, blocks=40, cached=False,
                      norm="rms", out_dtype=torch.int8, return_normed=False):
    if any(v is not None and v.requires_grad for v in (x, weight, scale, shift)):
        raise ValueError('Experimental inference only; detach parameters explicitly')
    if norm not in _NORMS:
        raise ValueError(f"norm must be one of {sorted(_NORMS)}")
    if not (0 < blocks <= 40):
        raise RuntimeError("invalid epsilon/blocks")
    q, s, normed = xops.norm_affine_quant(x, weight, scale, shift, indices, float(eps), _NORMS[norm],
                                          out_dtype, bool(return_normed))
    return (q, s, normed) if return_normed else (q, s)
