"""Fused norm + AdaLN-table modulation + per-token quantization.

Reference surface: norm_affine_quant(x, weight, scale, shift, indices, *, eps=1e-5,
blocks=40, cached=False) -> (q, token_scale)  (x_base/x_base/operator/npu_fusion/nq2.py:18-26),
op torch.ops.h3_phaa_nq2.fused (npu_fusion/f2_nq2/op_extension/nq2_queued.asc:53-61).

Extensions for the DiT linear path: ``norm="layer"`` (LayerNorm without
affine, hunyuan.py:359) besides the reference's RMSNorm, ``out_dtype``
float8_e4m3fn besides int8, ``weight=None`` for a norm without affine, and
``return_normed`` to also return the pre-quantization bf16 rows (the
reference kernel's debug output, f2bc_kernel.asc:86), and
``scale_is_one_plus`` when ``scale`` already holds bf16(1 + scale)
(``adaln_one_plus``: prepared once per table instead of once per token, the
same values).  ``blocks`` and ``cached`` are accepted for signature
compatibility; the HIP kernel sizes its own grid and reads table rows
through L2.
"""
from __future__ import annotations

import torch

from .. import _native as N
from ..ops import xops

_NORMS = {"rms": N.NORM_RMS, "layer": N.NORM_LAYER}


def library_path(cached=False):
    """The library holding the kernel (nq2.py:10-15 resolves one per `cached` variant; both
    variants are the one HIP library here, XGEN_AMD_LIBRARY overriding its location)."""
    return N.library_path()


def norm_affine_quant(x, weight, scale, shift, indices, *, eps=1e-5, blocks=40, cached=False,
                      norm="rms", out_dtype=torch.int8, return_normed=False, scale_is_one_plus=False):
    if any(v is not None and v.requires_grad for v in (x, weight, scale, shift)):
        raise ValueError('Experimental inference only; detach parameters explicitly')
    if norm not in _NORMS:
        raise ValueError(f"norm must be one of {sorted(_NORMS)}")
    if not (0 < blocks <= 40):
        raise RuntimeError("invalid epsilon/blocks")
    kind = _NORMS[norm] | (N.NORM_SCALE_ONE_PLUS if scale_is_one_plus else 0)
    q, s, normed = xops.norm_affine_quant(x, weight, scale, shift, indices, float(eps), kind,
                                          out_dtype, bool(return_normed))
    return (q, s, normed) if return_normed else (q, s)


def adaln_one_plus(scale: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(1 + scale) of a BF16 [T, H] table (unit last stride) on the GPU — the eager
    modulation's `1.0 + scale` (h3_indexed_affine.py:22-28), prepared once per table for
    norm_affine_quant(..., scale_is_one_plus=True)."""
    if scale.dim() != 2 or scale.dtype != torch.bfloat16 or scale.stride(1) != 1 or scale.device.type != "cuda":
        raise ValueError("adaln_one_plus: a BF16 CUDA table [T, H] with unit last stride is required")
    if out is None:
        out = torch.empty(scale.shape, dtype=torch.bfloat16, device=scale.device)
    elif out.shape != scale.shape or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError("adaln_one_plus: out must be a BF16 [T, H] tensor with unit last stride")
    st = N.lib().xgen_adaln_one_plus(scale.data_ptr(), scale.shape[0], scale.shape[1], scale.stride(0),
                                     out.data_ptr(), out.stride(0), N.stream_of(scale))
    N.check(st, "xgen_adaln_one_plus")
    return out
