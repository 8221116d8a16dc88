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

A holder of scale tables (the AdaLN loader) can register bf16(1 + scale) for
a table it keeps (``register_one_plus``): a call given that table itself —
the same memory, shape and strides, not written since (its version counter)
— then reads the prepared table, as the reference's callers pass the raw one.
A table written after it was prepared is prepared again on its next use; calls
captured into a HIP graph read the table they are given.
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


# registered tables: key of the raw scale table -> [raw table, prepared table, raw version when prepared]
_ONE_PLUS: dict = {}
prepared_hits = 0  # calls that read a registered prepared table


def _table_key(t: torch.Tensor):
    return (t.device.type, t.device.index, t.data_ptr(), tuple(t.shape), tuple(t.stride()))


def register_one_plus(scale: torch.Tensor, prepared: torch.Tensor) -> None:
    """Have norm_affine_quant read `prepared` (= adaln_one_plus(scale), same shape) when it is given
    `scale` itself; the registry keeps both tensors until unregister_one_plus(scale)."""
    if prepared.shape != scale.shape or prepared.dtype != torch.bfloat16 or prepared.device != scale.device:
        raise ValueError("register_one_plus: the prepared table must match the scale table")
    _ONE_PLUS[_table_key(scale)] = [scale, prepared, scale._version]


def unregister_one_plus(scale: torch.Tensor) -> None:
    _ONE_PLUS.pop(_table_key(scale), None)


def _registered_one_plus(scale: torch.Tensor):
    """The prepared table registered for `scale` (re-prepared if `scale` was written since), or None."""
    entry = _ONE_PLUS.get(_table_key(scale)) if _ONE_PLUS else None
    if entry is None or entry[0].untyped_storage().data_ptr() != scale.untyped_storage().data_ptr():
        return None
    if scale._version != entry[2]:
        adaln_one_plus(scale, entry[1])
        entry[2] = scale._version
    return entry[1]


def norm_affine_quant(x, weight, scale, shift, indices, *, eps=1e-5, blocks=40, cached=False,
                      norm="rms", out_dtype=torch.int8, return_normed=False, scale_is_one_plus=False):
    global prepared_hits
    if any(v is not None and v.requires_grad for v in (x, weight, scale, shift)):
        raise ValueError('Experimental inference only; detach parameters explicitly')
    if norm not in _NORMS:
        raise ValueError(f"norm must be one of {sorted(_NORMS)}")
    if not (0 < blocks <= 40):
        raise RuntimeError("invalid epsilon/blocks")
    # (not under graph capture: a captured call keeps reading the table it was given, as replays
    # of the raw form would see later writes to it)
    if not scale_is_one_plus and scale.is_cuda and not torch.cuda.is_current_stream_capturing():
        prepared = _registered_one_plus(scale)
        if prepared is not None:
            scale, scale_is_one_plus = prepared, True
            prepared_hits += 1
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
