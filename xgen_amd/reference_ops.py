"""The reference's fused operators under their own names, on the HIP kernels.

The reference's Python wrappers call torch.ops namespaces its compiled
libraries define (TORCH_LIBRARY + device + Meta registrations):

  h3_phaa_nq2::fused, h3_phaa_nq2_cached::fused
      (x, weight, scale, shift, indices, eps=1e-5, blocks=40) -> (q int8, scale)
      npu_fusion/f2_nq2/op_extension/nq2_queued.asc:47-51
  h3_phaa_gate_residual::gate_residual
      (residual, branch, gate_table, indices, tile=5376, blocks=40) -> out
      npu_fusion/f2a/op_extension/gate_residual_queued.asc:31
  h3_phaa_fusion_quant[_vector|_reuse]::swiglu_quantize
      (u, tile, blocks=40, scale_mode=1) -> (q int8, scale)
      npu_fusion/f1b/op_extension/swiglu_quant{,_vector,_reuse}_queued.asc:33
  h3_phaa_merge_quant::fused
      (back_recv, blocks=40) -> (q int8, scale)
      npu_fusion/f4_merge_quant/op_extension/merge_quant_queued.asc:26
  h3_phaa_layout::pack / back / merge
      (inputs, Tensor(a!) outputs..., tile=64, blocks=40) -> ()
      npu_fusion/f4/op_extension/layout_queued.asc:59-63

Here they are defined with the same schemas, with CUDA (HIP) and Meta
implementations that are the xgen_amd.operator functions mirroring those
wrappers (RMSNorm x weight -> INT8 for nq2, as the reference's NPU kernel),
behind the reference's schema checks and messages (RuntimeError, its shape
limits included), so code that holds the op handles runs unchanged once
xgen_amd is imported.  A namespace some other library already defined in this
process is left to it.
"""
from __future__ import annotations

import logging

import torch

from .operator import gate_residual as _gate
from .operator import merge_quant as _merge
from .operator import phaa_layout as _layout
from .operator import nq2 as _nq2
from .operator import swiglu_quant as _swiglu

_NQ2 = ("fused(Tensor x, Tensor weight, Tensor scale, Tensor shift, Tensor indices, float eps=0.00001, "
        "int blocks=40) -> (Tensor, Tensor)")
_GATE = ("gate_residual(Tensor residual, Tensor branch, Tensor gate_table, Tensor indices, int tile=5376, "
         "int blocks=40) -> Tensor")


_MERGE = "fused(Tensor back_recv, int blocks=40) -> (Tensor, Tensor)"
_LAYOUT = (
    ("pack", "pack(Tensor q, Tensor k, Tensor v, Tensor(a!) qo, Tensor(b!) ko, Tensor(c!) vo, int tile=64, "
             "int blocks=40) -> ()", _layout.pack_op, _layout.check_pack),
    ("back", "back(Tensor x, Tensor(a!) y, int S, int L, int tile=64, int blocks=40) -> ()",
     _layout.back_op, _layout.check_back),
    ("merge", "merge(Tensor x, Tensor(a!) y, int tile=64, int blocks=40) -> ()", _layout.merge_op,
     _layout.check_merge),
)


def _swiglu_schema(tile: int) -> str:
    return f"swiglu_quantize(Tensor u, int tile={tile}, int blocks=40, int scale_mode=1) -> (Tensor, Tensor)"


def _require(ok: bool, message: str) -> None:
    """The reference's TORCH_CHECK: a RuntimeError with its message, before any launch."""
    if not ok:
        raise RuntimeError(message)


def _nq2_impl(x, weight, scale, shift, indices, eps=1e-5, blocks=40):
    # the schema checks of nq2_queued.asc:20-25 (its NPU kernel's H <= 6144 included)
    _require(x.dim() == 3 and 0 < x.size(2) <= 6144 and x.dtype == torch.bfloat16 and x.stride(2) == 1,
             "BF16 [B,S,H], last stride1, H<=6144 required")
    _require(weight.dim() == 1 and weight.size(0) == x.size(2) and weight.is_contiguous()
             and weight.dtype in (torch.float32, torch.bfloat16), "BF16/FP32 norm weight [H] required")
    _require(scale.dim() == 2 and scale.size(0) > 0 and scale.size(1) == x.size(2) and shift.shape == scale.shape
             and scale.dtype == torch.bfloat16 and shift.dtype == torch.bfloat16 and scale.stride(1) == 1
             and shift.stride(1) == 1, "BF16 tables [M,H] required")
    _require(indices.dim() == 1 and indices.size(0) == x.size(1) and indices.dtype == torch.int64
             and indices.is_contiguous(), "contiguous INT64 indices [S] required")
    _require(0 < eps < 1 and 0 < blocks <= 40, "invalid epsilon/blocks")
    return _nq2.norm_affine_quant(x, weight, scale, shift, indices, eps=eps, blocks=blocks)


def _gate_impl(residual, branch, gate_table, indices, tile=5376, blocks=40):
    # gate_residual_queued.asc:10-19
    _require(residual.dim() == 3 and branch.shape == residual.shape and residual.size(2) > 0,
             "residual/branch [B,S,H] shapes must match")
    _require(gate_table.dim() == 2 and gate_table.size(0) > 0 and gate_table.size(1) == residual.size(2),
             "gate_table [M,H] required")
    _require(indices.dim() == 1 and indices.size(0) == residual.size(1) and indices.dtype == torch.int64
             and indices.is_contiguous(), "contiguous INT64 indices [S] required")
    _require(all(t.dtype == torch.bfloat16 for t in (residual, branch, gate_table)), "BF16 inputs required")
    _require(residual.stride(2) == 1 and branch.stride(2) == 1 and gate_table.stride(1) == 1,
             "last strides must be 1")
    return _gate.gate_residual(residual, branch, gate_table, indices, tile=tile, blocks=blocks)


def _merge_impl(back_recv, blocks=40):
    # merge_quant_queued.asc:10-13
    _merge.check_back_recv(back_recv, blocks)
    return _merge.xops.merge_quant(back_recv, torch.int8)


def _swiglu_impl(fn, tiles, default_tile):
    # (the schema's defaults again: a Python kernel receives the arguments as the caller gave them)
    def impl(u, tile=default_tile, blocks=40, scale_mode=1):
        # swiglu_quant{,_vector,_reuse}_queued.asc:10-14
        _require(u.dim() == 3 and u.size(2) > 0 and u.size(2) % 2 == 0 and u.size(2) <= 28672,
                 "[B,S,2F], 1<=F<=14336 required")
        _require(u.dtype == torch.bfloat16 and u.stride(2) == 1, "BF16, last stride=1 required")
        _require(tile in tiles, f"tile must be {', '.join(map(str, tiles))}")
        return fn(u, tile=tile, blocks=blocks, scale_mode=scale_mode)
    return impl


# namespace -> (schema, op name, implementation)
OPS = {
    "h3_phaa_nq2": (_NQ2, "fused", _nq2_impl),
    "h3_phaa_nq2_cached": (_NQ2, "fused", _nq2_impl),
    "h3_phaa_gate_residual": (_GATE, "gate_residual", _gate_impl),
    "h3_phaa_fusion_quant": (_swiglu_schema(2048), "swiglu_quantize",
                             _swiglu_impl(_swiglu.swiglu_quantize, (1024, 2048), 2048)),
    "h3_phaa_fusion_quant_vector": (_swiglu_schema(2048), "swiglu_quantize",
                                    _swiglu_impl(_swiglu.swiglu_quantize_vector, (1024, 2048), 2048)),
    "h3_phaa_fusion_quant_reuse": (_swiglu_schema(4096), "swiglu_quantize",
                                   _swiglu_impl(_swiglu.swiglu_quantize_reuse, (1024, 2048, 4096), 4096)),
    "h3_phaa_merge_quant": (_MERGE, "fused", _merge_impl),
}

_LIBS: dict = {}


def register() -> list:
    """Defines every namespace of OPS not yet defined in this process (idempotent); returns the
    namespaces this call defined."""
    defined = []
    for ns, (schema, name, impl) in OPS.items():
        if ns in _LIBS:
            continue
        try:
            lib = torch.library.Library(ns, "DEF")
            lib.define(schema)
        except RuntimeError as error:  # another library registered the namespace first
            logging.getLogger(__name__).info("torch.ops.%s left to its earlier registration: %s", ns, error)
            continue
        lib.impl(name, impl, "CUDA")
        lib.impl(name, impl, "Meta")
        _LIBS[ns] = lib
        defined.append(ns)
    if "h3_phaa_layout" not in _LIBS:
        try:
            lib = torch.library.Library("h3_phaa_layout", "DEF")
            for name, schema, _, _ in _LAYOUT:
                lib.define(schema)
        except RuntimeError as error:
            logging.getLogger(__name__).info("torch.ops.h3_phaa_layout left to its earlier registration: %s", error)
        else:
            for name, _, gpu, meta in _LAYOUT:
                lib.impl(name, gpu, "CUDA")
                lib.impl(name, meta, "Meta")   # the Meta implementations only check, as the reference's
            _LIBS["h3_phaa_layout"] = lib
            defined.append("h3_phaa_layout")
    return defined


register()
