"""Per-head FP8 transport for the head-parallel attention all-to-all, on the HIP wire codec.

Mirrors x_base/x_base/phaa/fp8_transport.py:81-144.  fp8_all_to_all_many packs one
tensor or a Q/K/V triple into one uint8 send buffer whose rows are `head_dim`
e4m3fn bytes followed by the row's float32 scale (max|v| / 448, floored at
1e-12), ordered [peer][stream][peer row]; exchanges it with a single
torch.distributed.all_to_all_single; and decodes the received rows into the
caller's (contiguous) outputs.  XGEN_PHAA_FP8_ALIGN16=1 pads each peer's block
to a multiple of 16 bytes with zeros (fp8_transport.py:103-112).

Strided inputs: a 5-D [peers, seq, batch, heads, head_dim] view with unit last
stride is read in place, with per-stream strides (what the reference does for
uniform Q/K/V strides, and under XGEN_PHAA_FP8_MIXED_STRIDES=1 for mixed ones);
other layouts are made contiguous first, as in the reference.  The wire bytes
are the same either way.  Encode and decode are the HIP kernels of
libxgen_amd.so (xgen_fp8_wire_encode / xgen_fp8_wire_decode); there is no
other implementation.
"""
from __future__ import annotations

import logging
import os

import torch
import torch.distributed as dist

from .. import _native as N

_mixed_stride_metrics = dict(calls=0, avoided_contiguous_bytes=0)
_peer_alignment_metrics = dict(calls=0, padded_calls=0, padding_bytes=0)
_WIRE_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def mixed_stride_metrics():
    """Scalar diagnostics only; no tensor or communication-buffer cache (fp8_transport.py:16-18)."""
    return dict(_mixed_stride_metrics)


def peer_alignment_metrics():
    """Scalar counters for the opt-in peer-aligned wire layout (fp8_transport.py:21-23)."""
    return dict(_peer_alignment_metrics)


def peer_padding(streams: int, peer_rows: int, head_dim: int, align16: bool) -> int:
    """Zero bytes after each peer's block: (-peer_bytes) mod 16 when aligning, else 0."""
    return int(N.lib().xgen_fp8_wire_peer_padding(streams, peer_rows, head_dim, int(bool(align16))))


def wire_shape(streams: int, rows: int, head_dim: int, peers: int, padding: int):
    """(peers, peer_bytes + padding) when padded, else (streams * rows, head_dim + 4) (fp8_transport.py:112)."""
    peer_bytes = rows // peers * streams * (head_dim + 4)
    return (peers, peer_bytes + padding) if padding else (streams * rows, head_dim + 4)


def _views(tensors, head_dim: int, peers: int):
    """Input tensors with unit last stride, their [peer, seq, batch, head] element strides and
    (seq, batch, heads): 5-D [peers, ...] views are read in place, anything else as contiguous rows."""
    shape = tensors[0].shape
    if len(shape) == 5 and shape[0] == peers and shape[-1] == head_dim:
        views = tuple(t if t.stride(-1) == 1 else t.contiguous() for t in tensors)
        return views, [list(t.stride()[:4]) for t in views], tuple(shape[1:4])
    views = tuple(t if t.is_contiguous() else t.contiguous() for t in tensors)
    pr = views[0].numel() // head_dim // peers
    return views, [[pr * head_dim, head_dim, 0, 0] for _ in views], (pr, 1, 1)


def encode_wire(tensors, head_dim: int, peers: int, *, align16: bool = False, out: torch.Tensor | None = None):
    """Encodes 1 or 3 equal-shaped CUDA tensors into a uint8 send buffer (new, or `out` when given:
    a contiguous uint8 tensor of wire_shape(...)); returns (wire, padding)."""
    streams = len(tensors)
    rows = tensors[0].numel() // head_dim
    pad = peer_padding(streams, rows // peers, head_dim, align16)
    shape = wire_shape(streams, rows, head_dim, peers, pad)
    if out is None:
        wire = torch.empty(shape, dtype=torch.uint8, device=tensors[0].device)
    else:
        if out.dtype != torch.uint8 or tuple(out.shape) != shape or not out.is_contiguous():
            raise ValueError(f"encode_wire: out must be a contiguous uint8 tensor of shape {shape}")
        wire = out
    views, strides, (seq, batch, heads) = _views(tensors, head_dim, peers)
    flat = [x for st in strides for x in st]
    arr = (N._c_i64 * len(flat))(*flat)
    ptrs = [v.data_ptr() for v in views] + [None] * (3 - streams)
    st = N.lib().xgen_fp8_wire_encode(
        N.dtype_code(tensors[0].dtype), streams, *ptrs, arr, peers, seq, batch, heads, head_dim, pad,
        wire.data_ptr(), N.stream_of(wire))
    N.check(st, "xgen_fp8_wire_encode")
    return wire, pad


def decode_wire(wire: torch.Tensor, outputs, head_dim: int, peers: int, padding: int) -> None:
    """Decodes a received wire buffer into 1 or 3 contiguous outputs (in place)."""
    streams = len(outputs)
    rows = outputs[0].numel() // head_dim
    ptrs = [o.data_ptr() for o in outputs] + [None] * (3 - streams)
    st = N.lib().xgen_fp8_wire_decode(
        N.dtype_code(outputs[0].dtype), streams, wire.data_ptr(), peers, rows // peers, head_dim, padding, *ptrs,
        N.stream_of(wire))
    N.check(st, "xgen_fp8_wire_decode")


def fp8_all_to_all(output, tensor, head_dim, group):
    """Single-tensor form (fp8_transport.py:81-82)."""
    fp8_all_to_all_many((output,), (tensor,), head_dim, group)


def fp8_all_to_all_many(outputs, tensors, head_dim, group):
    """Exchange equal-shaped tensors and their row scales in one byte collective (fp8_transport.py:85-144)."""
    streams = len(tensors)
    if streams not in (1, 3) or len(outputs) != streams:
        raise ValueError("PHAA FP8 transport expects one tensor or a QKV triple")
    if any(t.device.type != "cuda" for t in (*outputs, *tensors)):
        raise ValueError("PHAA FP8 transport requires CUDA tensors")
    shape = tensors[0].shape
    if head_dim % 4 or any(x.shape != shape for x in (*outputs, *tensors)):
        raise ValueError("PHAA FP8 transport requires matching shapes and head dim divisible by four")
    if any(not out.is_contiguous() for out in outputs):
        raise ValueError("PHAA FP8 transport requires contiguous outputs")
    if any(t.dtype not in _WIRE_DTYPES for t in (*outputs, *tensors)) or \
            any(t.dtype != tensors[0].dtype for t in tensors) or any(o.dtype != outputs[0].dtype for o in outputs):
        raise ValueError("PHAA FP8 transport supports bfloat16, float16 and float32 tensors "
                         "(one dtype for the inputs, one for the outputs)")
    rows = tensors[0].numel() // head_dim
    peers = dist.get_world_size(group)
    if rows % peers or tensors[0].numel() % head_dim:
        raise ValueError("PHAA FP8 rows must divide evenly among peers")
    align_peers = os.environ.get("XGEN_PHAA_FP8_ALIGN16", "0") == "1"
    if align_peers:
        pad = peer_padding(streams, rows // peers, head_dim, True)
        if _peer_alignment_metrics["calls"] == 0:
            logging.getLogger(__name__).info("PHAA FP8 per-peer 16-byte alignment enabled")
        _peer_alignment_metrics["calls"] += 1
        _peer_alignment_metrics["padded_calls"] += int(pad > 0)
        _peer_alignment_metrics["padding_bytes"] += peers * pad
    strides = tensors[0].stride()
    if (os.environ.get("XGEN_PHAA_FP8_MIXED_STRIDES", "0") == "1" and streams == 3 and len(shape) == 5
            and shape[0] == peers and shape[-1] == head_dim and all(x.stride(-1) == 1 for x in tensors)
            and not all(x.stride() == strides for x in tensors)):
        if _mixed_stride_metrics["calls"] == 0:
            logging.getLogger(__name__).info(
                "PHAA FP8 mixed-stride packing enabled: shape=%s strides=%s", tuple(shape),
                tuple(x.stride() for x in tensors))
        _mixed_stride_metrics["calls"] += 1
        _mixed_stride_metrics["avoided_contiguous_bytes"] += sum(
            x.numel() * x.element_size() for x in tensors if not x.is_contiguous())
    send, pad = encode_wire(tensors, head_dim, peers, align16=align_peers)
    recv = torch.empty_like(send)
    dist.all_to_all_single(recv, send, group=group)
    decode_wire(recv, outputs, head_dim, peers, pad)
