"""Asynchronous FP8 exchange of the head-parallel attention, on the HIP wire codec.

Mirrors x_base/x_base/phaa/fp8_async_transport.py:84-193.  submit_fp8_exchange
encodes one tensor or a Q/K/V triple into a uint8 send buffer (rows of head_dim
e4m3fn bytes followed by the row's float32 scale max|v| / 448 floored at 1e-12,
ordered [peer][stream][peer row], no peer padding) and enqueues
torch.distributed.all_to_all_single(async_op=True); finish_fp8_exchange makes
the consuming stream wait for the collective, keeps both buffers alive on it
and decodes the received rows.  The layouts of the reference's _encode /
_decode kernels (:13-80):

* plain: rows in the input's row-major order (a [peers, seq, batch, heads,
  head_dim] view with a unit last stride is read in place, anything else as its
  contiguous rows), decoded into contiguous outputs of the input's shape;
* fused return pack (return_shard_seq > 0): an attention output [batch, heads,
  seq, head_dim] (read in place when its last stride is 1) travels as
  [peers, return_shard_seq, batch, heads] rows, the positions past its seq as
  zero rows (scale 1e-12, zero bytes);
* direct gather (direct_gather=True): Q/K/V head shards [peers, shard_seq,
  batch, heads, head_dim] decode straight into [batch, heads, seq, head_dim]
  attention inputs, positions at or past seq dropped;
* return layout (finish_fp8_exchange(pending, output=..., return_layout=(seq,
  batch, peers, heads_per_peer, chunk_heads, head_start))): each peer's chunk of
  heads decodes into its place in a [batch, seq, peers * heads_per_peer *
  head_dim] output.

Encode and decode are xgen_fp8_wire_encode_masked, xgen_fp8_wire_decode and
xgen_fp8_wire_decode_strided of libxgen_amd.so, launched on the current stream;
there is no other implementation.  row_tiling picks the reference's Triton tile
(four rows per program); the HIP kernels walk the rows with one persistent
grid, so it is accepted and changes nothing.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import NamedTuple

import torch
import torch.distributed as dist

from .. import _native as N
from .fp8_transport import _WIRE_DTYPES, _views


@dataclass(frozen=True)
class AsyncFP8Options:
    """Switches of the asynchronous exchange (fp8_async_transport.py:84-93)."""
    direct_return: bool = False
    row_tiling: bool = False
    fused_return_pack: bool = False
    direct_gather: bool = False

    def __post_init__(self):
        if self.fused_return_pack and not self.direct_return:
            raise ValueError("PHAA fused return pack requires direct return")


class PendingFP8Exchange(NamedTuple):
    """An enqueued exchange (fp8_async_transport.py:96-101)."""
    work: object
    send: torch.Tensor
    recv: torch.Tensor
    outputs: tuple | None
    decode_args: tuple


class _WireRows(NamedTuple):
    """What the receiving side needs to decode: the logical rows per stream, the stream count, the row
    width, the peer count and, for the direct gather, the sender's (sequence positions, batch, heads)."""
    rows: int
    streams: int
    head_dim: int
    peers: int
    gather: tuple | None


def submit_fp8_exchange(outputs, tensors, head_dim, group, *, row_tiling=False, return_shard_seq=0,
                        direct_gather=False):
    """Encode on the current stream and enqueue the byte all-to-all (fp8_async_transport.py:104-113)."""
    send, recv, rows = _pack_exchange(outputs, tensors, head_dim, group, row_tiling=row_tiling,
                                      return_shard_seq=return_shard_seq, direct_gather=direct_gather)
    work = dist.all_to_all_single(recv, send, group=group, async_op=True)
    return PendingFP8Exchange(work, send, recv, outputs, rows)


def finish_fp8_exchange(pending, *, output=None, return_layout=()):
    """Order the current stream after the collective and decode (fp8_async_transport.py:116-123)."""
    consumer = torch.cuda.current_stream(pending.recv.device)
    pending.work.block_current_stream()
    for buffer in (pending.send, pending.recv):
        buffer.record_stream(consumer)
    targets = (output,) if return_layout else pending.outputs
    _unpack_exchange(pending.recv, targets, pending.decode_args, return_layout)


def _check_tensors(tensors, what):
    if any(t.device.type != "cuda" for t in tensors):
        raise ValueError("PHAA FP8 transport requires CUDA tensors")
    if any(t.dtype not in _WIRE_DTYPES for t in tensors) or any(t.dtype != tensors[0].dtype for t in tensors):
        raise ValueError(f"PHAA FP8 transport supports bfloat16, float16 and float32 {what} (one dtype)")


def _pack_exchange(outputs, tensors, head_dim, group, *, row_tiling=False, return_shard_seq=0,
                   direct_gather=False):
    """Checks the call as fp8_async_transport.py:126-160 does (same messages), then encodes.
    Returns (send, recv, _WireRows)."""
    del row_tiling  # a Triton tile size; one persistent grid here
    streams = len(tensors)
    if streams not in (1, 3) or (outputs is None and streams != 1):
        raise ValueError("PHAA FP8 transport expects one tensor or a QKV triple")
    if outputs is not None and len(outputs) != streams:
        raise ValueError("PHAA FP8 transport requires one output per input")
    shape = tuple(tensors[0].shape)
    if head_dim % 4 or any(tuple(t.shape) != shape for t in tensors):
        raise ValueError("PHAA FP8 transport requires matching shapes and head dim divisible by four")
    gather = None
    if direct_gather:
        if streams != 3 or len(shape) != 5 or shape[-1] != head_dim:
            raise ValueError("PHAA direct gather expects QKV head shards")
        shard_peers, shard_seq, batches, chunk_heads = shape[:4]
        seen = outputs[0].shape[-2]
        if not 0 < seen <= shard_peers * shard_seq or \
                any(tuple(o.shape) != (batches, chunk_heads, seen, head_dim) for o in outputs):
            raise ValueError("PHAA direct gather requires matching attention output shapes")
        gather = (shard_peers * shard_seq, batches, chunk_heads)
    elif outputs is not None and any(tuple(o.shape) != shape for o in outputs):
        raise ValueError("PHAA FP8 transport requires matching input and output shapes")
    if outputs is not None and any(not o.is_contiguous() for o in outputs):
        raise ValueError("PHAA FP8 transport requires contiguous outputs")
    peers = dist.get_world_size(group)
    rows = tensors[0].numel() // head_dim
    valid = None
    if return_shard_seq:
        if outputs is not None or streams != 1 or len(shape) != 4 or shape[-1] != head_dim:
            raise ValueError("PHAA return pack expects an attention output and direct return")
        batches, chunk_heads, valid, _ = shape
        if not 0 < valid <= peers * return_shard_seq:
            raise ValueError("PHAA return pack received an invalid sequence length")
        rows = peers * return_shard_seq * batches * chunk_heads
    if rows % peers or tensors[0].numel() % head_dim:
        raise ValueError("PHAA FP8 rows must divide evenly among peers")
    _check_tensors(tensors, "inputs")
    if outputs is not None:
        _check_tensors(outputs, "outputs")

    send = torch.empty((streams * rows, head_dim + 4), dtype=torch.uint8, device=tensors[0].device)
    recv = torch.empty_like(send)
    _encode_rows(tensors, head_dim, peers, return_shard_seq, send)
    return send, recv, _WireRows(rows, streams, head_dim, peers, gather)


def _encode_rows(tensors, head_dim, peers, return_shard_seq, send):
    """Encodes checked inputs into `send` on the current stream.  With return_shard_seq the input is an
    attention output [batch, heads, seq, D] read as [peer, shard seq, batch, head] rows: a position's
    sequence index is peer * shard_seq + s (so the peer stride is shard_seq sequence strides), and the
    positions from seq on travel as zero rows."""
    streams = len(tensors)
    if return_shard_seq:
        (attn,) = tensors
        if attn.stride(-1) != 1:
            attn = attn.contiguous()
        sb, sh, ss = attn.stride()[:3]
        views, strides = (attn,), [[return_shard_seq * ss, ss, sb, sh]]
        seq, batch, heads, valid = return_shard_seq, attn.shape[0], attn.shape[1], attn.shape[2]
    else:
        views, strides, (seq, batch, heads) = _views(tensors, head_dim, peers)
        valid = peers * seq
    flat = [x for st in strides for x in st]
    ptrs = [v.data_ptr() for v in views] + [None] * (3 - streams)
    st = N.lib().xgen_fp8_wire_encode_masked(
        N.dtype_code(tensors[0].dtype), streams, *ptrs, (N._c_i64 * len(flat))(*flat), peers, seq, batch, heads,
        head_dim, valid, send.data_ptr(), N.stream_of(send))
    N.check(st, "xgen_fp8_wire_encode_masked")


def _decode_strided(recv, outputs, rows, geometry, strides, valid, offset=0):
    """Strided decode of every stream: geometry (peers, seq, batch, heads), element strides over them,
    `offset` elements into each output."""
    peers, seq, batch, heads = geometry
    width = rows.head_dim
    eb = outputs[0].element_size()
    ptrs = [o.data_ptr() + offset * eb for o in outputs] + [None] * (3 - len(outputs))
    st = N.lib().xgen_fp8_wire_decode_strided(
        N.dtype_code(outputs[0].dtype), len(outputs), recv.data_ptr(), peers, seq, batch, heads, width,
        (N._c_i64 * 4)(*strides), valid, *ptrs, N.stream_of(recv))
    N.check(st, "xgen_fp8_wire_decode_strided")


def _unpack_exchange(recv, outputs, decode_args, return_layout=()):
    """Decodes the received rows (fp8_async_transport.py:183-193) into the outputs' layout."""
    rows = decode_args
    if outputs is None or len(outputs) != rows.streams or any(o is None for o in outputs):
        raise ValueError("PHAA FP8 transport requires one output per input")
    _check_tensors(outputs, "outputs")
    if any(not o.is_contiguous() for o in outputs):
        raise ValueError("PHAA FP8 transport requires contiguous outputs")
    D, peers = rows.head_dim, rows.peers
    peer_rows = rows.rows // peers
    if rows.gather is not None:
        positions, batch, heads = rows.gather
        if positions % peers:
            raise ValueError("PHAA direct gather requires the sequence to divide evenly among peers")
        shard_seq, seen = positions // peers, outputs[0].shape[-2]
        if not 0 < seen <= positions or any(tuple(o.shape) != (batch, heads, seen, D) for o in outputs):
            raise ValueError("PHAA direct gather requires matching attention output shapes")
        # [batch, heads, seq, D]: sequence position peer * shard_seq + s
        _decode_strided(recv, outputs, rows, (peers, shard_seq, batch, heads),
                        (shard_seq * D, D, heads * seen * D, seen * D), seen)
    elif return_layout:
        seq, batch, out_peers, heads_per_peer, chunk_heads, head_start = (int(x) for x in return_layout)
        (out,) = outputs
        if seq * batch * chunk_heads != peer_rows or out_peers != peers or head_start < 0 or \
                head_start + chunk_heads > heads_per_peer or out.numel() != batch * seq * peers * heads_per_peer * D:
            raise ValueError("PHAA return layout does not match the received rows or the output")
        # [batch, seq, peers, heads_per_peer, D], this chunk's heads from head_start
        _decode_strided(recv, outputs, rows, (peers, seq, batch, chunk_heads),
                        (heads_per_peer * D, peers * heads_per_peer * D, seq * peers * heads_per_peer * D, D),
                        peers * seq, offset=head_start * D)
    else:
        if any(o.numel() != rows.rows * D for o in outputs):
            raise ValueError("PHAA FP8 transport requires matching input and output shapes")
        ptrs = [o.data_ptr() for o in outputs] + [None] * (3 - len(outputs))
        st = N.lib().xgen_fp8_wire_decode(N.dtype_code(outputs[0].dtype), rows.streams, recv.data_ptr(), peers,
                                          peer_rows, D, 0, *ptrs, N.stream_of(recv))
        N.check(st, "xgen_fp8_wire_decode")
