"""BF16 layouts of the head-parallel attention's exchange on the HIP kernels.

Mirrors x_base/x_base/operator/npu_fusion/phaa_layout.py:13-28 (the ops
torch.ops.h3_phaa_layout.{pack, back, merge} of f4/op_extension/layout_queued.asc:59-63, which
`import xgen_amd` registers here with the reference's schemas and checks): the caller owns the
outputs and the stream order.

  pack_qkv(q, k, v, q_send, k_send, v_send)  Q/K/V [1, S, 56, 128] -> sends [7, 4, S, 1, 2, 128]
  unpack_qkv(q_recv, k_recv, v_recv, L=...)  received [4, S, 1, 2, 128] -> views [1, 2, L, 128]
  pack_back(attn, back_send, L=..., S=...)   attention output [1, 2, L, 128] -> [4, S, 1, 256]
                                             (rows from L on zero: one padding token at most)
  merge_back(back_recv, merged)              [7, 4, S, 1, 256] -> [1, S, 7168]

W / P / C (owners, chunks, heads per chunk) are validated against the one geometry the
reference supports (SP4, PHAA7, 2 heads per chunk); `tile` and `blocks` are the NPU kernel's
knobs, validated and otherwise unused.  ValueError for tensors that require grad or another
geometry, RuntimeError for the ops' schema checks, as the reference.  The kernels are
xgen_phaa_pack_qkv / xgen_phaa_pack_back / xgen_phaa_merge_back of libxgen_amd.so; there is no
host implementation.
"""
from __future__ import annotations

import torch

from .. import _native as N


def library_path():
    """The library holding the kernels (phaa_layout.py:7; XGEN_AMD_LIBRARY overrides it)."""
    return N.library_path()


def _require(ok, message):
    if not ok:
        raise RuntimeError(message)


def _byte_range(t):
    start = t.storage_offset() * t.element_size()
    extent = sum((n - 1) * st for n, st in zip(t.shape, t.stride())) + 1 if t.numel() else 0
    return start, start + extent * t.element_size()


def _overlap(a, b):
    if a.numel() == 0 or b.numel() == 0 or a.untyped_storage()._cdata != b.untyped_storage()._cdata:
        return False
    (a0, a1), (b0, b1) = _byte_range(a), _byte_range(b)
    return a0 < b1 and b0 < a1


def _check(x, out, tile, blocks):
    # layout_queued.asc:10-16
    _require(x.dtype == torch.bfloat16 and out.dtype == torch.bfloat16, "BF16 required")
    _require(x.device == out.device and out.is_contiguous(), "same device, contiguous output required")
    _require(tile in (16, 32, 64, 128), "tile 16/32/64/128 required")
    _require(0 < blocks <= 40, "1..40 Vector blocks")
    _require(not _overlap(x, out), "unsupported operation: some elements of the input tensor and the written-to "
                                   "tensor refer to a single memory location")


def check_pack(q, k, v, qo, ko, vo, tile=64, blocks=40):
    """layout_queued.asc:17-26."""
    for x in (q, k, v):
        _require(x.dim() == 4 and x.shape[0] == 1 and x.shape[1] > 0 and x.shape[2] == 56 and x.shape[3] == 128,
                 "[1,S,56,128] required")
        _require(x.stride(3) == 1 and x.stride(2) == 128 and 7168 <= x.stride(1) < (1 << 30),
                 "head contiguous and nonoverlapping row stride required")
        _require(x.shape == q.shape and x.device == q.device, "QKV shapes/devices must match")
        for y in (qo, ko, vo):
            _check(x, y, tile, blocks)
    for y in (qo, ko, vo):
        _require(tuple(y.shape) == (7, 4, q.shape[1], 1, 2, 128), "send shape mismatch")
    for a, b in ((qo, ko), (qo, vo), (ko, vo)):
        _require(not _overlap(a, b), "unsupported operation: some elements of the input tensor and the written-to "
                                     "tensor refer to a single memory location")


def check_back(x, y, S, L, tile=64, blocks=40):
    """layout_queued.asc:35-39."""
    _check(x, y, tile, blocks)
    _require(S > 0 and (L == 4 * S or L == 4 * S - 1), "only zero/one padding token supported")
    _require(tuple(x.shape) == (1, 2, L, 128) and x.stride(3) == 1 and x.stride(2) >= 128 and x.stride(1) >= 128
             and x.stride(2) < (1 << 30), "attn shape/stride mismatch")
    _require(tuple(y.shape) == (4, S, 1, 256), "back_send shape mismatch")


def check_merge(x, y, tile=64, blocks=40):
    """layout_queued.asc:46-49."""
    _check(x, y, tile, blocks)
    _require(x.dim() == 5 and x.shape[0] == 7 and x.shape[1] == 4 and x.shape[2] > 0 and x.shape[3] == 1
             and x.shape[4] == 256 and x.is_contiguous(), "contiguous [7,4,S,1,256] required")
    _require(tuple(y.shape) == (1, x.shape[2], 7168), "merged shape mismatch")


def _aligned(*ts):
    return all(t.data_ptr() % 16 == 0 for t in ts)


def _written(outs):
    """The buffers the kernel writes for `outs`: each output itself, or an aligned scratch copied
    into it afterwards (the kernels store 16-byte units)."""
    return [y if _aligned(y) else torch.empty_like(y, memory_format=torch.contiguous_format) for y in outs]


def _copy_back(outs, written):
    for y, w in zip(outs, written):
        if w is not y:
            y.copy_(w)


def pack_op(q, k, v, qo, ko, vo, tile=64, blocks=40):
    """torch.ops.h3_phaa_layout.pack on a HIP device (layout_queued.asc:27-34)."""
    check_pack(q, k, v, qo, ko, vo, tile, blocks)
    _require(q.is_cuda, "HIP (cuda) device required")
    # (a base or row stride off the 16-byte grid: the kernel reads from an aligned copy)
    srcs = [x if _aligned(x) and x.stride(1) % 8 == 0 else x.clone(memory_format=torch.contiguous_format)
            for x in (q, k, v)]
    outs = _written((qo, ko, vo))
    st = N.lib().xgen_phaa_pack_qkv(*(x.data_ptr() for x in srcs), q.shape[1], 4, 7, 2, 128,
                                    *(x.stride(1) for x in srcs), *(y.data_ptr() for y in outs), N.stream_of(q))
    N.check(st, "xgen_phaa_pack_qkv")
    _copy_back((qo, ko, vo), outs)


def back_op(x, y, S, L, tile=64, blocks=40):
    """torch.ops.h3_phaa_layout.back on a HIP device (layout_queued.asc:40-45)."""
    check_back(x, y, S, L, tile, blocks)
    _require(x.is_cuda, "HIP (cuda) device required")
    if not (_aligned(x) and x.stride(1) % 8 == 0 and x.stride(2) % 8 == 0):
        x = x.clone(memory_format=torch.contiguous_format)
    (out,) = _written((y,))
    st = N.lib().xgen_phaa_pack_back(x.data_ptr(), 2, L, 128, x.stride(1), x.stride(2), 4 * S, out.data_ptr(),
                                     N.stream_of(x))
    N.check(st, "xgen_phaa_pack_back")
    _copy_back((y,), (out,))


def merge_op(x, y, tile=64, blocks=40):
    """torch.ops.h3_phaa_layout.merge on a HIP device (layout_queued.asc:50-55)."""
    check_merge(x, y, tile, blocks)
    _require(x.is_cuda, "HIP (cuda) device required")
    if not _aligned(x):
        x = x.clone()
    (out,) = _written((y,))
    st = N.lib().xgen_phaa_merge_back(x.data_ptr(), 7, 4, x.shape[2], 1, 256, out.data_ptr(), N.stream_of(x))
    N.check(st, "xgen_phaa_merge_back")
    _copy_back((y,), (out,))


def _inference_only(*xs):
    if any(x.requires_grad for x in xs):
        raise ValueError("Inference only")


def _ops():
    from .. import reference_ops  # noqa: F401  (defines torch.ops.h3_phaa_layout)
    return torch.ops.h3_phaa_layout


def pack_qkv(q, k, v, q_send, k_send, v_send, *, W=4, P=7, C=2, tile=64, blocks=40):
    if (W, P, C) != (4, 7, 2):
        raise ValueError("Only SP4/PHAA7/2 heads supported")
    _inference_only(q, k, v, q_send, k_send, v_send)
    _ops().pack(q, k, v, q_send, k_send, v_send, tile, blocks)


def unpack_qkv(q_recv, k_recv, v_recv, *, L):
    """Views of the received Q/K/V as attention inputs [1, 2, L, 128] (phaa_layout.py:17-23): the
    four peers' sequence shards in order, the padding tokens past L dropped."""
    views = []
    for x in (q_recv, k_recv, v_recv):
        if (x.dim() != 5 or x.shape[0] != 4 or tuple(x.shape[2:]) != (1, 2, 128) or not x.is_contiguous()
                or x.dtype != torch.bfloat16):
            raise ValueError("contiguous BF16 [4,S,1,2,128] required")
        if not 0 < L <= 4 * x.shape[1]:
            raise ValueError("Invalid effective length")
        views.append(x.reshape(-1, 1, 2, 128).movedim(0, 2)[:, :, :L])
    return tuple(views)


def pack_back(attn, back_send, *, L, S, W=4, tile=64, blocks=40):
    if W != 4:
        raise ValueError("Only SP4 supported")
    _inference_only(attn, back_send)
    _ops().back(attn, back_send, S, L, tile, blocks)


def merge_back(back_recv, merged, *, W=4, P=7, C=2, tile=64, blocks=40):
    if (W, P, C) != (4, 7, 2):
        raise ValueError("Only SP4/PHAA7/2 heads supported")
    _inference_only(back_recv, merged)
    _ops().merge(back_recv, merged, tile, blocks)
