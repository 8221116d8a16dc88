"""GPU: every operator gives the same bytes on views its kernel cannot read in place (a base off the
16-byte alignment, row strides off the 8-element alignment, a contiguous tensor at an unaligned
offset) as on contiguous copies of them; the wrappers copy such views.  Views the kernels do read in
place (aligned row strides above the width) are covered by each operator's own tests."""
import pytest
import torch

import xgen_amd  # noqa: F401
from xgen_amd import _native as N

pytestmark = pytest.mark.gpu
xops = torch.ops.xgen_amd
FP8 = torch.float8_e4m3fn


def bits(t):
    return t.view(torch.uint8) if t.element_size() == 1 else t.view(torch.int16 if t.element_size() == 2
                                                                     else torch.int32)


def same(a, b):
    assert a.shape == b.shape and torch.equal(bits(a.contiguous()), bits(b.contiguous()))


def shifted(t, first):
    """t's values in a view of a wider buffer, `first` elements into each row (unaligned for odd first)."""
    big = torch.zeros((*t.shape[:-1], t.shape[-1] + 24), dtype=t.dtype, device=t.device)
    big[..., first:first + t.shape[-1]] = t
    return big[..., first:first + t.shape[-1]]


def unaligned_flat(t, offset=1):
    """A contiguous tensor equal to t whose base sits `offset` elements past an aligned allocation."""
    flat = torch.zeros(t.numel() + offset, dtype=t.dtype, device=t.device)
    flat[offset:] = t.reshape(-1)
    return flat[offset:].view(t.shape)


def test_norm_affine_quant_views(cuda):
    g = torch.Generator().manual_seed(1)
    B, S, H, T = 2, 9, 512, 5
    x = torch.randn((B, S, H), generator=g).to(torch.bfloat16).to(cuda)
    scale = (torch.randn((T, H), generator=g) * 0.1).to(torch.bfloat16).to(cuda)
    shift = (torch.randn((T, H), generator=g) * 0.1).to(torch.bfloat16).to(cuda)
    idx = torch.randint(T, (S,), generator=g).to(cuda)
    w = (torch.randn((H,), generator=g) * 0.3 + 1).to(torch.bfloat16).to(cuda)
    for norm in (N.NORM_LAYER, N.NORM_RMS):
        ref = xops.norm_affine_quant(x, w, scale, shift, idx, 1e-6, norm, FP8, True)
        for xv, sv, tv, wv in ((shifted(x, 1), shifted(scale, 3), shifted(shift, 5), unaligned_flat(w)),
                               (unaligned_flat(x), unaligned_flat(scale), unaligned_flat(shift), w)):
            got = xops.norm_affine_quant(xv, wv, sv, tv, idx, 1e-6, norm, FP8, True)
            for a, b in zip(got, ref):
                same(a, b)


def test_gate_residual_views(cuda):
    g = torch.Generator().manual_seed(2)
    B, S, H, T = 2, 7, 264, 3
    res = torch.randn((B, S, H), generator=g).to(torch.bfloat16).to(cuda)
    br = torch.randn((B, S, H), generator=g).to(torch.bfloat16).to(cuda)
    gate = torch.randn((T, H), generator=g).to(torch.bfloat16).to(cuda)
    idx = torch.randint(T, (S,), generator=g).to(cuda)
    ref = xops.gate_residual(res, br, gate, idx)
    same(xops.gate_residual(shifted(res, 1), shifted(br, 2), shifted(gate, 3), idx), ref)
    same(xops.gate_residual(unaligned_flat(res), unaligned_flat(br), unaligned_flat(gate), idx), ref)


def test_swiglu_quant_views(cuda):
    g = torch.Generator().manual_seed(3)
    u = torch.randn((2, 5, 2 * 136), generator=g).to(torch.bfloat16).to(cuda)
    for out in (FP8, torch.int8):
        ref = xops.swiglu_quant(u, False, out, 1, True)
        for uv in (shifted(u, 1), unaligned_flat(u)):
            for a, b in zip(xops.swiglu_quant(uv, False, out, 1, True), ref):
                same(a, b)


def test_per_tensor_quantizer_views(cuda):
    g = torch.Generator().manual_seed(4)
    x = torch.randn((37, 100), generator=g).to(torch.bfloat16).to(cuda)
    peak, scale = xops.abs_peak(x), xops.fp8_tensor_scale(x)
    q = xops.fp8_pack(x, scale)
    for xv in (unaligned_flat(x), shifted(x, 1)):
        same(xops.abs_peak(xv), peak)
        same(xops.fp8_tensor_scale(xv), scale)
        same(xops.fp8_pack(xv, scale), q)


def test_quantize_rows_views(cuda):
    g = torch.Generator().manual_seed(5)
    x = torch.randn((33, 200), generator=g).to(torch.bfloat16).to(cuda)
    for out in (FP8, torch.int8):
        ref = xops.quantize_rows(x, out)
        for xv in (unaligned_flat(x), shifted(x, 1)):
            for a, b in zip(xops.quantize_rows(xv, out), ref):
                same(a, b)
