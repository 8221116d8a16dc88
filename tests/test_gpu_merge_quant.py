"""GPU parity of the merge + per-token quantization of the head-parallel attention's returned
chunks (torch.ops.h3_phaa_merge_quant.fused, merge_quant_kernel.asc:20-87): bytes and scales
bit-exact against the oracle (the reference kernel's copy, pinned on the CPU, then the row
quantizers) at the reference geometry [7, 4, S, 1, 256] and at general ones covering every
register-chunk count of the kernel; zero and NaN rows; the op handles; and the consumer chain
(x_base/x_base/phaa/fused_layout.py:44-48 -> QuantizedRows -> quant_matmul) equal to quantizing
the merged rows."""
import pytest
import torch

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd.operator import runtime
from xgen_amd.operator.matmul import WeightQuantLinearModule
from xgen_amd.operator.merge_quant import merge_quant
from xgen_amd.operator.quantized import QuantizedRows

pytestmark = pytest.mark.gpu
xops = torch.ops.xgen_amd
FP8 = torch.float8_e4m3fn


def back_recv(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def check(q, s, x, out):
    rq, rs = R.merge_quant(x, out="int8" if out == torch.int8 else "fp8")
    assert q.dtype == out and q.shape == rq.shape and s.shape == rs.shape
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(s.cpu(), rs)


@pytest.mark.parametrize("seq", [1, 17, 333])
@pytest.mark.parametrize("out", [torch.int8, FP8])
def test_reference_geometry_bit_exact(cuda, seq, out):
    x = back_recv((7, 4, seq, 1, 256), seed=seq)
    q, s = merge_quant(x.to(cuda), out_dtype=out)
    check(q, s, x, out)
    if out == torch.int8:
        q2, s2 = torch.ops.h3_phaa_merge_quant.fused(x.to(cuda))
        assert torch.equal(q2, q) and torch.equal(s2, s)


@pytest.mark.parametrize("shape", [
    (1, 1, 5, 3, 8),        # one 16-byte chunk per row
    (3, 2, 7, 2, 64),       # batch 2: rows b * seq + s
    (7, 4, 9, 1, 64),       # 224 chunks: one per thread
    (5, 3, 11, 2, 96),      # 180 chunks of segments of 12
    (4, 4, 6, 1, 256),      # 512 chunks: two per thread
    (8, 8, 3, 1, 256),      # 16,384 values: eight per thread
])
@pytest.mark.parametrize("out", [torch.int8, FP8])
def test_general_geometry_bit_exact(cuda, shape, out):
    x = back_recv(shape, seed=sum(shape))
    q, s = xops.merge_quant(x.to(cuda), out)
    check(q, s, x, out)


def test_zero_and_nan_rows(cuda):
    x = back_recv((7, 4, 6, 1, 256), seed=3)
    x[:, :, 1] = 0                      # zero row: zero bytes, zero scale (INT8)
    x[2, 3, 4, 0, 17] = float("nan")    # a NaN in owner 3's chunk 2 of row 4
    x[0, 0, 5, 0, 0] = float("inf")
    for out in (torch.int8, FP8):
        q, s = xops.merge_quant(x.to(cuda), out)
        rq, rs = R.merge_quant(x, out="int8" if out == torch.int8 else "fp8")
        assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))
        nan = torch.isnan(rs)
        assert nan.tolist() == [False, False, False, False, True, False]
        assert torch.equal(torch.isnan(s.cpu()), nan) and torch.equal(s.cpu()[~nan], rs[~nan])
    q, s = xops.merge_quant(x.to(cuda), torch.int8)
    assert s[1] == 0 and not q[1].any()


def test_strided_input_is_made_contiguous(cuda):
    x = back_recv((4, 7, 9, 1, 256), seed=4).transpose(0, 1)   # a [7, 4, ...] view, not contiguous
    q, s = xops.merge_quant(x.to(cuda), torch.int8)
    check(q, s, x.contiguous(), torch.int8)


def test_feeds_the_out_projection_as_quantized_rows(cuda):
    """fused_layout.py:44-48 + h3_npu_fusion.py:142-145: QuantizedRows(q, scale, (B, S, width)) into
    quant_matmul through the INT8 out-projection == quantizing the merged rows first."""
    seq, width, n_out = 40, 7168, 512
    x = back_recv((7, 4, seq, 1, 256), seed=6).to(cuda)
    g = torch.Generator().manual_seed(7)
    w = (torch.randn((n_out, width), generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn((n_out,), generator=g) * 0.01).to(torch.bfloat16)
    layer = WeightQuantLinearModule(w.to(cuda), b.to(cuda)).to(cuda)
    assert runtime.quant_linear(layer, width, x.device)
    q, s = merge_quant(x)
    value = QuantizedRows(q, s, (1, seq, width))
    out = runtime.quant_matmul(value.q, value.scale, layer, value.shape)
    rows = R.merge_rows(x).to(cuda)
    q_ref, s_ref = xops.quantize_rows(rows, torch.int8)
    assert torch.equal(q, q_ref) and torch.equal(s, s_ref)
    expected = runtime.quant_matmul(q_ref, s_ref, layer, (1, seq, width))
    assert out.shape == (1, seq, n_out) and torch.equal(out, expected)
    assert torch.equal(out.view(seq, n_out), layer(rows.view(1, seq, width)).view(seq, n_out))


def test_kernels_resolve_merge_quant(cuda):
    d = runtime.Diagnostics()
    k = runtime.Kernels(d)
    module = k.get("merge_quant", torch.zeros(1, dtype=torch.bfloat16, device=cuda))
    assert module is not None and module.merge_quant is merge_quant
    assert not d.fallbacks


def test_beyond_the_last_level_cache(cuda):
    """A call whose footprint exceeds the 256 MB last-level cache reads non-temporally: S = 13,000
    (279 MB), sampled rows bit-exact against the oracle on those rows (rows are independent)."""
    seq = 13000
    g = torch.Generator(device=cuda).manual_seed(8)
    x = torch.randn((7, 4, seq, 1, 256), generator=g, device=cuda).to(torch.bfloat16)
    q, s = merge_quant(x)
    rows = torch.tensor([0, 1, 4095, 6500, 12998, 12999])
    sample = x[:, :, rows.to(cuda)].cpu()
    rq, rs = R.merge_quant(sample)
    assert torch.equal(q[rows.to(cuda)].cpu(), rq) and torch.equal(s[rows.to(cuda)].cpu(), rs)


@pytest.mark.parametrize("accumulation", ["exact", "mfma"])
def test_fp8_rows_feed_the_fp8_out_projection(cuda, accumulation):
    """The FP8 form (out_dtype=float8_e4m3fn) into the FP8 out-projection (H3FP8Linear with per-token
    activation scales) through quant_matmul: equal to that module's own forward on the merged rows
    (which quantizes them with the same FP8 row quantizer)."""
    from xgen_amd.operator.h3_fp8 import H3FP8Linear
    seq, width, n_out = 48, 7168, 384
    x = back_recv((7, 4, seq, 1, 256), seed=13).to(cuda)
    g = torch.Generator().manual_seed(14)
    w = (torch.randn((n_out, width), generator=g) * 0.02).to(torch.bfloat16).to(cuda)
    b = (torch.randn((n_out,), generator=g) * 0.01).to(torch.bfloat16).to(cuda)
    layer = H3FP8Linear(w, b, activation_scaling="token", accumulation=accumulation)
    assert runtime.quant_linear(layer, width, x.device)
    q, s = merge_quant(x, out_dtype=FP8)
    value = QuantizedRows(q, s, (1, seq, width))
    out = runtime.quant_matmul(value.q, value.scale, layer, value.shape)
    rows = R.merge_rows(x).to(cuda).view(1, seq, width)
    assert torch.equal(out.view(torch.int16), layer(rows).view(torch.int16))


def test_reference_maximum_sequence(cuda):
    """S = 2^20, the reference op's largest (merge_quant_queued.asc:12): a 15 GB back_recv whose source
    offsets pass 2^32 bytes, merged + quantized (7.5 GB of rows) and merged in BF16; sampled rows
    (first, last, around each 2^30-byte segment boundary) against the oracle."""
    from xgen_amd.operator import phaa_layout
    seq = 1 << 20
    g = torch.Generator(device=cuda).manual_seed(15)
    x = torch.randn((7, 4, seq, 1, 256), generator=g, device=cuda, dtype=torch.bfloat16)
    q, s = merge_quant(x)
    rows = torch.tensor([0, 1, 2047, 2048, 524287, 524288, seq - 2, seq - 1])
    sample = x[:, :, rows.to(cuda)].cpu()
    rq, rs = R.merge_quant(sample)
    assert torch.equal(q[rows.to(cuda)].cpu(), rq) and torch.equal(s[rows.to(cuda)].cpu(), rs)
    del q, s
    merged = torch.empty((1, seq, 7168), dtype=torch.bfloat16, device=cuda)
    phaa_layout.merge_back(x, merged)
    assert torch.equal(merged[0, rows.to(cuda)].cpu(), R.merge_rows(sample))
