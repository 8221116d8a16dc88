"""GPU parity of the FP8 wire codec (xgen_fp8_wire_encode / _decode) and of the transport
surface (xgen_amd.phaa.fp8_transport, mirroring x_base/x_base/phaa/fp8_transport.py):
wire bytes and decoded values bit-exact against the oracle, the reference tests' transport
facts through a patched collective, and size-independent properties at H3 geometry."""
from unittest.mock import patch

import pytest
import torch
import torch.distributed as dist

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd.phaa import fp8_transport as transport

pytestmark = pytest.mark.gpu


def qkv(shape, streams, seed, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(shape, generator=g) * scale).to(dtype) for _ in range(streams))


def encode_pair(tensors, width, peers, align16, cuda):
    """(GPU wire, oracle wire, padding) for CPU tensors."""
    wire, pad = transport.encode_wire(tuple(t.to(cuda) for t in tensors), width, peers, align16=align16)
    ref = R.fp8_wire_encode(tensors, width, peers, align16)
    return wire.cpu(), ref, pad


def decoded(wire, streams, rows, width, peers, pad, dtype, cuda):
    outs = tuple(torch.empty((rows, width), dtype=dtype, device=cuda) for _ in range(streams))
    transport.decode_wire(wire.to(cuda), outs, width, peers, pad)
    return [o.cpu() for o in outs]


def same(a, b):
    """Bit equality of two CPU float tensors, NaN matching NaN whatever its payload and sign (an
    invalid product is 0xffc00000 on x86 and 0x7fc00000 on the GPU)."""
    nan_a, nan_b = torch.isnan(a), torch.isnan(b)
    if not torch.equal(nan_a, nan_b):
        return False
    bits = {torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.float16: torch.int16}[a.dtype]
    return torch.equal(a.view(bits)[~nan_a], b.view(bits)[~nan_b])


@pytest.mark.parametrize("streams", [1, 3])
@pytest.mark.parametrize("seq", [17, 20])
@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("align16", [False, True])
def test_encode_decode_bit_exact(cuda, streams, seq, batch, align16):
    peers, heads, width = 2, 3, 128
    t = qkv((peers, seq, batch, heads, width), streams, seed=42 + seq + batch)
    wire, ref, pad = encode_pair(t, width, peers, align16, cuda)
    assert wire.shape == ref.shape and torch.equal(wire, ref)
    rows = peers * seq * batch * heads
    out = decoded(wire, streams, rows, width, peers, pad, torch.bfloat16, cuda)
    expect = R.fp8_wire_decode(ref, streams, rows, width, peers, pad, torch.bfloat16)
    assert all(same(a, b) for a, b in zip(out, expect))


@pytest.mark.parametrize("width", [4, 12, 64, 68, 96, 256, 260, 520, 1024])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_widths_and_dtypes(cuda, width, dtype):
    peers, rows = 4, 4 * 37
    g = torch.Generator().manual_seed(width)
    x = (torch.randn(rows, width, generator=g) * torch.logspace(-4, 4, rows)[:, None]).to(dtype)
    wire, ref, pad = encode_pair((x,), width, peers, True, cuda)
    assert torch.equal(wire, ref)
    for out_dtype in (torch.bfloat16, torch.float16, torch.float32):
        out = decoded(wire, 1, rows, width, peers, pad, out_dtype, cuda)[0]
        assert same(out, R.fp8_wire_decode(ref, 1, rows, width, peers, pad, out_dtype)[0])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_element_aligned_inputs_and_outputs(cuda, dtype):
    """Storage offset of one element: the kernels' element-wise load / store path."""
    peers, rows, width = 2, 2 * 19, 64
    g = torch.Generator().manual_seed(5)
    base = torch.randn(rows * width + 1, generator=g).to(dtype)
    x = base[1:].reshape(rows, width)
    wire, pad = transport.encode_wire((base.to(cuda)[1:].reshape(rows, width),), width, peers)
    ref = R.fp8_wire_encode((x,), width, peers)
    assert torch.equal(wire.cpu(), ref)
    out_store = torch.empty(rows * width + 1, dtype=dtype, device=cuda)
    out = out_store[1:].reshape(rows, width)
    transport.decode_wire(wire, (out,), width, peers, pad)
    assert same(out.cpu(), R.fp8_wire_decode(ref, 1, rows, width, peers, pad, dtype)[0])


def test_special_rows(cuda):
    """Zero rows (scale floor), tiny rows below 448e-12, the 448 / 464 boundaries, exact e4m3
    midpoints, outliers, and non-finite rows (this build's NaN convention, see the oracle)."""
    width = 64
    x = torch.randn(16, width)
    x[0] = 0.0
    x[1] = torch.linspace(-1, 1, width) * 3e-10
    x[2] = -0.0
    x[3, :4] = torch.tensor([448.0, -448.0, 464.0, -464.0])
    x[4] = torch.tensor([1.0625, 1.1875, 2.125, 17.0, 272.0, 448.0, 0.5 * 2.0 ** -9, 1.5 * 2.0 ** -9] * 8)
    x[5, 7] = 1e4
    x[6, 3] = float("nan")
    x[7, 2], x[7, 9] = float("inf"), float("-inf")
    x[8] = 1e-38
    x = x.to(torch.bfloat16)
    wire, ref, pad = encode_pair((x,), width, 1, False, cuda)
    assert torch.equal(wire, ref)
    out = decoded(wire, 1, 16, width, 1, pad, torch.float32, cuda)[0]
    assert same(out, R.fp8_wire_decode(ref, 1, 16, width, 1, pad, torch.float32)[0])


def test_decode_every_code(cuda):
    """A wire written on the CPU with every byte value and a non-trivial scale."""
    import struct
    width = 256
    row = list(range(256)) + list(struct.pack("<f", 0.3))
    ref = torch.tensor([row, row[::-1][4:] + list(struct.pack("<f", 3e-5))], dtype=torch.uint8)
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        out = decoded(ref, 1, 2, width, 1, 0, dtype, cuda)[0]
        assert same(out, R.fp8_wire_decode(ref, 1, 2, width, 1, 0, dtype)[0])


@pytest.mark.parametrize("layout", ["mixed", "uniform", "last_stride_two", "single"])
@pytest.mark.parametrize("batch", [1, 2])
def test_mixed_stride_views_bit_exact(cuda, monkeypatch, layout, batch):
    """test_phaa_fp8_mixed_strides.py:9-48: views of a fused QKV projection (head slice 4:,
    permuted to [peer, seq, batch, head, width]) produce the same wire as contiguous copies,
    read in place; the mixed-stride counter moves for the mixed layout only."""
    peers, seq, heads, width = 2, 17, 14, 96
    g = torch.Generator(device=cuda).manual_seed(24)
    fused = torch.randn((batch, seq, 3 * heads * width), device=cuda, dtype=torch.bfloat16, generator=g)
    q, k, v = fused.chunk(3, dim=-1)
    if layout != "uniform":
        q, k = q.contiguous(), k.contiguous()
    if layout == "last_stride_two":
        v = v.repeat_interleave(2, dim=-1)[..., ::2]
    inputs = tuple(t.unflatten(-1, (peers, heads // peers, width))[:, :, :, 4:, :].permute(2, 1, 0, 3, 4)
                   for t in (q, k, v))
    if layout == "single":
        inputs = inputs[:1]
    wires = []

    def exchange(output, tensor, **kwargs):
        wires.append(tensor.clone())
        output.copy_(tensor)

    before = transport.mixed_stride_metrics()
    with patch.object(dist, "get_world_size", return_value=peers), \
            patch.object(dist, "all_to_all_single", side_effect=exchange):
        monkeypatch.setenv("XGEN_PHAA_FP8_MIXED_STRIDES", "0")
        old = tuple(torch.empty(t.shape, device=cuda, dtype=t.dtype) for t in inputs)
        transport.fp8_all_to_all_many(old, inputs, width, None)
        assert transport.mixed_stride_metrics() == before
        monkeypatch.setenv("XGEN_PHAA_FP8_MIXED_STRIDES", "1")
        new = tuple(torch.empty_like(t) for t in old)
        transport.fp8_all_to_all_many(new, inputs, width, None)
    assert torch.equal(wires[0], wires[1])
    assert all(torch.equal(a, b) for a, b in zip(old, new))
    expected = 1 if layout == "mixed" else 0
    assert transport.mixed_stride_metrics()["calls"] - before["calls"] == expected
    ref = R.fp8_wire_encode(tuple(t.cpu() for t in inputs), width, peers)
    assert torch.equal(wires[1].cpu(), ref)


@pytest.mark.parametrize("streams", [1, 3])
@pytest.mark.parametrize("seq", [17, 20])
@pytest.mark.parametrize("batch", [1, 2])
def test_peer_padding_preserves_transport(cuda, monkeypatch, streams, seq, batch):
    """test_phaa_fp8_alignment.py:24-53 through the transport entry point."""
    peers, heads, width = 2, 3, 128
    g = torch.Generator(device=cuda).manual_seed(42)
    tensors = tuple(torch.randn((peers, seq, batch, heads, width), device=cuda, dtype=torch.bfloat16, generator=g)
                    for _ in range(streams))
    wires = []

    def exchange(output, tensor, **kwargs):
        wires.append(tensor.clone())
        output.copy_(tensor)

    outputs = []
    with patch.object(dist, "get_world_size", return_value=peers), \
            patch.object(dist, "all_to_all_single", side_effect=exchange):
        monkeypatch.delenv("XGEN_PHAA_FP8_ALIGN16", raising=False)
        for enabled in (False, True):
            if enabled:
                monkeypatch.setenv("XGEN_PHAA_FP8_ALIGN16", "1")
            result = tuple(torch.empty_like(t) for t in tensors)
            transport.fp8_all_to_all_many(result, tensors, width, None)
            outputs.append(result)
    valid = seq * batch * heads * (width + 4) * streams
    old, new = wires[0].reshape(peers, -1), wires[1].reshape(peers, -1)
    assert wires[0].shape == (streams * peers * seq * batch * heads, width + 4)
    assert new.shape[1] % 16 == 0
    assert torch.equal(old, new[:, :valid])
    assert bool(torch.all(new[:, valid:] == 0))
    assert all(torch.equal(a, b) for a, b in zip(*outputs))
    for t, o in zip(tensors, outputs[0]):
        assert torch.nn.functional.cosine_similarity(t.float().flatten(), o.float().flatten(), dim=0) > 0.99


def test_wire_buffer_reused_padding_is_rewritten(cuda):
    """The encoder writes the zero tail itself: a send buffer full of garbage ends up equal to
    the oracle's wire after encoding into it."""
    peers, width = 2, 128
    t = qkv((peers, 17, 1, 3, width), 1, seed=9)
    wire, ref, pad = encode_pair(t, width, peers, True, cuda)
    assert pad > 0
    dirty = torch.full_like(wire, 0xAB, device=cuda)
    from xgen_amd import _native as N
    views, strides, (s, b, h) = transport._views(tuple(x.to(cuda) for x in t), width, peers)
    arr = (N._c_i64 * 4)(*strides[0])
    st = N.lib().xgen_fp8_wire_encode(N.DTYPE_BF16, 1, views[0].data_ptr(), None, None, arr, peers, s, b, h,
                                      width, pad, dirty.data_ptr(), N.stream_of(dirty))
    N.check(st, "xgen_fp8_wire_encode")
    assert torch.equal(dirty.cpu(), ref)


def test_h3_geometry_properties(cuda):
    """One GPU's Q/K/V share at H3 geometry (15,624 tokens x 24 heads x 128, read in place from a
    fused [M, 3d] projection output as [8 peers, M, 1, 3, 128] views): sampled rows bit-exact
    against the oracle at their wire positions, round-trip error bound on every row."""
    M, heads, width, peers = 15624, 24, 128, 8
    g = torch.Generator(device=cuda).manual_seed(1)
    fused = torch.randn((M, 3 * heads * width), device=cuda, dtype=torch.bfloat16, generator=g)
    views = tuple(t.unflatten(-1, (peers, heads // peers, width)).unsqueeze(1).permute(2, 0, 1, 3, 4)
                  for t in fused.chunk(3, dim=-1))
    assert views[0].shape == (peers, M, 1, heads // peers, width)
    wire, pad = transport.encode_wire(views, width, peers, align16=True)
    rows = M * heads
    pr = rows // peers
    outs = tuple(torch.empty((rows, width), device=cuda, dtype=torch.bfloat16) for _ in range(3))
    transport.decode_wire(wire, outs, width, peers, pad)
    per = wire.reshape(peers, -1)[:, :3 * pr * (width + 4)].reshape(peers, 3, pr, width + 4)
    idx = torch.randint(rows, (4096,), generator=torch.Generator().manual_seed(2))
    for s in range(3):
        src = views[s].reshape(rows, width)
        sample = src[idx.to(cuda)].cpu()
        q, sc = R.wire_rows_fp8(sample.float())
        got = per[:, s].reshape(rows, width + 4)[idx.to(cuda)].cpu()
        assert torch.equal(got[:, :width], q)
        assert torch.equal(got[:, width:].contiguous().view(torch.float32).reshape(-1), sc)
        xf = src.float()
        scale = (xf.abs().amax(-1, keepdim=True) / 448).clamp_min(1e-12)
        err = (outs[s].float() - xf).abs()
        bound = xf.abs() * (2.0 ** -4 + 2.0 ** -8) + scale * 2.0 ** -10
        assert bool(torch.all(err <= bound * (1 + 2.0 ** -8)))
    assert bool(torch.all(wire.reshape(peers, -1)[:, 3 * pr * (width + 4):] == 0))
