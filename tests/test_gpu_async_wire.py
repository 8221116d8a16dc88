"""GPU parity of the asynchronous FP8 exchange's layouts (xgen_fp8_wire_encode_masked,
xgen_fp8_wire_decode_strided, and xgen_amd.phaa.fp8_async_transport mirroring
x_base/x_base/phaa/fp8_async_transport.py): send bytes and decoded values bit-exact against the
oracle in every layout, and the reference test's check (x_base/tests/test_phaa_fp8.py:70-139) that a
head-parallel exchange gives the same result through the plain, direct-gather, direct-return and
fused-return-pack layouts, over a patched asynchronous collective."""
from unittest.mock import patch

import pytest
import torch
import torch.distributed as dist

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd.phaa import fp8_async_transport as T

pytestmark = pytest.mark.gpu


def same(a, b):
    """Bit equality of two CPU float tensors, NaN matching NaN whatever its payload."""
    nan_a, nan_b = torch.isnan(a), torch.isnan(b)
    if not torch.equal(nan_a, nan_b):
        return False
    bits = {torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.float16: torch.int16}[a.dtype]
    return torch.equal(a.view(bits)[~nan_a], b.view(bits)[~nan_b])


def pack(peers, outputs, tensors, width, **kw):
    with patch.object(dist, "get_world_size", return_value=peers):
        return T._pack_exchange(outputs, tensors, width, None, **kw)


@pytest.mark.parametrize("streams", [1, 3])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("form", ["shards", "rows"])
def test_plain_layout_bit_exact(cuda, streams, dtype, form):
    peers, seq, batch, heads, width = 2, 7, 2, 3, 64
    g = torch.Generator().manual_seed(streams + 10 * len(form))
    t = tuple((torch.randn((peers, seq, batch, heads, width), generator=g) *
               torch.logspace(-3, 3, heads)[:, None]).to(dtype) for _ in range(streams))
    if form == "rows":
        t = tuple(x.reshape(-1, width) for x in t)
    cu = tuple(x.to(cuda) for x in t)
    outs = tuple(torch.empty_like(x) for x in cu) if streams == 3 else None
    send, recv, rows = pack(peers, outs, cu, width)
    ref = R.fp8_async_encode(t, width, peers)
    assert torch.equal(send.cpu(), ref)
    recv.copy_(send)
    for out_dtype in (torch.bfloat16, torch.float32):
        got = tuple(torch.empty(x.shape, dtype=out_dtype, device=cuda) for x in cu)
        T._unpack_exchange(recv, got, rows)
        expect = R.fp8_async_decode(ref, [torch.empty(x.shape, dtype=out_dtype) for x in t], rows.rows, width, peers)
        assert all(same(a.cpu(), b) for a, b in zip(got, expect))


@pytest.mark.parametrize("valid", [1, 9, 16])
@pytest.mark.parametrize("layout", ["contiguous", "transposed", "channel_stride_two"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_return_pack_bit_exact(cuda, valid, layout, dtype):
    """RETURN_SEQ: an attention output [batch, heads, valid, D] packed as [peers, shard_seq, batch,
    heads] rows (zero rows past `valid`), then decoded through the return layout."""
    peers, shard_seq, batch, heads, width, hpp, start = 2, 8, 2, 3, 128, 5, 1
    g = torch.Generator().manual_seed(valid)
    base = torch.randn((batch, valid, heads, width), generator=g).to(dtype)
    attn_cpu = base.transpose(1, 2)
    attn = base.to(cuda).transpose(1, 2)          # [batch, heads, valid, D], seq stride heads * D
    if layout == "contiguous":
        attn = attn.contiguous()
    elif layout == "channel_stride_two":
        attn = attn.repeat_interleave(2, dim=-1)[..., ::2]
    send, recv, rows = pack(peers, None, (attn,), width, return_shard_seq=shard_seq)
    ref = R.fp8_async_encode((attn_cpu,), width, peers, return_shard_seq=shard_seq)
    assert torch.equal(send.cpu(), ref)
    recv.copy_(send)
    layout_args = (shard_seq, batch, peers, hpp, heads, start)
    out = torch.full((batch, shard_seq, peers * hpp * width), -3.0, dtype=dtype, device=cuda)
    expect = out.cpu()
    T._unpack_exchange(recv, (out,), rows, layout_args)
    R.fp8_async_decode(ref, (expect,), rows.rows, width, peers, layout=layout_args)
    assert same(out.cpu(), expect)


@pytest.mark.parametrize("gather", [1, 13, 24])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_direct_gather_bit_exact(cuda, gather, out_dtype):
    """GATHER_SEQ: Q/K/V head shards decode straight into [batch, heads, gather, D]."""
    peers, shard_seq, batch, heads, width = 2, 12, 2, 3, 64
    g = torch.Generator().manual_seed(gather)
    t = tuple(torch.randn((peers, shard_seq, batch, heads, width), generator=g).to(torch.bfloat16) for _ in range(3))
    outs = tuple(torch.full((batch, heads, gather, width), -3.0, dtype=out_dtype, device=cuda) for _ in range(3))
    send, recv, rows = pack(peers, outs, tuple(x.to(cuda) for x in t), width, direct_gather=True)
    ref = R.fp8_async_encode(t, width, peers)
    assert torch.equal(send.cpu(), ref)
    recv.copy_(send)
    T._unpack_exchange(recv, outs, rows)
    expect = R.fp8_async_decode(ref, [torch.empty((batch, heads, gather, width), dtype=out_dtype) for _ in range(3)],
                                rows.rows, width, peers, gather_seq=gather)
    assert all(same(a.cpu(), b) for a, b in zip(outs, expect))


def test_return_layout_leaves_other_heads(cuda):
    """Two head chunks of a [batch, seq, peers * heads_per_peer * D] output filled by two returns; the
    heads neither writes keep their values."""
    peers, sq, batch, hpp, width = 2, 6, 2, 5, 32
    out = torch.full((batch, sq, peers * hpp * width), 11.0, dtype=torch.bfloat16, device=cuda)
    expect = out.cpu()
    for chunk, start, seed in ((2, 0, 1), (2, 3, 2)):
        x = torch.randn((peers * sq * batch * chunk, width), generator=torch.Generator().manual_seed(seed))
        send, recv, rows = pack(peers, None, (x.to(torch.bfloat16).to(cuda),), width)
        recv.copy_(send)
        T._unpack_exchange(recv, (out,), rows, (sq, batch, peers, hpp, chunk, start))
        R.fp8_async_decode(send.cpu(), (expect,), rows.rows, width, peers, layout=(sq, batch, peers, hpp, chunk, start))
    assert same(out.cpu(), expect)
    untouched = out.view(batch, sq, peers, hpp, width)[:, :, :, 2:3]
    assert bool(torch.all(untouched == 11.0))


def test_return_layout_rejects_a_mismatch(cuda):
    peers, sq, batch, hpp, width = 2, 6, 2, 5, 32
    x = torch.zeros((peers * sq * batch * 2, width), dtype=torch.bfloat16, device=cuda)
    send, recv, rows = pack(peers, None, (x,), width)
    out = torch.empty((batch, sq, peers * hpp * width), dtype=torch.bfloat16, device=cuda)
    for bad in ((sq, batch, peers, hpp, 2, 4), (sq, batch, peers + 1, hpp, 2, 0), (sq - 1, batch, peers, hpp, 2, 0)):
        with pytest.raises(ValueError, match="return layout"):
            T._unpack_exchange(recv, (out,), rows, bad)


class LocalWork:
    """The work handle of the patched collective: the copy ran on the collective stream."""

    def __init__(self, done):
        self.done = done

    def block_current_stream(self):
        torch.cuda.current_stream().wait_event(self.done)


def head_parallel(q, k, v, *, peers, heads, width, chunks, pad, mode):
    """One head-parallel attention exchange in the shape of phaa_attention.py:155-338 with an
    elementwise stand-in for the attention: the chunk's Q/K/V head shards gathered, combined, returned
    and placed into the [batch, seq, heads * D] output."""
    B, S, _ = q.shape
    hpd = heads // peers
    sizes = [hpd // chunks + (1 if i < hpd % chunks else 0) for i in range(chunks)]
    offsets = [sum(sizes[:i]) for i in range(chunks)]
    direct_gather = mode in ("direct_gather",)
    direct_return = mode in ("direct_return", "fused", "direct_gather")
    fused = mode in ("fused", "direct_gather")
    out = torch.empty((B, S, heads * width), dtype=q.dtype, device=q.device)
    split = [t.unflatten(-1, (heads, width)).unflatten(2, (peers, hpd)) for t in (q, k, v)]
    valid = peers * S - pad
    for size, off in zip(sizes, offsets):
        inputs = tuple(t[:, :, :, off:off + size, :].permute(2, 1, 0, 3, 4) for t in split)
        if direct_gather:
            bufs = tuple(torch.empty((B, size, valid, width), dtype=q.dtype, device=q.device) for _ in range(3))
        else:
            bufs = tuple(torch.empty((peers, S, B, size, width), dtype=q.dtype, device=q.device) for _ in range(3))
        pending = T.submit_fp8_exchange(bufs, inputs, width, None, direct_gather=direct_gather)
        T.finish_fp8_exchange(pending)
        if direct_gather:
            qa, ka, va = bufs
        else:
            qa, ka, va = (b.flatten(0, 1).permute(1, 2, 0, 3).narrow(2, 0, valid) for b in bufs)
        attn = qa.float() * 0.5 + ka.float() - va.float() * 0.25
        attn = attn.to(q.dtype)                                     # [B, size, valid, D]
        if fused:
            pending = T.submit_fp8_exchange(None, (attn,), width, None, return_shard_seq=S)
        else:
            padded = torch.cat([attn, attn.new_zeros((B, size, pad, width))], dim=2)
            hidden = padded.unflatten(2, (peers, -1)).permute(2, 3, 0, 1, 4).flatten(-2, -1)
            back = None if direct_return else (torch.empty(hidden.shape, dtype=q.dtype, device=q.device),)
            pending = T.submit_fp8_exchange(back, (hidden,), width, None)
        if direct_return:
            T.finish_fp8_exchange(pending, output=out, return_layout=(S, B, peers, hpd, size, off))
        else:
            T.finish_fp8_exchange(pending)
            got = pending.outputs[0].view(peers, S, B, size, width).permute(2, 1, 0, 3, 4)
            out.view(B, S, peers, hpd, width)[:, :, :, off:off + size] = got
    return out


@pytest.mark.parametrize("batch", [1, 2])
def test_layouts_agree_through_a_patched_async_collective(cuda, batch):
    """test_phaa_fp8.py:70-139 on this transport: the same exchange through every layout gives the
    same output, bit for bit; every collective is asynchronous over uint8 rows of D + 4 bytes."""
    peers, heads, width, S, chunks, pad = 2, 14, 64, 32, 4, 1
    g = torch.Generator(device=cuda).manual_seed(42)
    q, k, v = (torch.randn((batch, S, heads * width), dtype=torch.bfloat16, device=cuda, generator=g)
               for _ in range(3))
    collective = torch.cuda.Stream()
    calls = []

    def local_copy(output, tensor, **kwargs):
        calls.append((output.dtype, tensor.dtype, tuple(tensor.shape), kwargs.get("async_op")))
        collective.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(collective):
            output.copy_(tensor)
            return LocalWork(collective.record_event())

    results = {}
    with patch.object(dist, "get_world_size", return_value=peers), \
            patch.object(dist, "all_to_all_single", side_effect=local_copy):
        for mode in ("plain", "direct_return", "fused", "direct_gather"):
            results[mode] = head_parallel(q, k, v, peers=peers, heads=heads, width=width, chunks=chunks, pad=pad,
                                          mode=mode)
    torch.cuda.synchronize()
    assert len(calls) == 4 * 2 * chunks
    assert all(o == t == torch.uint8 and shape[-1] == width + 4 and a for o, t, shape, a in calls)
    for mode in ("direct_return", "fused", "direct_gather"):
        assert torch.equal(results["plain"], results[mode]), mode
    assert torch.isfinite(results["plain"].float()).all()


def test_h3_geometry_direct_gather_and_return_pack(cuda):
    """One GPU's share at H3 geometry (15,624 tokens, 24 heads of 128 over 8 peers, one chunk of all 3
    local heads): direct-gather decode and fused return pack; sampled rows bit-exact against the
    oracle's per-row quantizer at their layout positions, round-trip bound on every value."""
    M, heads, width, peers = 15624, 24, 128, 8
    hpd = heads // peers
    g = torch.Generator(device=cuda).manual_seed(3)
    fused = torch.randn((1, M, 3 * heads * width), device=cuda, dtype=torch.bfloat16, generator=g)
    views = tuple(t.unflatten(-1, (heads, width)).unflatten(2, (peers, hpd)).permute(2, 1, 0, 3, 4)
                  for t in fused.chunk(3, dim=-1))                 # [peers, M, 1, hpd, D]
    seen = peers * M - 5
    outs = tuple(torch.empty((1, hpd, seen, width), dtype=torch.bfloat16, device=cuda) for _ in range(3))
    send, recv, rows = pack(peers, outs, views, width, direct_gather=True)
    recv.copy_(send)
    T._unpack_exchange(recv, outs, rows)
    idx = torch.randint(seen, (2048,), generator=torch.Generator().manual_seed(4))
    for src, got in zip(views, outs):
        # gathered position p * M + s of head h is row (p, s, 0, h) of the shards
        full = src.reshape(peers * M, hpd, width).permute(1, 0, 2)          # [hpd, peers * M, D]
        sample = full[:, idx.to(cuda)].float().cpu().reshape(-1, width)
        q, s = R.wire_rows_fp8(sample)
        expect = (q.view(torch.float8_e4m3fn).float() * s[:, None]).to(torch.bfloat16)
        assert torch.equal(got[0][:, idx.to(cuda)].cpu().reshape(-1, width), expect)
        xf = full[:, :seen].float()
        scale = (xf.abs().amax(-1, keepdim=True) / 448).clamp_min(1e-12)
        err = (got[0].float() - xf).abs()
        assert bool(torch.all(err <= (xf.abs() * (2.0 ** -4 + 2.0 ** -8) + scale * 2.0 ** -10) * (1 + 2.0 ** -8)))
    attn = outs[0]                                                           # [1, hpd, seen, D]
    send, recv, rows = pack(peers, None, (attn,), width, return_shard_seq=M)
    wire = send.view(peers, M, 1, hpd, width + 4)
    flat = wire.reshape(peers * M, hpd, width + 4)
    assert bool(torch.all(flat[seen:, :, :width] == 0))
    sc = flat[:, :, width:].contiguous().view(torch.float32).reshape(peers * M, hpd)
    assert bool(torch.all(sc[seen:] == 1e-12))
    pos = idx.to(cuda)
    q, s = R.wire_rows_fp8(attn[0][:, pos].float().cpu().reshape(-1, width))
    assert torch.equal(flat[pos][:, :, :width].permute(1, 0, 2).reshape(-1, width).cpu(), q)
    assert torch.equal(sc[pos].t().reshape(-1).cpu(), s)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_return_pack_special_rows_and_odd_geometry(cuda, dtype):
    """Three peers, three batches, the narrowest rows (width 4) and special rows in a ragged
    attention output: zero, tiny, outlier, NaN and Inf rows, bytes and scales bit-exact against the
    oracle, decoded through the return layout (NaN matching NaN)."""
    peers, shard_seq, batch, heads, width, valid = 3, 5, 3, 2, 4, 13
    g = torch.Generator().manual_seed(11)
    attn = torch.randn((batch, heads, valid, width), generator=g)
    attn[0, 0, 0] = 0.0
    attn[0, 1, 1] = 1e-30
    attn[1, 0, 2, 1] = 3e4
    attn[1, 1, 3, 2] = float("nan")
    attn[2, 0, 4, 0] = float("inf")
    attn = attn.to(dtype)
    send, recv, rows = pack(peers, None, (attn.to(cuda),), width, return_shard_seq=shard_seq)
    ref = R.fp8_async_encode((attn,), width, peers, return_shard_seq=shard_seq)
    assert torch.equal(send.cpu(), ref)
    recv.copy_(send)
    layout = (shard_seq, batch, peers, heads + 1, heads, 1)
    out = torch.full((batch, shard_seq, peers * (heads + 1) * width), 5.0, dtype=dtype, device=cuda)
    expect = out.cpu()
    T._unpack_exchange(recv, (out,), rows, layout)
    R.fp8_async_decode(ref, (expect,), rows.rows, width, peers, layout=layout)
    assert same(out.cpu(), expect)


@pytest.mark.parametrize("width", [4, 12, 68, 260])
def test_direct_gather_widths(cuda, width):
    """Row widths off the 16-byte chunk (the kernels' 4-value and element-wise forms)."""
    peers, shard_seq, batch, heads, gather = 2, 3, 1, 2, 5
    g = torch.Generator().manual_seed(width)
    t = tuple(torch.randn((peers, shard_seq, batch, heads, width), generator=g).to(torch.bfloat16) for _ in range(3))
    outs = tuple(torch.empty((batch, heads, gather, width), dtype=torch.float32, device=cuda) for _ in range(3))
    send, recv, rows = pack(peers, outs, tuple(x.to(cuda) for x in t), width, direct_gather=True)
    ref = R.fp8_async_encode(t, width, peers)
    assert torch.equal(send.cpu(), ref)
    recv.copy_(send)
    T._unpack_exchange(recv, outs, rows)
    expect = R.fp8_async_decode(ref, [torch.empty((batch, heads, gather, width)) for _ in range(3)], rows.rows,
                                width, peers, gather_seq=gather)
    assert all(same(a.cpu(), b) for a, b in zip(outs, expect))
