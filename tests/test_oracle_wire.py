"""Pins the oracle's FP8 wire codec (oracle/ref.py fp8_wire_encode / fp8_wire_decode) to the
reference's transport (x_base/x_base/phaa/fp8_transport.py:26-144): the facts its own tests
assert, its per-row index formula, all-to-all delivery, the already-pinned row quantizer where
the scale floors agree, closed forms at the 1e-12 floor, and an exhaustive check of the
kernels' division at that floor."""
import concurrent.futures
import struct

import numpy as np
import pytest
import torch

import oracle.ref as R


def qkv(peers, seq, batch, heads, width, streams, seed=42, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn((peers, seq, batch, heads, width), generator=g).to(dtype) for _ in range(streams))


@pytest.mark.parametrize("streams", [1, 3])
@pytest.mark.parametrize("seq", [17, 20])
@pytest.mark.parametrize("batch", [1, 2])
def test_peer_padding_facts_of_the_reference_test(streams, seq, batch):
    """test_phaa_fp8_alignment.py:30-53: unpadded wire (streams*rows, width+4); padded rows are
    16-byte multiples holding the unpadded bytes then zeros; decoded outputs identical."""
    peers, heads, width = 2, 3, 128
    t = qkv(peers, seq, batch, heads, width, streams)
    old = R.fp8_wire_encode(t, width, peers, align16=False)
    new = R.fp8_wire_encode(t, width, peers, align16=True)
    rows = peers * seq * batch * heads
    valid = seq * batch * heads * (width + 4) * streams
    assert old.dtype == new.dtype == torch.uint8
    assert old.shape == (streams * rows, width + 4)
    pad = R.wire_peer_padding(streams, rows // peers, width, True)
    if pad:
        assert new.shape == (peers, valid + pad)
    assert new.reshape(peers, -1).shape[1] % 16 == 0
    assert torch.equal(old.reshape(peers, -1), new.reshape(peers, -1)[:, :valid])
    assert bool(torch.all(new.reshape(peers, -1)[:, valid:] == 0))
    a = R.fp8_wire_decode(old, streams, rows, width, peers, 0)
    b = R.fp8_wire_decode(new, streams, rows, width, peers, pad)
    assert all(torch.equal(x, y) for x, y in zip(a, b))


def test_row_is_head_dim_plus_four_bytes():
    """test_phaa_fp8.py:57-59: uint8 wire, rows of 64 e4m3 bytes + 4 scale bytes."""
    t = qkv(2, 16, 1, 7, 64, 3)
    w = R.fp8_wire_encode(t, 64, 2)
    assert w.dtype == torch.uint8 and w.shape[-1] == 64 + 4


def _rows_quantized(t, width):
    """Bytes and scales of each row, from the pinned per-row quantizer (floor inactive here)."""
    q, s = R.quantize_rows_fp8(t.reshape(-1, width))
    return q.view(torch.uint8).reshape(-1, width), s


@pytest.mark.parametrize("streams,align16", [(1, False), (3, False), (1, True), (3, True)])
def test_layout_equals_the_reference_index_formula(streams, align16):
    """The block-wise oracle equals the reference's per-row addressing, fp8_transport.py:53-63:
    wire_row = row + (row // PEER_ROWS * (STREAMS - 1) + slot) * PEER_ROWS,
    offset = wire_row * (WIDTH + 4) + peer * PEER_PADDING, scale at offset + WIDTH,
    zeros at peer * (PEER_ROWS*STREAMS*(WIDTH+4) + PEER_PADDING) + PEER_ROWS*STREAMS*(WIDTH+4)."""
    peers, seq, batch, heads, width = 3, 5, 2, 1, 12
    t = qkv(peers, seq, batch, heads, width, streams, seed=7)
    rows = peers * seq * batch * heads
    peer_rows = rows // peers
    pad = R.wire_peer_padding(streams, peer_rows, width, align16)
    wire = R.fp8_wire_encode(t, width, peers, align16).reshape(-1).numpy()
    assert wire.size == peers * (peer_rows * streams * (width + 4) + pad)
    for slot in range(streams):
        q, s = _rows_quantized(t[slot], width)
        for row in range(rows):
            peer = row // peer_rows
            wire_row = row + (row // peer_rows * (streams - 1) + slot) * peer_rows
            offset = wire_row * (width + 4) + peer * pad
            assert np.array_equal(wire[offset:offset + width], q[row].numpy())
            assert wire[offset + width:offset + width + 4].tobytes() == struct.pack("<f", float(s[row]))
    for peer in range(peers):
        tail = peer * (peer_rows * streams * (width + 4) + pad) + peer_rows * streams * (width + 4)
        assert not wire[tail:tail + pad].any()


def test_simulated_all_to_all_delivers_each_peers_rows():
    """P ranks exchange equal chunks of their send buffers (all_to_all_single semantics): rank j
    decodes, for each stream, rank i's rows destined to peer j as rows [i*PR, (i+1)*PR) — the
    per-row quantize/dequantize of rank i's tensor[j]."""
    peers, seq, batch, heads, width, streams = 3, 4, 2, 2, 32, 3
    ranks = [qkv(peers, seq, batch, heads, width, streams, seed=100 + i) for i in range(peers)]
    sends = [R.fp8_wire_encode(t, width, peers, align16=True).reshape(peers, -1) for t in ranks]
    rows = peers * seq * batch * heads
    pr = rows // peers
    pad = R.wire_peer_padding(streams, pr, width, True)
    for j in range(peers):
        recv = torch.cat([sends[i][j:j + 1] for i in range(peers)], dim=0)
        out = R.fp8_wire_decode(recv, streams, rows, width, peers, pad, torch.float32)
        for i in range(peers):
            for s in range(streams):
                q, sc = R.quantize_rows_fp8(ranks[i][s][j].reshape(-1, width))
                expect = q.float() * sc[:, None]
                assert torch.equal(out[s][i * pr:(i + 1) * pr], expect)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_bytes_and_scales_equal_the_row_quantizer_above_the_floor(dtype):
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(64, 96, generator=g) * torch.logspace(-3, 3, 64)[:, None]).to(dtype)
    wire = R.fp8_wire_encode((x,), 96, 1)
    q, s = R.quantize_rows_fp8(x)
    assert torch.equal(wire[:, :96], q.view(torch.uint8))
    assert torch.equal(wire[:, 96:].contiguous().view(torch.float32).reshape(-1), s)


def test_scale_floor_closed_forms():
    """A zero row: scale float32(1e-12), zero bytes.  A row of bf16 values below 448e-12: scale
    exactly float32(1e-12) and bytes e4m3(x / 1e-12) (IEEE float32 division, the pinned C encoder)."""
    floor32 = np.float32(1e-12)
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    x[1] = (torch.linspace(-1, 1, 64) * 3e-10).to(torch.bfloat16)
    wire = R.fp8_wire_encode((x,), 64, 1)
    scales = wire[:, 64:].contiguous().view(torch.float32).reshape(-1).numpy()
    assert scales.view(np.uint32).tolist() == [floor32.view(np.uint32)] * 2
    assert not wire[0, :64].any()
    expect = R.e4m3_encode(x[1].float().numpy() / floor32)
    assert np.array_equal(wire[1, :64].numpy(), expect)
    assert wire[1, :64].numpy().any()


def test_decode_of_every_code_equals_the_e4m3_table():
    """One row holding bytes 0..255 with scale 1 and 2^-3 decodes to the (pinned) e4m3 table,
    exactly in float32 and rounded to nearest even in bfloat16."""
    table = R.e4m3_decode_table()
    for scale in (1.0, 0.125):
        row = np.concatenate([np.arange(256, dtype=np.uint8), np.frombuffer(struct.pack("<f", scale), np.uint8)])
        wire = torch.from_numpy(row.copy()).reshape(1, 260)
        f32 = R.fp8_wire_decode(wire, 1, 1, 256, 1, 0, torch.float32)[0].reshape(-1).numpy()
        assert np.array_equal(f32, table * np.float32(scale), equal_nan=True)
        bf = R.fp8_wire_decode(wire, 1, 1, 256, 1, 0, torch.bfloat16)[0].reshape(-1).float().numpy()
        assert np.array_equal(bf, R.round_bf16_np(table * np.float32(scale)), equal_nan=True)


def test_round_trip_error_bound_and_cosine():
    """|decode - x| <= |x| * 2^-4 + scale * 2^-10 (e4m3 rounding: half an ulp of a 3-bit mantissa,
    or of the subnormal step 2^-9) plus the bf16 output rounding; cosine > 0.99 as
    test_phaa_fp8.py:66 asserts for the whole transport."""
    t = qkv(2, 32, 1, 14, 64, 3, seed=42)
    rows = 2 * 32 * 14
    wire = R.fp8_wire_encode(t, 64, 2)
    out = R.fp8_wire_decode(wire, 3, rows, 64, 2, 0, torch.bfloat16)
    for x, y in zip(t, out):
        xf = x.float().reshape(rows, 64)
        scale = (xf.abs().amax(-1, keepdim=True) / 448).clamp_min(1e-12)
        err = (y.float() - xf).abs()
        bound = xf.abs() * 2.0 ** -4 + scale * 2.0 ** -10
        assert bool(torch.all(err <= bound * (1 + 2.0 ** -8) + xf.abs() * 2.0 ** -8))
        assert torch.nn.functional.cosine_similarity(xf.flatten(), y.float().flatten(), dim=0) > 0.99


def test_non_finite_rows_follow_nan_propagation():
    """Parity unpinned (the reference leaves NaN to its min/max lowering): a NaN row gets a NaN
    scale and NaN bytes; an inf row gets scale inf, NaN bytes for +-inf and signed zeros elsewhere."""
    x = torch.ones(2, 8, dtype=torch.bfloat16)
    x[0, 3] = float("nan")
    x[1, 2], x[1, 5], x[1, 6] = float("inf"), float("-inf"), -1.0
    wire = R.fp8_wire_encode((x,), 8, 1)
    s = wire[:, 8:].contiguous().view(torch.float32).reshape(-1)
    assert torch.isnan(s[0]) and torch.isinf(s[1])
    assert (wire[0, :8] == 0x7F).all()
    assert wire[1, :8].tolist() == [0, 0, 0x7F, 0, 0, 0x7F, 0x80, 0]


def test_wire_division_exhaustive_at_the_floor():
    """Every bf16 (x, amax) pair with amax up to 2^-29 (the 1e-12 scale floor is active below
    448e-12): the kernels' division (div_by_row_scale) gives IEEE's e4m3 byte.  Above the floor the wire
    scale equals the row quantizer's, covered by test_fast_division_exhaustive; f16 amax never
    reaches the floor (smallest subnormal 2^-24)."""
    L = R.clib()
    hi = 0x3100
    bounds = np.concatenate([[1], (np.sqrt(np.linspace(0, 1, 9)[1:]) * hi).astype(np.int64) + 1])
    with concurrent.futures.ThreadPoolExecutor(8) as pool:
        bad = sum(pool.map(lambda i: L.oracle_check_wire_division(0, int(bounds[i]), int(bounds[i + 1] - 1)),
                           range(8)))
    assert bad == 0


# --------------------------------------------------------------------------- asynchronous layouts
# fp8_async_encode / fp8_async_decode restate the reference's per-row index formulas
# (fp8_async_transport.py:13-80); each is held here to the synchronous codec composed with plain
# torch reshapes, permutes and slices, which share none of that index arithmetic.


@pytest.mark.parametrize("streams", [1, 3])
@pytest.mark.parametrize("batch", [1, 2])
def test_async_plain_layout_is_the_unpadded_sync_wire(streams, batch):
    peers, seq, heads, width = 2, 5, 3, 64
    t = qkv(peers, seq, batch, heads, width, streams, seed=7)
    wire = R.fp8_async_encode(t, width, peers)
    assert torch.equal(wire, R.fp8_wire_encode(t, width, peers, align16=False))
    rows = peers * seq * batch * heads
    outs = R.fp8_async_decode(wire, [torch.empty(rows, width, dtype=torch.float32) for _ in range(streams)],
                              rows, width, peers)
    ref = R.fp8_wire_decode(wire, streams, rows, width, peers, 0, torch.float32)
    assert all(torch.equal(a, b) for a, b in zip(outs, ref))


@pytest.mark.parametrize("valid", [1, 7, 11, 12])
@pytest.mark.parametrize("batch", [1, 2])
def test_async_return_pack_is_the_sync_wire_of_the_padded_permuted_output(valid, batch):
    """RETURN_SEQ: an attention output [batch, heads, valid, D] travels as [peers, shard_seq, batch,
    heads] rows; positions past `valid` as zero rows (scale 1e-12, zero bytes)."""
    peers, shard_seq, heads, width = 3, 4, 2, 32
    g = torch.Generator().manual_seed(valid + 10 * batch)
    out = torch.randn((batch, heads, valid, width), generator=g).to(torch.bfloat16)
    wire = R.fp8_async_encode((out,), width, peers, return_shard_seq=shard_seq)
    padded = torch.zeros((batch, heads, peers * shard_seq, width), dtype=out.dtype)
    padded[:, :, :valid] = out
    rows_view = padded.reshape(batch, heads, peers, shard_seq, width).permute(2, 3, 0, 1, 4).contiguous()
    assert torch.equal(wire, R.fp8_wire_encode((rows_view,), width, peers))
    rows = wire.reshape(peers, shard_seq, batch, heads, width + 4)
    dead = rows[:, :, :, :, :width].reshape(peers * shard_seq, -1)[valid:]
    assert bool(torch.all(dead == 0))
    scales = rows[..., width:].contiguous().view(torch.float32).reshape(peers * shard_seq, -1)[valid:]
    assert bool(torch.all(scales == torch.tensor(1e-12, dtype=torch.float32)))


@pytest.mark.parametrize("gather", [1, 6, 9, 10])
def test_async_direct_gather_is_the_sync_decode_permuted(gather):
    """GATHER_SEQ: Q/K/V head shards [peers, shard_seq, batch, heads, D] decode into [batch, heads,
    gather, D] attention inputs; positions at or past `gather` are dropped."""
    peers, shard_seq, batch, heads, width = 2, 5, 2, 3, 16
    t = qkv(peers, shard_seq, batch, heads, width, 3, seed=gather)
    wire = R.fp8_async_encode(t, width, peers)
    rows = peers * shard_seq * batch * heads
    sentinel = -7.0
    outs = [torch.full((batch, heads, gather, width), sentinel) for _ in range(3)]
    R.fp8_async_decode(wire, outs, rows, width, peers, gather_seq=gather)
    plain = R.fp8_wire_decode(wire, 3, rows, width, peers, 0, torch.float32)
    for got, flat in zip(outs, plain):
        full = flat.reshape(peers * shard_seq, batch, heads, width).permute(1, 2, 0, 3)
        assert torch.equal(got, full[:, :, :gather])


@pytest.mark.parametrize("start", [0, 2])
def test_async_return_layout_is_the_sync_decode_placed(start):
    """CHUNK_HEADS / HEAD_START: one chunk of `chunk` heads per peer decodes into its place in a
    [batch, sq, peers * heads_per_peer * D] output; the other heads stay as they were."""
    peers, sq, batch, chunk, hpp, width = 2, 3, 2, 2, 5, 8
    g = torch.Generator().manual_seed(start)
    x = torch.randn((peers * sq * batch * chunk, width), generator=g)
    wire = R.fp8_async_encode((x,), width, peers)
    rows = x.shape[0]
    output = torch.full((batch, sq, peers * hpp * width), -7.0)
    expect = output.clone()
    R.fp8_async_decode(wire, (output,), rows, width, peers, layout=(sq, batch, peers, hpp, chunk, start))
    flat = R.fp8_wire_decode(wire, 1, rows, width, peers, 0, torch.float32)[0]
    placed = flat.reshape(peers, sq, batch, chunk, width).permute(2, 1, 0, 3, 4)
    expect.view(batch, sq, peers, hpp, width)[:, :, :, start:start + chunk] = placed
    assert torch.equal(output, expect)


def test_async_return_round_trip():
    """The fused return pack decoded through the return layout puts every valid position of every
    head back (head chunk at head_start), as the unfused return does."""
    peers, shard_seq, batch, heads, width, valid, hpp, start = 2, 3, 1, 2, 16, 5, 4, 1
    g = torch.Generator().manual_seed(3)
    attn = torch.randn((batch, heads, valid, width), generator=g).to(torch.bfloat16)
    wire = R.fp8_async_encode((attn,), width, peers, return_shard_seq=shard_seq)
    rows = peers * shard_seq * batch * heads
    output = torch.zeros((batch, shard_seq, peers * hpp * width), dtype=torch.float32)
    R.fp8_async_decode(wire, (output,), rows, width, peers, layout=(shard_seq, batch, peers, hpp, heads, start))
    got = output.view(batch, shard_seq, peers, hpp, width)[:, :, :, start:start + heads]
    got = got.permute(0, 3, 2, 1, 4).reshape(batch, heads, peers * shard_seq, width)
    scale = (attn.float().abs().amax(-1, keepdim=True) / 448).clamp_min(1e-12)
    err = (got[:, :, :valid] - attn.float()).abs()
    assert bool(torch.all(err <= attn.float().abs() * 2.0 ** -4 + scale * 2.0 ** -9))
    assert bool(torch.all(got[:, :, valid:] == 0))
