"""Pins the oracle's INT8 per-row quantizer (f2bc_kernel.asc:89-107) by a second
restatement and by the closed-form properties the arithmetic fixes."""
import numpy as np
import pytest
import torch

import oracle.ref as R


def rows(dtype):
    torch.manual_seed(0)
    x = torch.randn(96, 320)
    x[:8] *= torch.logspace(-20, 20, 8)[:, None]
    x[8] = 0
    x[9] = -0.0
    x[10, 5] = float("inf")
    x[11, 9] = float("nan")
    x[12] = torch.linspace(-127, 127, 320)
    return x.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_torch_restatement_equals_c(dtype):
    x = rows(dtype)
    q_t, s_t = R.quantize_rows_int8(x)
    q_c, s_c = R.quantize_rows_c(x, "int8")
    assert torch.equal(q_t, q_c)
    assert torch.equal(s_t.view(torch.int32), s_c.view(torch.int32))


def test_range_and_extremes():
    x = rows(torch.bfloat16)[:8].float()
    x = torch.cat([x, torch.randn(64, 320)]).to(torch.bfloat16)
    q, s = R.quantize_rows_int8(x)
    assert q.abs().max() <= 127
    am = x.float().abs().argmax(dim=-1)
    picked = q.gather(1, am[:, None]).squeeze(1)
    assert (picked.abs() == 127).all()
    # |x - q * s| <= s/2 (+ a few float32 ulps of the dequantized value)
    err = (x.float() - q.float() * s[:, None]).abs()
    bound = s[:, None] * 0.5 + x.float().abs() * 2e-6 + 1e-30
    assert (err <= bound).all()


def test_round_half_to_even_ties():
    # amax = 127 -> alpha = 127/127 = 1 exactly, so x*alpha = x: bf16 halves are exact ties
    vals = torch.tensor([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5, -126.5, 0.25, 64.5])
    q, s = R.quantize_rows_int8(vals[None].to(torch.bfloat16))
    assert q[0].tolist() == [127, 0, 2, 2, 0, -2, -2, 4, 126, -126, 0, 64]
    assert s[0].item() == np.float32(127.0) * np.float32(np.float32(1.0) / np.float32(127.0))


def test_zero_row_gives_zero_scale_and_bytes():
    # npu_fusion/f1b/op_kernel/swiglu_quant_kernel.asc:72-75
    q, s = R.quantize_rows_int8(torch.zeros(3, 64, dtype=torch.bfloat16))
    assert (q == 0).all() and (s == 0).all()


def test_scale_uses_reciprocal_multiplier():
    # scale = amax * fl(1/127), not amax / 127 (f2bc_kernel.asc:97): differs on some amax
    amax = torch.tensor([3.0, 5.0, 7.0, 1e-3, 123.456], dtype=torch.float32)
    x = torch.zeros(5, 16)
    x[:, 0] = amax
    _, s = R.quantize_rows_int8(x.to(torch.bfloat16))
    a = x[:, 0].to(torch.bfloat16).float()
    assert torch.equal(s, a * (torch.tensor(1.0) / 127.0))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_subnormal_amax_row_quantizes_to_zeros(dtype):
    """127/amax overflows for a subnormal amax: every product is non-finite or
    -0 * inf = NaN, and the row comes out as zeros (the flushed-zero-row rule),
    in the torch and the C restatement alike."""
    tiny = 2.0 ** -130 if dtype == torch.bfloat16 else 2.0 ** -24
    x = torch.zeros(2, 64)
    x[0, :] = -0.0
    x[0, 3] = tiny
    x[1, 5] = -tiny
    x = x.to(dtype)
    q, s = R.quantize_rows_int8(x)
    qc, sc = R.quantize_rows_c(x, "int8")
    if dtype == torch.bfloat16:   # f16's smallest subnormal still gives a finite 127/amax
        assert (q == 0).all()
    assert torch.equal(q, qc) and torch.equal(s.view(torch.int32), sc.view(torch.int32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_symmetries(dtype):
    """Negating a row negates every byte and keeps its scale (round half to even and the max are
    symmetric); scaling a row by 2^k keeps every byte and scales the scale by exactly 2^k (the
    multiplier 127/amax moves by 2^-k, each product is unchanged); permuting a row's columns permutes
    its bytes."""
    torch.manual_seed(5)
    x = (torch.randn(40, 200) * torch.logspace(-2, 2, 40)[:, None]).to(dtype)
    q, s = R.quantize_rows_int8(x)
    qn, sn = R.quantize_rows_int8(-x)
    assert torch.equal(qn, -q) and torch.equal(sn, s)
    for k in (-3, 1, 4):
        qk, sk = R.quantize_rows_int8((x.float() * 2.0 ** k).to(dtype))
        assert torch.equal(qk, q) and torch.equal(sk, s * 2.0 ** k)
    perm = torch.randperm(200, generator=torch.Generator().manual_seed(6))
    qp, sp = R.quantize_rows_int8(x[:, perm])
    assert torch.equal(qp, q[:, perm]) and torch.equal(sp, s)


# ------------------------------------------------------------------ merge + quant
def _reference_copy(back_recv):
    """The reference kernel's copy, restated from its DataCopyPad parameters
    (merge_quant_kernel.asc:25-29): for each row and owner, 7 blocks of 512 bytes read from
    element (owner * seq + row) * 256 at a source stride of (4 * seq - 1) * 512 bytes between
    blocks, written contiguously from element owner * 1792 of the row."""
    flat = back_recv.reshape(-1)
    seq = back_recv.shape[2]
    rows = torch.empty((seq, 7168), dtype=back_recv.dtype)
    for row in range(seq):
        for owner in range(4):
            src = (owner * seq + row) * 256
            for block in range(7):
                rows[row, owner * 1792 + block * 256: owner * 1792 + (block + 1) * 256] = \
                    flat[src + block * 4 * seq * 256: src + block * 4 * seq * 256 + 256]
    return rows


@pytest.mark.parametrize("seq", [1, 3, 17])
def test_merge_rows_is_the_reference_copy(seq):
    g = torch.Generator().manual_seed(seq)
    x = torch.randn((7, 4, seq, 1, 256), generator=g).to(torch.bfloat16)
    assert torch.equal(R.merge_rows(x), _reference_copy(x))
    # plausible mistakes fail it: chunk-major columns, or the owner and chunk axes read swapped
    wrong_order = x.permute(3, 2, 0, 1, 4).reshape(seq, 7168)
    wrong_axes = x.reshape(4, 7, seq, 1, 256).permute(3, 2, 0, 1, 4).reshape(seq, 7168)
    assert not torch.equal(wrong_order, _reference_copy(x))
    assert not torch.equal(wrong_axes, _reference_copy(x))


def test_merge_rows_general_geometry():
    """Row b * seq + s, column (o * splits + c) * chunk + j holds back_recv[c, o, s, b, j]
    (element by element, on a batch of 2)."""
    splits, owners, seq, batch, chunk = 3, 2, 4, 2, 8
    x = torch.arange(splits * owners * seq * batch * chunk, dtype=torch.float32).reshape(
        splits, owners, seq, batch, chunk)
    rows = R.merge_rows(x)
    assert rows.shape == (batch * seq, owners * splits * chunk)
    for c in range(splits):
        for o in range(owners):
            for s in range(seq):
                for b in range(batch):
                    col = (o * splits + c) * chunk
                    assert torch.equal(rows[b * seq + s, col: col + chunk], x[c, o, s, b])


def test_merge_quant_is_the_row_quantizer_of_the_merged_rows():
    g = torch.Generator().manual_seed(5)
    x = torch.randn((7, 4, 9, 1, 256), generator=g).to(torch.bfloat16)
    x[:, :, 2] = 0  # a zero row: zero bytes and scale
    q, s = R.merge_quant(x)
    rq, rs = R.quantize_rows_int8(_reference_copy(x))
    assert torch.equal(q, rq) and torch.equal(s, rs)
    assert s[2] == 0 and not q[2].any()
    q8, s8 = R.merge_quant(x, out="fp8")
    f8, fs = R.quantize_rows_fp8(_reference_copy(x))
    assert torch.equal(q8.view(torch.uint8), f8.view(torch.uint8)) and torch.equal(s8, fs)


# ------------------------------------------------------------------ PHAA bf16 layouts
def _loop_pack(x):
    """layout_kernel.asc:36-43: for each (chunk c, owner d), rows of 256 values copied from
    s * row_stride + (d * 14 + c * 2) * 128 to ((c * 4 + d) * S + s) * 256."""
    S, sr = x.shape[1], x.stride(1)
    flat = x.as_strided(((S - 1) * sr + 56 * 128,), (1,))   # the rows with the gaps between them
    out = torch.empty(7 * 4 * S * 256, dtype=x.dtype)
    for c in range(7):
        for d in range(4):
            for s in range(S):
                src = s * sr + (d * 14 + c * 2) * 128
                out[((c * 4 + d) * S + s) * 256: ((c * 4 + d) * S + s + 1) * 256] = flat[src: src + 256]
    return out.reshape(7, 4, S, 1, 2, 128)


def _loop_back(x, S):
    """layout_kernel.asc:45-52: rows s < L of head h from h * sh + s * st to s * 256 + h * 128; row L
    (when L < 4S) zero."""
    L = x.shape[2]
    out = torch.full((4 * S * 256,), float("nan"), dtype=x.dtype)
    for h in range(2):
        for s in range(L):
            out[s * 256 + h * 128: s * 256 + h * 128 + 128] = x[0, h, s]
    if L < 4 * S:
        out[L * 256: L * 256 + 256] = 0
    return out.reshape(4, S, 1, 256)


def _loop_merge(x):
    """layout_kernel.asc:53-58: rows of 256 from ((c * 4 + d) * S + s) * 256 to s * 7168 + (d * 14 + c * 2) * 128."""
    S = x.shape[2]
    flat = x.reshape(-1)
    out = torch.empty(S * 7168, dtype=x.dtype)
    for c in range(7):
        for d in range(4):
            for s in range(S):
                src = ((c * 4 + d) * S + s) * 256
                out[s * 7168 + (d * 14 + c * 2) * 128: s * 7168 + (d * 14 + c * 2) * 128 + 256] = flat[src: src + 256]
    return out.reshape(1, S, 7168)


@pytest.mark.parametrize("S", [1, 5])
def test_phaa_layouts_are_the_reference_copies(S):
    g = torch.Generator().manual_seed(S)
    x = torch.randn((1, S, 56, 128), generator=g).to(torch.bfloat16)
    assert torch.equal(R.phaa_pack_qkv(x), _loop_pack(x))
    wide = torch.randn((1, S, 60, 128), generator=g).to(torch.bfloat16)[:, :, :56]   # row stride 7,680
    assert torch.equal(R.phaa_pack_qkv(wide), _loop_pack(wide))
    for L in (4 * S, 4 * S - 1):
        attn = torch.randn((1, 2, L, 128), generator=g).to(torch.bfloat16)
        assert torch.equal(R.phaa_pack_back(attn, S), _loop_back(attn, S))
    back = torch.randn((7, 4, S, 1, 256), generator=g).to(torch.bfloat16)
    assert torch.equal(R.phaa_merge_back(back), _loop_merge(back))
    # the round trip of the layouts a peer applies: merge(pack) of one position's heads is the identity
    assert torch.equal(R.phaa_merge_back(R.phaa_pack_qkv(x).reshape(7, 4, S, 1, 256)), x.reshape(1, S, 7168))
