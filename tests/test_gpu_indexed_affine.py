"""GPU parity of the indexed affine (x_base/x_base/operator/h3_indexed_affine.py:32-49): the
modulation kernel bit-exact against the oracle's eager-bf16 expression and its explicit-rounding
numpy form, with the reference test's chunk-view tables (x_base/tests/test_h3_indexed_affine.py:
13-23), strided rows, prepared tables and a bad index; the output AdaLN dispatch bitwise equal to
the eager expression at the reference's shapes (x_base/tests/test_h3_output_adaln.py:32-47); the
block forward with both affines on the kernels equal to the eager block."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch
from torch import nn

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd.operator import nq2
from xgen_amd.operator.h3_indexed_affine import _apply, block_forward, output_adaln

pytestmark = pytest.mark.gpu
xops = torch.ops.xgen_amd


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16)


def inputs(B, S, H, T, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((B, S, H), generator=g, dtype=torch.bfloat16)
    residual = torch.randn((B, S, H), generator=g, dtype=torch.bfloat16)
    tables = torch.randn((T, 6 * H), generator=g, dtype=torch.bfloat16)
    idx = torch.randint(T, (S,), generator=g)
    return x, residual, tables, idx


@pytest.mark.parametrize("B,S,H", [(2, 37, 128), (1, 300, 3072), (3, 5, 5376), (1, 1, 8)])
def test_modulation_bit_exact(cuda, B, S, H):
    x, residual, tables, idx = inputs(B, S, H, 7, seed=S * 7 + H)
    shift, scale, gate = tables.chunk(6, dim=-1)[:3]          # row-strided views
    out = _apply(x.to(cuda), scale.to(cuda), shift.to(cuda), idx.to(cuda), modulation=True)
    ref = R.modulate(x, scale.index_select(0, idx), shift.index_select(0, idx))
    assert out.shape == (B, S, H) and out.dtype == torch.bfloat16
    assert torch.equal(u16(out), u16(ref))
    # the explicit round-after-each-op form of the Triton kernel (h3_indexed_affine.py:20-29)
    f32 = lambda t: t.float().numpy()
    ref_np = R.modulate_np(f32(x), f32(scale.index_select(0, idx)), f32(shift.index_select(0, idx)))
    assert np.array_equal(out.float().cpu().numpy(), ref_np)
    gated = _apply(x.to(cuda), gate.to(cuda), residual.to(cuda), idx.to(cuda), modulation=False)
    assert torch.equal(u16(gated), u16(R.gate_residual(residual, x, gate, idx)))


def test_modulation_special_values(cuda):
    # scale -1 (factor 0), huge scales (overflow to inf), NaN shift, subnormal products
    H = 64
    x = torch.tensor([1.0, -2.0, 3e38, 1e-38, 0.0, -0.0, float("inf"), 5.0] * (H // 8),
                     dtype=torch.bfloat16).reshape(1, 1, H).repeat(1, 4, 1)
    scale = torch.tensor([[-1.0, 2.0, 1e38, -0.5, 0.25, 7.0, -1.0, 3e38] * (H // 8)] * 2, dtype=torch.bfloat16)
    shift = torch.tensor([[0.5, float("nan"), -1.0, 1e-39, -0.0, 2.0, 0.0, -3e38] * (H // 8)] * 2,
                         dtype=torch.bfloat16)
    idx = torch.tensor([0, 1, 1, 0])
    out = _apply(x.to(cuda), scale.to(cuda), shift.to(cuda), idx.to(cuda), modulation=True)
    ref = R.modulate(x, scale.index_select(0, idx), shift.index_select(0, idx))
    # NaN results compare as NaN (the host's vectorised bf16 conversion and the device's give
    # different NaN payloads); every other value bit for bit
    nan = torch.isnan(ref.float())
    assert nan.any() and torch.isinf(ref.float()).any()
    assert torch.equal(torch.isnan(out.float().cpu()), nan)
    assert torch.equal(u16(out)[~nan], u16(ref)[~nan])


def test_strided_rows_and_bad_index(cuda):
    x, _, tables, idx = inputs(2, 24, 256, 4, seed=1)
    big = torch.cat([x, x], dim=-1).to(cuda)                  # row stride 512
    x_view = big[..., 256:]
    shift, scale = tables.chunk(6, dim=-1)[:2]
    idx = idx.clone()
    idx[5] = 4                                                 # one past the table
    out = xops.indexed_modulate(x_view, scale.to(cuda), shift.to(cuda), idx.to(cuda))
    ok = torch.arange(24) != 5
    ref = R.modulate(x[:, ok], scale.index_select(0, idx[ok]), shift.index_select(0, idx[ok]))
    assert torch.equal(u16(out[:, ok.to(cuda)]), u16(ref))
    assert torch.isnan(out[:, 5].float()).all()
    idx[5] = -1
    out = xops.indexed_modulate(x_view, scale.to(cuda), shift.to(cuda), idx.to(cuda))
    assert torch.isnan(out[:, 5].float()).all() and torch.equal(u16(out[:, ok.to(cuda)]), u16(ref))


def test_prepared_and_registered_tables(cuda):
    x, _, tables, idx = inputs(2, 50, 512, 5, seed=2)
    shift, scale = (t.to(cuda) for t in tables.chunk(6, dim=-1)[:2])
    plain = xops.indexed_modulate(x.to(cuda), scale, shift, idx.to(cuda))
    prepared = nq2.adaln_one_plus(scale)
    assert torch.equal(u16(xops.indexed_modulate(x.to(cuda), prepared, shift, idx.to(cuda), True)), u16(plain))
    nq2.register_one_plus(scale, prepared)
    try:
        out = _apply(x.to(cuda), scale, shift, idx.to(cuda), modulation=True)
        assert torch.equal(u16(out), u16(plain))
        scale.mul_(0.5)                                        # written after it was prepared
        again = _apply(x.to(cuda), scale, shift, idx.to(cuda), modulation=True)
        ref = R.modulate(x, scale.cpu().index_select(0, idx), shift.cpu().index_select(0, idx))
        assert torch.equal(u16(again), u16(ref))
    finally:
        nq2.unregister_one_plus(scale)


def test_int32_indices_and_empty(cuda):
    x, _, tables, idx = inputs(1, 9, 64, 3, seed=3)
    shift, scale = (t.to(cuda) for t in tables.chunk(6, dim=-1)[:2])
    a = _apply(x.to(cuda), scale, shift, idx.to(torch.int32).to(cuda), modulation=True)
    b = _apply(x.to(cuda), scale, shift, idx.to(cuda), modulation=True)
    assert torch.equal(u16(a), u16(b))
    empty = xops.indexed_modulate(x[:, :0].to(cuda), scale, shift, idx[:0].to(cuda))
    assert empty.shape == (1, 0, 64)


def _output_layer(width, device):
    return SimpleNamespace(norm=nn.LayerNorm(width, elementwise_affine=False).to(device),
                           linear=nn.Linear(16, width * 2, bias=False).to(device=device, dtype=torch.bfloat16))


@pytest.mark.parametrize("cached", [False, True])
@pytest.mark.parametrize("batch,width,seq", [(1, 5376, 2003), (2, 512, 137)])
def test_output_adaln_is_bitwise_eager(cuda, cached, batch, width, seq):
    torch.manual_seed(42)
    layer = _output_layer(width, cuda)
    x = torch.randn(batch, seq, width, device=cuda, dtype=torch.bfloat16)
    temb = torch.randn(3, 16, device=cuda, dtype=torch.bfloat16)
    indices = torch.arange(seq, device=cuda) % 3
    with torch.no_grad():
        if cached:
            modulation = torch.randn(3, width * 2, device=cuda, dtype=torch.bfloat16)
        else:
            modulation = layer.linear(nn.functional.silu(temb))
        shift, scale = modulation.chunk(2, dim=-1)
        normed = layer.norm(x)
        expected = normed * (1.0 + scale.index_select(0, indices)) + shift.index_select(0, indices)
        actual = output_adaln(normed, scale, shift, indices)
    assert torch.equal(actual.view(torch.int16), expected.view(torch.int16))


def test_block_forward_matches_eager_block(cuda):
    torch.manual_seed(7)
    H, S, T = 256, 40, 3
    lin = lambda: nn.Linear(H, H).to(device=cuda, dtype=torch.bfloat16)
    attn_proj, ff_proj, ada = lin(), lin(), nn.Linear(16, 6 * H).to(device=cuda, dtype=torch.bfloat16)
    norm = nn.LayerNorm(H, elementwise_affine=False).to(cuda)

    def eager(hidden, temb, indices, rotary, mask):
        sa, sc, ga, sf, scf, gf = (t.index_select(0, indices) for t in ada(temb).chunk(6, dim=-1))
        h = hidden + ga * attn_proj(norm(hidden) * (1.0 + sc) + sa)
        return h + gf * ff_proj(norm(h) * (1.0 + scf) + sf)

    block = SimpleNamespace(norm1=norm, norm2=norm, adaln_proj=lambda t: ada(t).chunk(6, dim=-1),
                            attn=lambda x, rotary, mask: attn_proj(x), ff=ff_proj,
                            _h3_eager_forward=eager, _h3_fused_indexed_affine=True)
    hidden = torch.randn(2, S, H, device=cuda, dtype=torch.bfloat16)
    temb = torch.randn(T, 16, device=cuda, dtype=torch.bfloat16)
    indices = torch.arange(S, device=cuda) % T
    with torch.no_grad():
        fused = block_forward(block, hidden, temb, indices, None)
        expected = eager(hidden, temb, indices, None, None)
    assert torch.equal(fused.view(torch.int16), expected.view(torch.int16))
    with torch.enable_grad():                                  # autograd: the block's own forward
        assert torch.equal(block_forward(block, hidden, temb, indices, None).detach().view(torch.int16),
                           expected.view(torch.int16))


def test_output_adaln_allocates_only_its_output(cuda):
    """The reference's memory check (x_base/tests/test_h3_output_adaln.py:50-66): at a full H3
    sequence (1, 32,768, 5,376) the fused output AdaLN needs less than half the eager expression's
    extra memory (the eager one expands both tables to the full sequence and keeps intermediates);
    here the only allocation is the output itself."""
    torch.manual_seed(42)
    width, seq = 5376, 32768
    x = torch.randn(1, seq, width, device=cuda, dtype=torch.bfloat16)
    modulation = torch.randn(3, width * 2, device=cuda, dtype=torch.bfloat16)
    shift, scale = modulation.chunk(2, dim=-1)
    indices = torch.arange(seq, device=cuda) % 3
    with torch.no_grad():
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        expected = x * (1.0 + scale.index_select(0, indices)) + shift.index_select(0, indices)
        torch.cuda.synchronize()
        eager_peak = torch.cuda.max_memory_allocated() - base
        reference = expected.cpu()
        del expected
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        actual = output_adaln(x, scale, shift, indices)
        torch.cuda.synchronize()
        fused_peak = torch.cuda.max_memory_allocated() - base
    assert torch.equal(actual.cpu().view(torch.int16), reference.view(torch.int16))
    assert fused_peak < eager_peak / 2, (eager_peak, fused_peak)
    assert fused_peak <= x.numel() * 2 + (1 << 21), fused_peak
