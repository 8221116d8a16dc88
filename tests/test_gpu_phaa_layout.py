"""GPU parity of the head-parallel exchange's BF16 layouts (torch.ops.h3_phaa_layout.{pack, back,
merge}, layout_kernel.asc:33-59): every byte equal to the oracle's layouts (pinned on the CPU against
loops restating the reference kernels' copies) for Q/K/V read in place from the fused QKV projection's
output (row stride 21,504), row strides that differ between Q, K and V, strided attention outputs with
and without the padding token, batched general geometries through the C ABI, and the round trip of a
peer's layouts."""
import pytest
import torch

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd import _native as N
from xgen_amd.operator import phaa_layout, runtime

pytestmark = pytest.mark.gpu


def bf16(shape, seed, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16).to(device)


def sends(S, cuda):
    return [torch.full((7, 4, S, 1, 2, 128), float("nan"), dtype=torch.bfloat16, device=cuda) for _ in range(3)]


@pytest.mark.parametrize("S", [1, 17, 300])
def test_pack_qkv_from_the_fused_projection(cuda, S):
    qkv = bf16((1, S, 3 * 7168), seed=S, device=cuda)           # one fused QKV projection output
    q, k, v = (qkv[..., i * 7168:(i + 1) * 7168].view(1, S, 56, 128) for i in range(3))
    assert S == 1 or q.stride(1) == 21504          # (a size-1 dimension has a free stride)
    out = sends(S, cuda)
    phaa_layout.pack_qkv(q, k, v, *out)
    for x, y in zip((q, k, v), out):
        assert torch.equal(y.cpu().view(torch.int16), R.phaa_pack_qkv(x.cpu()).view(torch.int16))


def test_pack_qkv_with_different_row_strides(cuda):
    S = 33
    q = bf16((1, S, 56, 128), seed=1, device=cuda)
    k = bf16((1, S, 64, 128), seed=2, device=cuda)[:, :, :56]     # row stride 8,192
    v = bf16((1, S, 72, 128), seed=3, device=cuda)[:, :, 8:64]    # row stride 9,216, offset 8 heads
    out = sends(S, cuda)
    torch.ops.h3_phaa_layout.pack(q, k, v, *out)
    for x, y in zip((q, k, v), out):
        assert torch.equal(y.cpu().view(torch.int16), R.phaa_pack_qkv(x.cpu()).view(torch.int16))


@pytest.mark.parametrize("S", [1, 17, 300])
@pytest.mark.parametrize("pad", [0, 1])
def test_pack_back(cuda, S, pad):
    L = 4 * S - pad
    # the attention's output as [1, L, 2, 128] transposed to [1, 2, L, 128]: head stride 128, position 256
    attn = bf16((1, L, 2, 128), seed=L, device=cuda).transpose(1, 2)
    back = torch.full((4, S, 1, 256), float("nan"), dtype=torch.bfloat16, device=cuda)
    phaa_layout.pack_back(attn, back, L=L, S=S)
    assert torch.equal(back.cpu().view(torch.int16), R.phaa_pack_back(attn.cpu(), S).view(torch.int16))
    contiguous = attn.contiguous()
    back2 = torch.full_like(back, float("nan"))
    phaa_layout.pack_back(contiguous, back2, L=L, S=S)
    assert torch.equal(back2.view(torch.int16), back.view(torch.int16))


@pytest.mark.parametrize("S", [1, 17, 300])
def test_merge_back(cuda, S):
    x = bf16((7, 4, S, 1, 256), seed=S + 1, device=cuda)
    merged = torch.full((1, S, 7168), float("nan"), dtype=torch.bfloat16, device=cuda)
    phaa_layout.merge_back(x, merged)
    assert torch.equal(merged.cpu().view(torch.int16), R.phaa_merge_back(x.cpu()).view(torch.int16))


@pytest.mark.parametrize("shape", [(3, 2, 5, 2, 64), (1, 1, 7, 3, 8), (5, 3, 4, 2, 96)])
def test_merge_back_general_geometry_through_the_c_abi(cuda, shape):
    x = bf16(shape, seed=sum(shape), device=cuda)
    chunks, owners, seq, batch, chunk = shape
    merged = torch.empty((batch, seq, owners * chunks * chunk), dtype=torch.bfloat16, device=cuda)
    N.check(N.lib().xgen_phaa_merge_back(x.data_ptr(), chunks, owners, seq, batch, chunk, merged.data_ptr(),
                                         N.stream_of(x)), "xgen_phaa_merge_back")
    assert torch.equal(merged.cpu().view(torch.int16), R.phaa_merge_back(x.cpu()).view(torch.int16))


def test_a_peers_layouts_round_trip(cuda):
    """pack then merge of the same rows (no exchange on one GPU) gives the projection rows back; and
    pack_back of a [1, 2, 4S, 128] output read through unpack_qkv's view of it is the identity."""
    S = 40
    q = bf16((1, S, 56, 128), seed=9, device=cuda)
    out = sends(S, cuda)
    phaa_layout.pack_qkv(q, q, q, *out)
    merged = torch.empty((1, S, 7168), dtype=torch.bfloat16, device=cuda)
    phaa_layout.merge_back(out[0].view(7, 4, S, 1, 256), merged)
    assert torch.equal(merged, q.reshape(1, S, 7168))
    recv = bf16((4, S, 1, 2, 128), seed=10, device=cuda)
    view, _, _ = phaa_layout.unpack_qkv(recv, recv, recv, L=4 * S)
    back = torch.empty((4, S, 1, 256), dtype=torch.bfloat16, device=cuda)
    phaa_layout.pack_back(view, back, L=4 * S, S=S)
    assert torch.equal(back.view(-1), recv.view(-1))


def test_kernels_resolve_phaa_layout(cuda):
    d = runtime.Diagnostics()
    module = runtime.Kernels(d).get("phaa_layout", torch.zeros(1, dtype=torch.bfloat16, device=cuda))
    assert module is phaa_layout and not d.fallbacks


def test_outputs_off_the_16_byte_grid(cuda):
    """Contiguous outputs that start 2 bytes into their storage (views of a larger buffer): the
    kernels write aligned scratch that is copied into them; inputs off the grid are read from
    aligned copies."""
    S = 9
    x = bf16((1, S, 56, 128), seed=11, device=cuda)
    store = torch.full((3, 7 * 4 * S * 256 + 1), float("nan"), dtype=torch.bfloat16, device=cuda)
    outs = [store[i, 1:].view(7, 4, S, 1, 2, 128) for i in range(3)]
    src = torch.empty(x.numel() + 1, dtype=torch.bfloat16, device=cuda)[1:].view_as(x).copy_(x)
    phaa_layout.pack_qkv(src, x, x, *outs)
    for y in outs:
        assert torch.equal(y.cpu().view(torch.int16), R.phaa_pack_qkv(x.cpu()).view(torch.int16))
    merged = torch.empty(S * 7168 + 1, dtype=torch.bfloat16, device=cuda)[1:].view(1, S, 7168)
    phaa_layout.merge_back(outs[0].view(7, 4, S, 1, 256), merged)
    assert torch.equal(merged, x.reshape(1, S, 7168))
    back = torch.empty(4 * S * 256 + 1, dtype=torch.bfloat16, device=cuda)[1:].view(4, S, 1, 256)
    attn = bf16((1, 2, 4 * S - 1, 128), seed=12, device=cuda)
    phaa_layout.pack_back(attn, back, L=4 * S - 1, S=S)
    assert torch.equal(back.cpu().view(torch.int16), R.phaa_pack_back(attn.cpu(), S).view(torch.int16))
