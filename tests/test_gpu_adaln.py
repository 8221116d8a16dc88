"""AdaLN tables loaded into HBM feed the HIP kernels directly: the fused front end reads the
scale / shift rows (strided [3M', H] views of the packed table) at adaln_indices, and the gated
residual reads the gate rows — bit-exact against the oracle on the same tables."""
import pytest
import torch
from safetensors.torch import save_file

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd import _native as N
from xgen_amd.operator import nq2
from xgen_amd.adaln_cache import AdalnScheduleCache, adaln_indices
from xgen_amd.operator.gate_residual import gate_residual
from xgen_amd.operator.nq2 import norm_affine_quant

pytestmark = pytest.mark.gpu


def table_file(path, H, M=2, blocks=2, seed=3):
    g = torch.Generator().manual_seed(seed)
    t = {"step0_timesteps": torch.tensor([0.25, 0.5])[:M], "const_timesteps": torch.tensor([.999, 1.])}
    for j in range(blocks):
        t[f"step0_block{j}"] = (torch.randn(M, 18 * H, generator=g) * 0.1).to(torch.bfloat16)
        t[f"const_block{j}"] = (torch.randn(2, 18 * H, generator=g) * 0.1).to(torch.bfloat16)
    t["step0_final"] = torch.randn(M, 2 * H, generator=g).to(torch.bfloat16)
    t["const_final"] = torch.randn(2, 2 * H, generator=g).to(torch.bfloat16)
    save_file(t, path, metadata=dict(num_steps="2", num_blocks=str(blocks), quantization="none"))
    return t


@pytest.mark.parametrize("H", [256, 3072, 5376])
@pytest.mark.parametrize("out", ["fp8", "int8"])
def test_loaded_tables_feed_front_end_and_gate(cuda, tmp_path, H, out):
    path = tmp_path / "tables.safetensors"
    t = table_file(path, H)
    cache = AdalnScheduleCache(None, str(path), "video", device=cuda)
    cache.maybe_install(torch.cat([t["step0_timesteps"], t["const_timesteps"][:1]]).to(cuda))
    S = 97
    g = torch.Generator().manual_seed(H)
    x = torch.randn(1, S, H, generator=g).to(torch.bfloat16)
    tstep = torch.randint(0, 3, (S,), generator=g)          # 2 step timesteps + the video constant
    tags = torch.randint(-1, 3, (S,), generator=g)          # -1 = padding token
    idx = adaln_indices(tstep, tags)
    blk = cache.lookup_block(1)
    assert blk.scale.stride(0) == 6 * H                      # read in place, no copy
    dt = torch.float8_e4m3fn if out == "fp8" else torch.int8
    q, s = norm_affine_quant(x.to(cuda), None, blk.scale, blk.shift, idx.to(cuda), eps=1e-6, norm="layer",
                             out_dtype=dt)
    rq, rs, _ = R.norm_affine_quant(x, None, blk.scale.cpu(), blk.shift.cpu(), idx, 1e-6, "layer", out)
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8).reshape(q.shape))
    assert torch.equal(s.cpu(), rs)
    residual = torch.randn(1, S, H, generator=g).to(torch.bfloat16)
    y = gate_residual(residual.to(cuda), x.to(cuda), blk.gate, idx.to(cuda))
    ref = R.gate_residual(residual, x, blk.gate.cpu(), idx)
    assert torch.equal(y.cpu().view(torch.int16), ref.view(torch.int16))


def test_prepared_one_plus_tables_match_plain_tables(cuda, tmp_path):
    """The loader's prepared bf16(1 + scale) tables give the plain path's bytes through the front end."""
    H = 3072
    path = tmp_path / "tables.safetensors"
    t = table_file(path, H, blocks=3)
    cache = AdalnScheduleCache(None, str(path), "none", device=cuda)
    cache.maybe_install(t["step0_timesteps"].to(cuda))
    x = torch.randn(1, 64, H, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(cuda)
    idx = adaln_indices(torch.randint(0, 2, (64,)), torch.randint(0, 3, (64,))).to(cuda)
    for j in range(3):
        blk = cache.lookup_block(j)
        f, f_mlp = cache.one_plus_scales(j)
        for scale, shift, prepared in ((blk.scale, blk.shift, f), (blk.scale_mlp, blk.shift_mlp, f_mlp)):
            # the plain table through the operator itself (the wrapper would take the registered one)
            q0, s0, _ = torch.ops.xgen_amd.norm_affine_quant(x, None, scale, shift, idx, 1e-6, N.NORM_LAYER,
                                                             torch.float8_e4m3fn, False)
            q1, s1 = norm_affine_quant(x, None, prepared, shift, idx, eps=1e-6, norm="layer",
                                       out_dtype=torch.float8_e4m3fn, scale_is_one_plus=True)
            assert torch.equal(q0.view(torch.uint8), q1.view(torch.uint8)) and torch.equal(s0, s1)
            assert torch.equal(prepared.cpu().view(torch.int16), (1.0 + scale.cpu()).view(torch.int16))


def test_installed_tables_are_read_prepared(cuda, tmp_path):
    """Once a schedule is installed, the front end given one of its scale tables as the reference's
    callers pass it (the raw view, detached) reads the loader's prepared bf16(1 + scale) table — the
    plain path's bytes and scales; after the raw table is written in place the prepared one is
    rebuilt on its next use (the bytes follow the new values)."""
    H = 3072
    path = tmp_path / "tables.safetensors"
    t = table_file(path, H, blocks=2)
    cache = AdalnScheduleCache(None, str(path), "none", device=cuda)
    cache.maybe_install(t["step0_timesteps"].to(cuda))
    x = torch.randn(1, 80, H, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(cuda)
    idx = adaln_indices(torch.randint(0, 2, (80,)), torch.randint(0, 3, (80,))).to(cuda)
    w = (torch.randn(H, generator=torch.Generator().manual_seed(7)) * 0.3 + 1).to(torch.bfloat16).to(cuda)
    blk = cache.lookup_block(1)

    def plain(scale):
        return torch.ops.xgen_amd.norm_affine_quant(x, w, scale, blk.shift_mlp, idx, 1e-5, N.NORM_RMS, torch.int8,
                                                    False)[:2]

    for step in range(2):
        before = nq2.prepared_hits
        q, s = norm_affine_quant(x, w, blk.scale_mlp.detach(), blk.shift_mlp.detach(), idx, eps=1e-5)
        assert nq2.prepared_hits == before + 1
        q0, s0 = plain(blk.scale_mlp)
        assert torch.equal(q, q0) and torch.equal(s, s0)
        if step == 0:
            blk.scale_mlp.mul_(1.5)  # written in place: the registered prepared table is stale
    other = blk.scale_mlp.clone()  # same values, other memory: not registered
    before = nq2.prepared_hits
    norm_affine_quant(x, w, other, blk.shift_mlp, idx, eps=1e-5)
    assert nq2.prepared_hits == before


def test_captured_call_reads_the_table_it_is_given(cuda, tmp_path):
    """Under HIP graph capture the front end reads the raw table it is given (no prepared-table
    substitution), so replays after an in-place write to the table see the new values."""
    H = 1024
    path = tmp_path / "tables.safetensors"
    t = table_file(path, H, blocks=1)
    cache = AdalnScheduleCache(None, str(path), "none", device=cuda)
    cache.maybe_install(t["step0_timesteps"].to(cuda))
    blk = cache.lookup_block(0)
    x = torch.randn(1, 48, H, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).to(cuda)
    idx = adaln_indices(torch.randint(0, 2, (48,)), torch.randint(0, 3, (48,))).to(cuda)

    def call():
        return norm_affine_quant(x, None, blk.scale, blk.shift, idx, eps=1e-6, norm="layer",
                                 out_dtype=torch.float8_e4m3fn)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    before = nq2.prepared_hits
    with torch.cuda.graph(graph):
        q, s = call()
    assert nq2.prepared_hits == before
    for rep in range(3):
        if rep:
            blk.scale.add_(0.125)
        graph.replay()
        torch.cuda.synchronize()
        q0, s0, _ = torch.ops.xgen_amd.norm_affine_quant(x, None, blk.scale, blk.shift, idx, 1e-6, N.NORM_LAYER,
                                                         torch.float8_e4m3fn, False)
        assert torch.equal(q.view(torch.uint8), q0.view(torch.uint8)) and torch.equal(s, s0)
