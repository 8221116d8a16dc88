"""The path under HIP graph capture (torch.cuda.CUDAGraph on ROCm): the ops launch on the current
stream, allocate their outputs through torch (the graph's pool while capturing) and record no
memset nodes, so a captured step replays the eager results.  Each graph is replayed several
times, with new inputs copied into its static buffers and the program's own eager work and
synchronizations in between, and every replay is compared bit for bit with the eager result on
the same inputs."""
import pytest
import torch

import xgen_amd  # noqa: F401
from xgen_amd import _native as N
from xgen_amd import workloads
from xgen_amd.operator.dit_chain import DiTLinearChain

pytestmark = pytest.mark.gpu
xops = torch.ops.xgen_amd
FP8 = torch.float8_e4m3fn


def capture(fn):
    """Warm fn up on a side stream (first-use set-up stays out of the graph), then capture it."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


def bits(t):
    return t.view(torch.uint8) if t.element_size() == 1 else t.view(torch.int16 if t.element_size() == 2 else torch.int32)


def same(a, b):
    return all(torch.equal(bits(x), bits(y)) for x, y in zip(a, b))


def test_c2_step_replays(cuda):
    """Per-token FP8 quantization + FP8 GEMM with the fused epilogue (the bench's step) at M = 2,000."""
    M, K, Nf = 2000, 3072, 9216
    g = workloads.generator(31, cuda)
    w, b = workloads.weight("qkv", g, cuda)
    qw, sw = xops.quantize_rows(w, FP8)
    x = torch.empty((M, K), dtype=torch.bfloat16, device=cuda)

    def step():
        qa, sa = xops.quantize_rows(x, FP8)
        out, _ = xops.scaled_mm(qa, qw, sa, sw, b, torch.bfloat16, N.ACT_NONE, False)
        return qa, sa, out

    x.copy_(workloads.activations(M, K, g, cuda)[0])
    graph, static = capture(step)
    for rep in range(4):
        x.copy_(workloads.activations(M, K, g, cuda)[0])
        graph.replay()
        torch.cuda.synchronize()
        eager = step()
        assert same(static, eager), rep
        xops.scaled_mm(eager[0], qw, eager[1], sw, None, torch.bfloat16, N.ACT_GELU_TANH, False)  # eager work between
        torch.cuda.synchronize()


@pytest.mark.parametrize("accumulation", [None, "mfma", "exact"])
def test_chain_replays(cuda, accumulation):
    """The C5 chain's kernels (front end, QKV, requant, out-projection, FFN up, GELU requant, FFN
    down) at S = 700, d = 512 in one graph."""
    B, S, d, T = 1, 700, 512, 20
    g = workloads.generator(32, cuda)
    weights = []
    for N_, K_ in ((3 * d, d), (d, d), (4 * d, d), (d, 4 * d)):
        weights += [(torch.randn((N_, K_), generator=g, device=cuda) * 0.02).to(torch.bfloat16),
                    (torch.randn((N_,), generator=g, device=cuda) * 0.01).to(torch.bfloat16)]
    chain = DiTLinearChain(*weights, accumulation=accumulation)
    shift, scale = workloads.adaln_tables(T, d, g, cuda)
    idx = torch.randint(T, (S,), generator=g, device=cuda)
    x = torch.empty((B, S, d), dtype=torch.bfloat16, device=cuda)

    def run():
        return chain(x, scale, shift, idx)

    x.copy_(workloads.activations(B * S, d, g, cuda)[0].reshape(B, S, d))
    graph, static = capture(run)
    for rep in range(3):
        x.copy_(workloads.activations(B * S, d, g, cuda)[0].reshape(B, S, d))
        idx.copy_(torch.randint(T, (S,), generator=g, device=cuda))
        graph.replay()
        torch.cuda.synchronize()
        assert same(static, run()), rep


@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_h3_ffn_ops_replay(cuda, kind):
    """SwiGLU + requant, the down GEMM with the gated residual fused, and the standalone gated
    residual (H3's FFN tail at reduced size) in one graph."""
    M, F, d, T = 600, 1024, 768, 6
    g = workloads.generator(33, cuda)
    dt = FP8 if kind == "fp8" else torch.int8
    wd = (torch.randn((d, F), generator=g, device=cuda) * 0.02).to(torch.bfloat16)
    bd = (torch.randn((d,), generator=g, device=cuda) * 0.01).to(torch.bfloat16)
    qd, sd = xops.quantize_rows(wd, dt)
    gate = (torch.randn((T, d), generator=g, device=cuda) * 0.1).to(torch.bfloat16)
    u = torch.empty((1, M, 2 * F), dtype=torch.bfloat16, device=cuda)
    res = torch.empty((M, d), dtype=torch.bfloat16, device=cuda)
    idx = torch.randint(T, (M,), generator=g, device=cuda)

    def run():
        qh, sh, _ = xops.swiglu_quant(u, False, dt, 1, False)
        qh = qh.reshape(M, F)
        fused = xops.scaled_mm_gate_residual(qh, qd, sh.reshape(-1), sd, bd, res, gate, idx)
        y, _ = xops.scaled_mm(qh, qd, sh.reshape(-1), sd, bd, torch.bfloat16, N.ACT_NONE, False)
        two = xops.gate_residual(res[None], y[None], gate, idx)
        return qh, sh, fused, two

    def refill():
        u.copy_(torch.randn((1, M, 2 * F), generator=g, device=cuda).to(torch.bfloat16))
        res.copy_(torch.randn((M, d), generator=g, device=cuda).to(torch.bfloat16))

    refill()
    graph, static = capture(run)
    for rep in range(3):
        refill()
        graph.replay()
        torch.cuda.synchronize()
        eager = run()
        assert same(static, eager), rep
        assert torch.equal(bits(static[2]), bits(static[3].reshape(M, d)))


def test_exchange_neighbours_replay(cuda):
    """The out-projection's side of the head-parallel exchange and the output AdaLN under capture:
    Q/K/V packed from a fused projection output into send buffers, the returned chunks merged (BF16)
    and merged + quantized (INT8), and the indexed modulation of normalised rows (H3 geometry,
    S = 96)."""
    from xgen_amd.operator import phaa_layout
    from xgen_amd.operator.h3_indexed_affine import output_adaln
    from xgen_amd.operator.merge_quant import merge_quant

    S = 96
    g = torch.Generator(device=cuda).manual_seed(5)
    qkv = torch.empty((1, S, 3 * 7168), dtype=torch.bfloat16, device=cuda)
    back = torch.empty((7, 4, S, 1, 256), dtype=torch.bfloat16, device=cuda)
    normed = torch.empty((1, S, 7168), dtype=torch.bfloat16, device=cuda)
    tables = torch.randn((3, 2 * 7168), generator=g, device=cuda).to(torch.bfloat16)
    shift, scale = tables.chunk(2, dim=-1)
    idx = torch.arange(S, device=cuda) % 3
    sends = [torch.empty((7, 4, S, 1, 2, 128), dtype=torch.bfloat16, device=cuda) for _ in range(3)]
    merged = torch.empty((1, S, 7168), dtype=torch.bfloat16, device=cuda)

    def fill():
        for t in (qkv, back, normed):
            t.copy_(torch.randn(t.shape, generator=g, device=cuda).to(torch.bfloat16))

    def step():
        q, k, v = (qkv[..., i * 7168:(i + 1) * 7168].view(1, S, 56, 128) for i in range(3))
        phaa_layout.pack_qkv(q, k, v, *sends)
        phaa_layout.merge_back(back, merged)
        qm, sm = merge_quant(back)
        return (*sends, merged, qm, sm, output_adaln(normed, scale, shift, idx))

    fill()
    graph, static = capture(step)
    for rep in range(4):
        fill()
        graph.replay()
        torch.cuda.synchronize()
        replayed = [t.clone() for t in static]
        eager = step()
        torch.cuda.synchronize()
        assert same(replayed, eager), f"replay {rep}"
