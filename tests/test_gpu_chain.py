"""GPU parity of the C5 chain (fused front end -> QKV -> out-proj -> FFN up ->
GELU-tanh + per-token requant -> FFN down) through DiTLinearChain.

Each stage is checked against the oracle applied to the kernel's own input of
that stage: quantized bytes and scales bit-exact, bf16 outputs within rel-L2
<= 1e-3 and cosine >= 0.9999.

End to end, every per-token requantization can turn a last-bit difference of
its bf16 input into a different e4m3 rounding (2^-4 relative), so differences
in the GEMMs' sums grow along the chain.  Three accumulation settings:

* the default (DEFAULT_ACCUMULATION: QKV exact, the other projections on the
  FP8 MFMA) and "exact" everywhere: all four outputs within the north_star bar
  (rel-L2 <= 1e-2, cosine >= 0.9999) of the exactly summed oracle composite,
  the reference's arithmetic (use_fast_accum=False).
* "mfma" everywhere: outside the bar at the FFN output (C5 ~2.2e-2, cosine
  ~0.9998); the distance is printed, and the outputs are held to the oracle
  composite run with the MFMA sum model (oracle/mfma_model.c) as a regression
  check of the kernels, not as parity.

Every setting is also held to that per-stage modelled composite (exact sums
where the stage is exact), from the kernel's own front-end bytes, within
MODEL_REL_MAX.
"""
import pytest
import torch

import oracle.ref as R
import xgen_amd  # noqa: F401
from xgen_amd import _native as N
from xgen_amd import workloads
from xgen_amd.operator.dit_chain import DEFAULT_ACCUMULATION, DiTLinearChain, stage_accumulation

pytestmark = pytest.mark.gpu
xops = torch.ops.xgen_amd
FP8 = torch.float8_e4m3fn
BAR_REL, BAR_COS = 1e-2, 0.9999       # north_star: bf16 outputs vs the reference path
MODEL_REL_MAX, MODEL_COS_MIN = 5e-3, 0.99999
NAMES = ("qkv", "out", "ffn_up", "ffn_down")


def chain_inputs(B, S, d, T, seed, dev, accumulation, gelu="requant"):
    g = workloads.generator(seed)
    x, _ = workloads.activations(B * S, d, g)
    shift, scale = workloads.adaln_tables(T, d, g)
    idx = torch.randint(T, (S,), generator=g)
    weights = {}
    for name, (N, K) in zip(NAMES, ((3 * d, d), (d, d), (4 * d, d), (d, 4 * d))):
        w = (torch.randn((N, K), generator=g) * 0.02).to(torch.bfloat16)
        b = (torch.randn((N,), generator=g) * 0.01).to(torch.bfloat16)
        weights[name] = (w, b)
    chain = DiTLinearChain(*[t.to(dev) for name in NAMES for t in weights[name]],
                           accumulation=None if accumulation == "default" else accumulation, gelu=gelu)
    return x.reshape(B, S, d), scale, shift, idx, weights, chain


def check_stage(lin, inp, out, rows=None, act=None, gelu=None):
    """out = lin(inp) per the oracle, given the kernel's own bf16 input (rows: optional sample);
    gelu: the GPU's GELU (the kernel_gelu fixture) where lin quantizes gelu_tanh of its input."""
    if rows is not None:
        inp, out = inp[rows], out[rows]
    qa, sa = xops.quantize_rows(inp.contiguous(), FP8, N.ACT_GELU_TANH if gelu else N.ACT_NONE)
    q2, s2 = R.quantize_rows_fp8(gelu(inp) if gelu else inp.cpu())
    assert torch.equal(qa.cpu().view(torch.uint8), q2.view(torch.uint8))
    assert torch.equal(sa.cpu().view(torch.int32), s2.view(torch.int32))
    acc = R.fp8_mfma_accumulate if lin.accumulation == "mfma" else None
    ref = R.w8a8_linear_fp8(q2, s2, lin.weight.cpu(), lin.weight_scale.cpu().reshape(-1), lin.bias.cpu(),
                            torch.bfloat16, act, acc)
    rel, cos = R.rel_l2(out, ref), R.cosine(out, ref)
    assert rel <= 1e-3 and cos >= 0.9999, (rel, cos)


def kinds_of(accumulation):
    return stage_accumulation(DEFAULT_ACCUMULATION if accumulation == "default" else accumulation)


def check_end_to_end(got, x, scale, shift, idx, weights, accumulation, front):
    """got: the chain's four outputs (rows as in x).  Returns {name: (rel, cos)} against the exact
    composite; asserts the bar unless every projection uses the FP8 MFMA sum, and agreement with
    the composite whose stages sum as the kernels' do."""
    kinds = kinds_of(accumulation)
    exact = R.dit_chain_fp8(x, scale, shift, idx, weights)
    dist = {n: (R.rel_l2(a, r), R.cosine(a, r)) for n, a, r in zip(NAMES, got, exact)}
    if set(kinds.values()) != {"mfma"}:
        for n, (rel, cos) in dist.items():
            assert rel <= BAR_REL and cos >= BAR_COS, (n, rel, cos)
    model = R.dit_chain_fp8(x, scale, shift, idx, weights, front=front,
                            accumulate={n: R.fp8_mfma_accumulate if k == "mfma" else None for n, k in kinds.items()})
    for n, a, r in zip(NAMES, got, model):
        rel, cos = R.rel_l2(a, r), R.cosine(a, r)
        assert rel <= MODEL_REL_MAX and cos >= MODEL_COS_MIN, (n, rel, cos)
    # the first projection sees the front end's bytes directly: the per-linear bar holds
    assert dist["qkv"][0] <= BAR_REL and dist["qkv"][1] >= BAR_COS
    return dist


@pytest.mark.parametrize("accumulation", ["default", "exact", "mfma"])
@pytest.mark.parametrize("B,S,d", [(2, 150, 256), (1, 333, 512)])
def test_chain_matches_oracle(cuda, kernel_gelu, B, S, d, accumulation):
    x, scale, shift, idx, weights, chain = chain_inputs(B, S, d, 20, seed=S + d, dev=cuda, accumulation=accumulation)
    qkv, o, h, y = chain(x.to(cuda), scale.to(cuda), shift.to(cuda), idx.to(cuda))
    M = B * S
    qkv, o, h, y = (t.reshape(M, -1) for t in (qkv, o, h, y))
    # stage by stage on the kernel's own inputs
    fq, fs = xops.norm_affine_quant(x.to(cuda), None, scale.to(cuda), shift.to(cuda), idx.to(cuda), 1e-6, 0, FP8,
                                    False)[:2]
    q, s, _ = R.norm_affine_quant(x, None, scale, shift, idx, 1e-6, "layer", "fp8")
    acc = R.fp8_mfma_accumulate if chain.qkv.accumulation == "mfma" else None
    ref_qkv = R.w8a8_linear_fp8(q, s, chain.qkv.weight.cpu(), chain.qkv.weight_scale.cpu().reshape(-1),
                                chain.qkv.bias.cpu(), accumulate=acc)
    assert R.rel_l2(qkv, ref_qkv) <= 1e-3 and R.cosine(qkv, ref_qkv) >= 0.9999
    check_stage(chain.out, qkv[:, 2 * d:], o)
    check_stage(chain.ff_up, o, h)
    check_stage(chain.ff_down, h, y, gelu=kernel_gelu)
    # the oracle composite's hidden is after the GELU
    check_end_to_end((qkv, o, kernel_gelu(h), y), x, scale, shift, idx, weights, accumulation,
                     (fq.cpu(), fs.cpu()))


def test_gelu_placements_agree(cuda, kernel_gelu):
    """gelu='requant' (GELU in ff_down's quantizer, the default) and gelu='epilogue' (GELU in
    ff_up's GEMM epilogue) give the same QKV, out-projection and FFN output bit for bit; the
    epilogue form's hidden is the GPU's GELU of the requant form's."""
    outs = {}
    for gelu in ("requant", "epilogue"):
        x, scale, shift, idx, _, chain = chain_inputs(1, 333, 512, 20, seed=7, dev=cuda, accumulation="mfma",
                                                      gelu=gelu)
        outs[gelu] = chain(x.to(cuda), scale.to(cuda), shift.to(cuda), idx.to(cuda))
    (qkv1, o1, h1, y1), (qkv2, o2, h2, y2) = outs["requant"], outs["epilogue"]
    for a, b in ((qkv1, qkv2), (o1, o2), (y1, y2)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(kernel_gelu(h1).view(torch.int16), h2.cpu().view(torch.int16))
    assert not torch.equal(h1.view(torch.int16), h2.view(torch.int16))


def run_c5(cuda, kernel_gelu, accumulation, seed):
    M, d = workloads.M_10S, workloads.D_MODEL
    g = workloads.generator(seed, cuda)
    x, _ = workloads.activations(M, d, g, cuda)
    shift, scale = workloads.adaln_tables(20, d, g, cuda)
    idx = torch.randint(20, (M,), generator=g, device=cuda)
    wb = {name: workloads.weight(name, g, cuda) for name in NAMES}
    chain = DiTLinearChain(*[t for name in NAMES for t in wb[name]],
                           accumulation=None if accumulation == "default" else accumulation)
    qkv, o, h, y = (t.reshape(M, -1) for t in chain(x[None], scale, shift, idx))
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(5))[:48]
    rows[0], rows[1] = 0, M - 1
    rc = rows.to(cuda)
    fq, fs = xops.norm_affine_quant(x[rc][None], None, scale, shift, idx[rc], 1e-6, 0, FP8, False)[:2]
    check_stage(chain.out, qkv[:, 2 * d:], o, rc)
    check_stage(chain.ff_up, o, h, rc)
    check_stage(chain.ff_down, h, y, rc, gelu=kernel_gelu)
    weights = {k: (w.cpu(), b.cpu()) for k, (w, b) in wb.items()}
    got = [t[rc].cpu() for t in (qkv, o, h, y)]
    got[2] = kernel_gelu(got[2])
    dist = check_end_to_end(got, x[rc][None].cpu(), scale.cpu(), shift.cpu(),
                            idx[rc].cpu(), weights, accumulation, (fq.cpu(), fs.cpu()))
    print(f"C5 end to end ({accumulation}, seed {seed}):",
          {n: f"rel {r:.2e} cos {c:.7f}" for n, (r, c) in dist.items()})


@pytest.mark.parametrize("accumulation", ["default", "exact", "mfma"])
def test_chain_full_size_c5_sampled_rows(cuda, kernel_gelu, accumulation):
    """C5 at M = 31,248 tokens (10 s clip, SP8 share), d = 3,072: the whole chain on the GPU,
    48 seeded rows (first and last included) checked stage by stage and end to end."""
    run_c5(cuda, kernel_gelu, accumulation, seed=0)


@pytest.mark.parametrize("seed", [1, 2])
def test_default_chain_full_size_c5_other_data(cuda, kernel_gelu, seed):
    """The default chain's end-to-end bar at C5 on two more seeded draws of activations, tables,
    indices and weights (the bar is not tuned to one draw)."""
    run_c5(cuda, kernel_gelu, "default", seed)
