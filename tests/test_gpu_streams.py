"""GPU: calls on different streams are independent.  The path's operators launched on two streams at
once (interleaved, each stream's work overlapping the other's), and from two host threads with a
stream each, give the bytes of the same calls run one after another on one stream."""
import threading

import pytest
import torch

import xgen_amd  # noqa: F401
from xgen_amd import _native as N

pytestmark = pytest.mark.gpu
xops = torch.ops.xgen_amd
FP8 = torch.float8_e4m3fn


def bits(t):
    return t.view(torch.uint8) if t.element_size() == 1 else t.view(torch.int16 if t.element_size() == 2
                                                                     else torch.int32)


def make_job(seed, cuda):
    """One small block front: front end -> QKV GEMM (both kinds) -> requant -> gated out-projection,
    plus the output AdaLN modulation and a merge + quant of a Q slice."""
    g = torch.Generator().manual_seed(seed)
    B, S, d, T = 1, 1536, 1024, 6
    x = torch.randn((B, S, d), generator=g).to(torch.bfloat16).to(cuda)
    scale = (torch.randn((T, d), generator=g) * 0.1).to(torch.bfloat16).to(cuda)
    shift = (torch.randn((T, d), generator=g) * 0.1).to(torch.bfloat16).to(cuda)
    gate = (torch.randn((T, d), generator=g) * 0.5).to(torch.bfloat16).to(cuda)
    idx = torch.randint(T, (S,), generator=g).to(cuda)
    wq, sq = xops.quantize_rows((torch.randn((3 * d, d), generator=g) * 0.02).to(torch.bfloat16).to(cuda), FP8)
    wo, so = xops.quantize_rows((torch.randn((d, d), generator=g) * 0.02).to(torch.bfloat16).to(cuda), FP8)

    def run():
        q, s = xops.norm_affine_quant(x, None, scale, shift, idx, 1e-6, N.NORM_LAYER, FP8, False)[:2]
        qkv, _ = xops.scaled_mm(q, wq, s, sq, None, torch.bfloat16, N.ACT_NONE, False)
        qkv_exact, _ = xops.scaled_mm(q, wq, s, sq, None, torch.bfloat16, N.ACT_NONE, False, True)
        qv, sv = xops.quantize_rows(qkv[:, 2 * d:], FP8)
        out = xops.scaled_mm_gate_residual(qv, wo, sv, so, None, x.reshape(-1, d), gate, idx)
        mod = xops.indexed_modulate(x, scale, shift, idx)
        mq, ms = xops.merge_quant(qkv[:, :d].reshape(4, 2, S, 1, 128), torch.int8)
        return [q, s, qkv, qkv_exact, qv, sv, out, mod, mq, ms]

    return run


def assert_same(got, ref):
    for a, b in zip(got, ref):
        assert torch.equal(bits(a), bits(b))


def test_two_streams_overlapping(cuda):
    jobs = [make_job(seed, cuda) for seed in (1, 2)]
    ref = [job() for job in jobs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for _ in range(3):
        got = [None, None]
        for _ in range(2):  # interleaved: both streams hold queued work at once
            for i, (job, st) in enumerate(zip(jobs, streams)):
                with torch.cuda.stream(st):
                    got[i] = job()
        torch.cuda.synchronize()
        for g, r in zip(got, ref):
            assert_same(g, r)


def test_two_host_threads(cuda):
    jobs = [make_job(seed, cuda) for seed in (3, 4)]
    ref = [job() for job in jobs]
    torch.cuda.synchronize()
    results, errors = [None, None], []

    def worker(i):
        try:
            torch.cuda.set_device(cuda)
            st = torch.cuda.Stream()
            with torch.cuda.stream(st):
                for _ in range(3):
                    out = jobs[i]()
                st.synchronize()
            results[i] = out
        except Exception as error:  # surfaced below, in the test's thread
            errors.append(error)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    for g, r in zip(results, ref):
        assert g is not None
        assert_same(g, r)

