"""The asynchronous FP8 exchange's host contract on the CPU (xgen_amd.phaa.fp8_async_transport,
mirroring x_base/x_base/phaa/fp8_async_transport.py:84-193): the options' rule, every argument check
of the pack with the reference's message, raised before any collective or kernel, and the refusal of
tensors that are not on the GPU."""
from unittest.mock import patch

import pytest
import torch
import torch.distributed as dist

from xgen_amd import _native as N
from xgen_amd.phaa import fp8_async_transport as T


def test_options_rule():
    """fp8_async_transport.py:91-93: the fused return pack needs the direct return."""
    with pytest.raises(ValueError, match="fused return pack requires direct return"):
        T.AsyncFP8Options(fused_return_pack=True)
    opts = T.AsyncFP8Options(direct_return=True, row_tiling=True, fused_return_pack=True, direct_gather=True)
    assert opts.fused_return_pack and opts.direct_gather
    with pytest.raises(Exception):
        opts.row_tiling = False  # frozen


def shards(shape=(2, 5, 1, 3, 64)):
    return tuple(torch.zeros(shape, dtype=torch.bfloat16) for _ in range(3))


CASES = [
    ("stream count", lambda: T.submit_fp8_exchange(None, shards()[:2], 64, None), "one tensor or a QKV triple"),
    ("qkv without outputs", lambda: T.submit_fp8_exchange(None, shards(), 64, None), "one tensor or a QKV triple"),
    ("output count", lambda: T.submit_fp8_exchange(shards()[:1], shards(), 64, None), "one output per input"),
    ("head dim", lambda: T.submit_fp8_exchange(shards((2, 5, 1, 3, 66)), shards((2, 5, 1, 3, 66)), 66, None),
     "head dim divisible by four"),
    ("mismatched inputs", lambda: T.submit_fp8_exchange(shards(), shards()[:2] + (torch.zeros(2, 5, 1, 3, 32),), 64,
                                                        None), "matching shapes"),
    ("gather of one stream", lambda: T.submit_fp8_exchange((torch.zeros(1, 3, 9, 64),), shards()[:1], 64, None,
                                                           direct_gather=True), "QKV head shards"),
    ("gather of 4-D shards", lambda: T.submit_fp8_exchange(shards((1, 3, 9, 64)), shards((10, 1, 3, 64)), 64, None,
                                                           direct_gather=True), "QKV head shards"),
    ("gather sequence too long", lambda: T.submit_fp8_exchange(shards((1, 3, 11, 64)), shards(), 64, None,
                                                               direct_gather=True), "attention output shapes"),
    ("gather output heads", lambda: T.submit_fp8_exchange(shards((1, 2, 9, 64)), shards(), 64, None,
                                                          direct_gather=True), "attention output shapes"),
    ("outputs of another shape", lambda: T.submit_fp8_exchange(shards((2, 5, 3, 1, 64)), shards(), 64, None),
     "matching input and output"),
    ("outputs not contiguous", lambda: T.submit_fp8_exchange(
        tuple(torch.zeros(2, 5, 1, 64, 3).transpose(3, 4) for _ in range(3)), shards(), 64, None), "contiguous outputs"),
    ("return pack with outputs", lambda: T.submit_fp8_exchange((torch.zeros(1, 3, 9, 64),), (torch.zeros(1, 3, 9, 64),),
                                                               64, None, return_shard_seq=5), "direct return"),
    ("return pack of a 5-D tensor", lambda: T.submit_fp8_exchange(None, shards()[:1], 64, None, return_shard_seq=5),
     "direct return"),
    ("return pack too long", lambda: T.submit_fp8_exchange(None, (torch.zeros(1, 3, 11, 64),), 64, None,
                                                           return_shard_seq=5), "invalid sequence length"),
    ("return pack empty", lambda: T.submit_fp8_exchange(None, (torch.zeros(1, 3, 0, 64),), 64, None,
                                                        return_shard_seq=5), "invalid sequence length"),
    ("rows over peers", lambda: T.submit_fp8_exchange(None, (torch.zeros(3, 64),), 64, None), "divide evenly"),
    ("cpu tensors", lambda: T.submit_fp8_exchange(shards(), shards(), 64, None), "requires CUDA tensors"),
    ("cpu return pack", lambda: T.submit_fp8_exchange(None, (torch.zeros(1, 3, 9, 64),), 64, None, return_shard_seq=5),
     "requires CUDA tensors"),
]


@pytest.mark.parametrize("name,call,message", CASES, ids=[c[0] for c in CASES])
def test_pack_checks_before_any_collective_or_kernel(name, call, message):
    def no_kernels():
        raise AssertionError("a kernel was reached")

    with patch.object(dist, "get_world_size", return_value=2), \
            patch.object(dist, "all_to_all_single") as exchange, patch.object(N, "lib", side_effect=no_kernels):
        with pytest.raises(ValueError, match=message):
            call()
    exchange.assert_not_called()


def test_unpack_checks_outputs():
    rows = T._WireRows(rows=2 * 5 * 3, streams=1, head_dim=64, peers=2, gather=None)
    recv = torch.zeros((30, 68), dtype=torch.uint8)
    with patch.object(N, "lib", side_effect=AssertionError("a kernel was reached")):
        with pytest.raises(ValueError, match="one output per input"):
            T._unpack_exchange(recv, (None,), rows, (5, 1, 2, 3, 3, 0))
        with pytest.raises(ValueError, match="requires CUDA tensors"):
            T._unpack_exchange(recv, (torch.zeros(30, 64),), rows)
