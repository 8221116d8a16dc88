"""The allocation-free per-tensor FP8 scale, xgen_fp8_tensor_scale_noalloc, against
the entry point it varies, xgen_fp8_tensor_scale (caller workspace), through the C
ABI: bit-identical scales on two calls in a row, the second with a smaller input
whose peak is below the first's (stale partial maxima in the shared scratch
would show), with a ragged tail; argument errors rejected before any launch."""
import pytest
import torch

import oracle.ref as R
from xgen_amd import _native as N

pytestmark = pytest.mark.gpu


def scale_with_workspace(L, code, x, stream):
    out = torch.empty(1, dtype=torch.float32, device=x.device)
    ws_bytes = L.xgen_abs_peak_workspace_bytes(x.numel())
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    N.check(L.xgen_fp8_tensor_scale(code, x.data_ptr(), x.numel(), out.data_ptr(), ws.data_ptr(), ws_bytes, stream),
            "xgen_fp8_tensor_scale")
    return out


def test_noalloc_tensor_scale_matches_workspace_form(cuda):
    L = N.lib()
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device=cuda).manual_seed(0)
    big = (torch.randn(15624 * 3072, generator=g, device=cuda) * 4).to(torch.bfloat16)   # C2 activations
    small = (torch.randn(77 * 1001 + 5, generator=g, device=cuda) * 0.5).to(torch.float16)  # ragged tail
    small[-3] = 3.0  # the peak sits in the tail the first workgroup reduces
    for x in (big, small):
        code = N.dtype_code(x.dtype)
        ref = scale_with_workspace(L, code, x, stream)
        got = torch.full((1,), float("nan"), dtype=torch.float32, device=cuda)
        N.check(L.xgen_fp8_tensor_scale_noalloc(code, x.data_ptr(), x.numel(), got.data_ptr(), stream),
                "xgen_fp8_tensor_scale_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32))
        assert torch.equal(got.cpu().reshape(()), R.quantize_per_tensor(x.cpu())[1])
    assert float(got) == float(torch.tensor(3.0) / 448.0)


def test_noalloc_tensor_scale_rejects_bad_arguments(cuda):
    L = N.lib()
    stream = torch.cuda.current_stream().cuda_stream
    x = torch.ones(64, dtype=torch.bfloat16, device=cuda)
    out = torch.empty(1, dtype=torch.float32, device=cuda)
    assert L.xgen_fp8_tensor_scale_noalloc(N.DTYPE_BF16, x.data_ptr(), 0, out.data_ptr(), stream) == \
        N.ERR_INVALID_ARGUMENT
    assert L.xgen_fp8_tensor_scale_noalloc(N.DTYPE_F32, x.data_ptr(), 64, out.data_ptr(), stream) == \
        N.ERR_INVALID_ARGUMENT
    assert L.xgen_fp8_tensor_scale_noalloc(N.DTYPE_BF16, None, 64, out.data_ptr(), stream) == N.ERR_INVALID_ARGUMENT
    assert L.xgen_fp8_tensor_scale_noalloc(N.DTYPE_BF16, x.data_ptr() + 2, 62, out.data_ptr(), stream) == \
        N.ERR_UNSUPPORTED
    assert b"16-byte" in L.xgen_last_error()
