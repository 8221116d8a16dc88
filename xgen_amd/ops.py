"""torch.library operators over the xgen_amd C ABI (namespace ``xgen_amd``).

Each operator has a CUDA-key implementation (PyTorch-ROCm exposes HIP devices
under the CUDA key) that allocates its outputs with the caching allocator and
launches on the current stream, and a Meta implementation with the same shape
and dtype contract, so shapes are checkable without a GPU.  This mirrors the
reference's TORCH_LIBRARY + device + Meta registrations
(x_base/x_base/operator/npu_fusion/f2_nq2/op_extension/nq2_queued.asc:53-61).
Contract violations raise RuntimeError before any launch.
"""
from __future__ import annotations

import torch

from . import _native as N

NAMESPACE = "xgen_amd"
_LIB = None

SCHEMAS = {
    "quantize_rows": "quantize_rows(Tensor x, ScalarType out_dtype, int activation=0) -> (Tensor, Tensor)",
    "abs_peak": "abs_peak(Tensor x) -> Tensor",
    "fp8_tensor_scale": "fp8_tensor_scale(Tensor x) -> Tensor",
    "fp8_pack": "fp8_pack(Tensor x, Tensor scale) -> Tensor",
    "norm_affine_quant": (
        "norm_affine_quant(Tensor x, Tensor? weight, Tensor scale, Tensor shift, Tensor indices, "
        "float eps, int norm_kind, ScalarType out_dtype, bool return_normed) -> (Tensor, Tensor, Tensor)"),
    "scaled_mm": (
        "scaled_mm(Tensor a, Tensor w, Tensor a_scale, Tensor w_scale, Tensor? bias, "
        "ScalarType out_dtype, int activation, bool return_acc, bool exact=False) -> (Tensor, Tensor)"),
    "gate_residual": "gate_residual(Tensor residual, Tensor branch, Tensor gate_table, Tensor indices) -> Tensor",
    "indexed_modulate": (
        "indexed_modulate(Tensor x, Tensor scale_table, Tensor shift_table, Tensor indices, "
        "bool scale_is_one_plus=False) -> Tensor"),
    "merge_quant": "merge_quant(Tensor back_recv, ScalarType out_dtype) -> (Tensor, Tensor)",
    "swiglu_quant": (
        "swiglu_quant(Tensor u, bool gate_first, ScalarType out_dtype, int scale_mode, bool return_act) "
        "-> (Tensor, Tensor, Tensor)"),
    "scaled_mm_gate_residual": (
        "scaled_mm_gate_residual(Tensor a, Tensor w, Tensor a_scale, Tensor w_scale, Tensor? bias, "
        "Tensor residual, Tensor gate_table, Tensor indices) -> Tensor"),
}


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _kernel_rows(t: torch.Tensor, row_align: int) -> torch.Tensor:
    """t [..., rows, cols] as the kernels read it: unit column stride, every outer stride a multiple
    of row_align elements, a row stride that covers the row, a 16-byte aligned base; other views
    are copied (the kernels move rows in 16-byte pieces)."""
    if (t.stride(-1) == 1 and t.stride(-2) >= t.shape[-1] and all(st % row_align == 0 for st in t.stride()[:-1])
            and t.data_ptr() % 16 == 0):
        return t
    return t.clone(memory_format=torch.contiguous_format)


def _aligned_flat(t: torch.Tensor) -> torch.Tensor:
    """t contiguous with a 16-byte aligned base (copied if not)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _rows_view(x: torch.Tensor) -> torch.Tensor:
    """[..., K] -> [M, K] with unit last stride (copies only if needed)."""
    m = x.reshape(-1, x.shape[-1])
    if m.stride(-1) != 1 or (m.shape[0] > 1 and m.stride(0) < m.shape[1]):
        m = m.contiguous()
    return m


# --------------------------------------------------------------------------- meta
def _quantize_rows_meta(x, out_dtype, activation=0):
    _require(x.dtype in (torch.bfloat16, torch.float16), "quantize_rows: BF16/F16 input required")
    _require(activation in (N.ACT_NONE, N.ACT_GELU_TANH), "quantize_rows: activation must be none or gelu_tanh")
    _require(out_dtype in (torch.float8_e4m3fn, torch.int8), "quantize_rows: out_dtype must be float8_e4m3fn or int8")
    _require(x.dim() >= 1 and x.shape[-1] > 0, "quantize_rows: input needs a non-empty last dimension")
    rows = x.numel() // x.shape[-1]
    return torch.empty(x.shape, dtype=out_dtype, device=x.device), torch.empty((rows,), dtype=torch.float32, device=x.device)


def _peak_meta(x):
    _require(x.dtype in (torch.bfloat16, torch.float16), "abs_peak: BF16/F16 input required")
    return torch.empty((), dtype=torch.float32, device=x.device)


def _pack_meta(x, scale):
    _require(x.dtype in (torch.bfloat16, torch.float16), "fp8_pack: BF16/F16 input required")
    _require(scale.dtype == torch.float32 and scale.numel() == 1, "fp8_pack: one float32 scale required")
    return torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)


def _norm_check(x, weight, scale, shift, indices, eps, norm_kind, out_dtype):
    _require(x.dim() == 3 and x.dtype == torch.bfloat16 and x.stride(2) == 1 and x.shape[2] > 0,
             "norm_affine_quant: BF16 [B,S,H] with last stride 1 required")
    H = x.shape[2]
    _require(H <= 8192, "norm_affine_quant: H <= 8192 required")
    _require(weight is None or (weight.dim() == 1 and weight.shape[0] == H and weight.is_contiguous()
                                and weight.dtype in (torch.bfloat16, torch.float32)),
             "norm_affine_quant: BF16/F32 norm weight [H] or None required")
    _require(scale.dim() == 2 and scale.shape[0] > 0 and scale.shape[1] == H and shift.shape == scale.shape
             and scale.dtype == torch.bfloat16 and shift.dtype == torch.bfloat16
             and scale.stride(1) == 1 and shift.stride(1) == 1,
             "norm_affine_quant: BF16 tables [T,H] with last stride 1 required")
    _require(indices.dim() == 1 and indices.shape[0] == x.shape[1] and indices.dtype == torch.int64
             and indices.is_contiguous(), "norm_affine_quant: contiguous INT64 indices [S] required")
    _require(0 < eps < 1, "norm_affine_quant: eps must be in (0, 1)")
    _require(norm_kind & ~N.NORM_SCALE_ONE_PLUS in (N.NORM_LAYER, N.NORM_RMS),
             "norm_affine_quant: norm_kind must be 0 (layer) or 1 (rms), optionally | 0x100 (scale is 1 + scale)")
    _require(out_dtype in (torch.float8_e4m3fn, torch.int8), "norm_affine_quant: out_dtype must be float8_e4m3fn or int8")


def _norm_meta(x, weight, scale, shift, indices, eps, norm_kind, out_dtype, return_normed):
    _norm_check(x, weight, scale, shift, indices, eps, norm_kind, out_dtype)
    rows = x.shape[0] * x.shape[1]
    H = x.shape[2]
    normed = x.new_empty((rows, H) if return_normed else (0,))
    return (torch.empty((rows, H), dtype=out_dtype, device=x.device),
            torch.empty((rows,), dtype=torch.float32, device=x.device), normed)


def _mm_check(a, w, a_scale, w_scale, bias, out_dtype, activation):
    _require(a.dtype in (torch.float8_e4m3fn, torch.int8) and w.dtype == a.dtype,
             "scaled_mm: operands must both be float8_e4m3fn or both int8")
    _require(a.dim() == 2 and w.dim() == 2 and a.shape[1] == w.shape[1],
             "scaled_mm: a [M,K] and w [N,K] required")
    M, K = a.shape
    Nf = w.shape[0]
    _require(a_scale.dtype == torch.float32 and a_scale.numel() in (1, M),
             "scaled_mm: float32 activation scale with 1 or M elements required")
    _require(w_scale.dtype == torch.float32 and w_scale.numel() in (1, Nf),
             "scaled_mm: float32 weight scale with 1 or N elements required")
    _require(bias is None or (bias.dim() == 1 and bias.shape[0] == Nf
                              and bias.dtype in (torch.bfloat16, torch.float16, torch.float32)),
             "scaled_mm: bias [N] of BF16/F16/F32 required")
    _require(out_dtype in (torch.bfloat16, torch.float16), "scaled_mm: out_dtype must be bfloat16 or float16")
    _require(activation in (N.ACT_NONE, N.ACT_GELU_TANH), "scaled_mm: activation must be 0 (none) or 1 (gelu_tanh)")
    _require(K % 16 == 0 and Nf % 16 == 0, "scaled_mm: K and N must be multiples of 16")


def _mm_meta(a, w, a_scale, w_scale, bias, out_dtype, activation, return_acc, exact=False):
    _mm_check(a, w, a_scale, w_scale, bias, out_dtype, activation)
    _require(not exact or a.dtype == torch.float8_e4m3fn, "scaled_mm: exact accumulation applies to FP8 operands")
    M, Nf = a.shape[0], w.shape[0]
    acc_dtype = torch.float32 if a.dtype == torch.float8_e4m3fn else torch.int32
    acc = torch.empty((M, Nf) if return_acc else (0,), dtype=acc_dtype, device=a.device)
    return torch.empty((M, Nf), dtype=out_dtype, device=a.device), acc


def _gate_check(residual, branch, gate_table, indices, what="gate_residual"):
    _require(residual.dim() == 3 and branch.shape == residual.shape and residual.shape[2] > 0,
             f"{what}: residual/branch [B,S,H] shapes must match")
    _require(gate_table.dim() == 2 and gate_table.shape[0] > 0 and gate_table.shape[1] == residual.shape[2],
             f"{what}: gate_table [T,H] required")
    _require(indices.dim() == 1 and indices.shape[0] == residual.shape[1] and indices.dtype == torch.int64,
             f"{what}: int64 indices [S] required")
    _require(residual.dtype == branch.dtype == gate_table.dtype == torch.bfloat16, f"{what}: BF16 inputs required")


def _gate_meta(residual, branch, gate_table, indices):
    _gate_check(residual, branch, gate_table, indices)
    return torch.empty(residual.shape, dtype=torch.bfloat16, device=residual.device)


def _modulate_meta(x, scale_table, shift_table, indices, scale_is_one_plus=False):
    what = "indexed_modulate"
    _require(x.dim() == 3 and x.shape[2] > 0, f"{what}: x [B,S,H] required")
    _require(scale_table.dim() == 2 and scale_table.shape[0] > 0 and scale_table.shape[1] == x.shape[2]
             and shift_table.shape == scale_table.shape, f"{what}: scale/shift tables [T,H] required")
    _require(indices.dim() == 1 and indices.shape[0] == x.shape[1] and indices.dtype == torch.int64,
             f"{what}: int64 indices [S] required")
    _require(x.dtype == scale_table.dtype == shift_table.dtype == torch.bfloat16, f"{what}: BF16 inputs required")
    return torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)


MERGE_MAX_WIDTH = 16384


def _merge_meta(back_recv, out_dtype):
    what = "merge_quant"
    _require(back_recv.dim() == 5 and back_recv.dtype == torch.bfloat16,
             f"{what}: BF16 back_recv [splits, owners, seq, batch, chunk] required")
    splits, owners, seq, batch, chunk = back_recv.shape
    _require(splits > 0 and owners > 0 and chunk > 0 and chunk % 8 == 0,
             f"{what}: chunk must be a positive multiple of 8")
    _require(splits * owners * chunk <= MERGE_MAX_WIDTH, f"{what}: splits*owners*chunk must be <= {MERGE_MAX_WIDTH}")
    _require(seq * batch < 2 ** 31, f"{what}: seq*batch must be below 2^31")
    _require(out_dtype in (torch.float8_e4m3fn, torch.int8), f"{what}: out_dtype must be float8_e4m3fn or int8")
    q = torch.empty((batch * seq, splits * owners * chunk), dtype=out_dtype, device=back_recv.device)
    return q, torch.empty((batch * seq,), dtype=torch.float32, device=back_recv.device)


SWIGLU_MAX_HALF = 16384


def _swiglu_meta(u, gate_first, out_dtype, scale_mode, return_act):
    _require(u.dim() == 3 and u.shape[2] > 0 and u.shape[2] % 2 == 0 and u.shape[2] <= 2 * SWIGLU_MAX_HALF,
             f"swiglu_quant: [B,S,2F], 1<=F<={SWIGLU_MAX_HALF} required")
    _require(u.dtype == torch.bfloat16, "swiglu_quant: BF16 input required")
    _require(out_dtype in (torch.float8_e4m3fn, torch.int8), "swiglu_quant: out_dtype must be float8_e4m3fn or int8")
    _require(scale_mode in (0, 1), "swiglu_quant: scale_mode must be 0 or 1")
    rows, F = u.shape[0] * u.shape[1], u.shape[2] // 2
    q = torch.empty((rows, F), dtype=out_dtype, device=u.device)
    s = torch.empty((rows,), dtype=torch.float32, device=u.device)
    act = torch.empty((rows, F) if return_act else (0,), dtype=torch.bfloat16, device=u.device)
    return q, s, act


def _mm_gate_check(a, w, a_scale, w_scale, bias, residual, gate_table, indices):
    _mm_check(a, w, a_scale, w_scale, bias, torch.bfloat16, N.ACT_NONE)
    M, Nf = a.shape[0], w.shape[0]
    _require(residual.dim() == 2 and tuple(residual.shape) == (M, Nf) and residual.dtype == torch.bfloat16,
             "scaled_mm_gate_residual: residual BF16 [M, N] required")
    _require(gate_table.dim() == 2 and gate_table.shape[1] == Nf and gate_table.shape[0] > 0
             and gate_table.dtype == torch.bfloat16, "scaled_mm_gate_residual: gate_table BF16 [T, N] required")
    _require(indices.dim() == 1 and indices.dtype == torch.int64 and indices.shape[0] > 0
             and M % indices.shape[0] == 0, "scaled_mm_gate_residual: int64 indices [S] with M % S == 0 required")


def _mm_gate_meta(a, w, a_scale, w_scale, bias, residual, gate_table, indices):
    _mm_gate_check(a, w, a_scale, w_scale, bias, residual, gate_table, indices)
    return torch.empty((a.shape[0], w.shape[0]), dtype=torch.bfloat16, device=a.device)


# --------------------------------------------------------------------------- device
def _on_gpu(*ts):
    dev = ts[0].device
    _require(dev.type == "cuda", "xgen_amd operators require tensors on a HIP (cuda) device")
    for t in ts[1:]:
        if t is not None:
            _require(t.device == dev, "xgen_amd operators require all tensors on the same device")


def _quantize_rows_gpu(x, out_dtype, activation=0):
    """Per-row quantization of x, or (activation = ACT_GELU_TANH) of dtype(gelu_tanh(x)) in the same pass."""
    _on_gpu(x)
    q, scale = _quantize_rows_meta(x, out_dtype, activation)
    if x.numel() == 0:
        return q, scale
    m = _rows_view(x)
    fn = "xgen_quantize_rows_gelu" if activation == N.ACT_GELU_TANH else "xgen_quantize_rows"
    st = getattr(N.lib(), fn)(N.dtype_code(x.dtype), m.data_ptr(), m.shape[0], m.shape[1], m.stride(0),
                              N.dtype_code(out_dtype), q.data_ptr(), m.shape[1], scale.data_ptr(), N.stream_of(x))
    N.check(st, fn)
    return q, scale


def _peak_common(x, fn):
    _on_gpu(x)
    out = _peak_meta(x)
    _require(x.numel() > 0, f"{fn}: empty input")
    xc = _aligned_flat(x)
    L = N.lib()
    ws_bytes = L.xgen_abs_peak_workspace_bytes(xc.numel())
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=x.device)
    st = getattr(L, fn)(N.dtype_code(x.dtype), xc.data_ptr(), xc.numel(), out.data_ptr(), ws.data_ptr(),
                        ws_bytes, N.stream_of(x))
    N.check(st, fn)
    return out


def _peak_gpu(x):
    return _peak_common(x, "xgen_abs_peak")


def _tensor_scale_gpu(x):
    return _peak_common(x, "xgen_fp8_tensor_scale")


def _pack_gpu(x, scale):
    _on_gpu(x, scale)
    q = _pack_meta(x, scale)
    if x.numel() == 0:
        return q
    xc = _aligned_flat(x)
    st = N.lib().xgen_fp8_pack(N.dtype_code(x.dtype), xc.data_ptr(), xc.numel(), scale.data_ptr(), q.data_ptr(),
                               N.stream_of(x))
    N.check(st, "xgen_fp8_pack")
    return q


def _norm_gpu(x, weight, scale, shift, indices, eps, norm_kind, out_dtype, return_normed):
    _on_gpu(x, weight, scale, shift, indices)
    q, s, normed = _norm_meta(x, weight, scale, shift, indices, eps, norm_kind, out_dtype, return_normed)
    if q.numel() == 0:
        return q, s, normed
    x, scale, shift = _kernel_rows(x, 8), _kernel_rows(scale, 8), _kernel_rows(shift, 8)
    weight = None if weight is None else _aligned_flat(weight)
    wcode = N.DTYPE_NONE if weight is None else N.dtype_code(weight.dtype)
    st = N.lib().xgen_norm_affine_quant(
        x.data_ptr(), x.shape[0], x.shape[1], x.shape[2], x.stride(0), x.stride(1), norm_kind,
        N.ptr(weight), wcode, float(eps), scale.data_ptr(), scale.stride(0), shift.data_ptr(), shift.stride(0),
        scale.shape[0], indices.data_ptr(), N.dtype_code(out_dtype), q.data_ptr(), s.data_ptr(),
        normed.data_ptr() if return_normed else None, N.stream_of(x))
    N.check(st, "xgen_norm_affine_quant")
    return q, s, normed


def _mm_gpu(a, w, a_scale, w_scale, bias, out_dtype, activation, return_acc, exact=False):
    _on_gpu(a, w, a_scale, w_scale, bias)
    out, acc = _mm_meta(a, w, a_scale, w_scale, bias, out_dtype, activation, return_acc, exact)
    M, K = a.shape
    Nf = w.shape[0]
    if M == 0:
        return out, acc
    a, w = _kernel_rows(a, 16), _kernel_rows(w, 16)
    a_scale = a_scale.contiguous()
    w_scale = w_scale.contiguous()
    bias = None if bias is None else bias.contiguous()
    sa_stride = 1 if a_scale.numel() == M and M > 1 else 0
    sw_stride = 1 if w_scale.numel() == Nf and Nf > 1 else 0
    if a.dtype == torch.float8_e4m3fn:
        fn = "xgen_scaled_mm_fp8_exact" if exact else "xgen_scaled_mm_fp8"
    else:
        fn = "xgen_quant_matmul_int8"
    st = getattr(N.lib(), fn)(
        a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), M, Nf, K, a_scale.data_ptr(), sa_stride,
        w_scale.data_ptr(), sw_stride, N.ptr(bias), N.DTYPE_NONE if bias is None else N.dtype_code(bias.dtype),
        activation, out.data_ptr(), N.dtype_code(out_dtype), out.stride(0),
        acc.data_ptr() if return_acc else None, N.stream_of(a))
    N.check(st, fn)
    return out, acc


def _gate_gpu(residual, branch, gate_table, indices):
    _on_gpu(residual, branch, gate_table, indices)
    out = _gate_meta(residual, branch, gate_table, indices)
    if out.numel() == 0:
        return out
    residual, branch, gate_table = _kernel_rows(residual, 8), _kernel_rows(branch, 8), _kernel_rows(gate_table, 8)
    indices = indices.contiguous()
    B, S, H = residual.shape
    st = N.lib().xgen_gate_residual(
        residual.data_ptr(), residual.stride(0), residual.stride(1), branch.data_ptr(), branch.stride(0),
        branch.stride(1), gate_table.data_ptr(), gate_table.stride(0), gate_table.shape[0], indices.data_ptr(),
        B, S, H, out.data_ptr(), N.stream_of(residual))
    N.check(st, "xgen_gate_residual")
    return out


def _modulate_gpu(x, scale_table, shift_table, indices, scale_is_one_plus=False):
    _on_gpu(x, scale_table, shift_table, indices)
    out = _modulate_meta(x, scale_table, shift_table, indices, scale_is_one_plus)
    if out.numel() == 0:
        return out
    x, scale_table, shift_table = _kernel_rows(x, 8), _kernel_rows(scale_table, 8), _kernel_rows(shift_table, 8)
    indices = indices.contiguous()
    B, S, H = x.shape
    st = N.lib().xgen_indexed_modulate(
        x.data_ptr(), x.stride(0), x.stride(1), scale_table.data_ptr(), scale_table.stride(0),
        shift_table.data_ptr(), shift_table.stride(0), scale_table.shape[0], indices.data_ptr(), B, S, H,
        int(bool(scale_is_one_plus)), out.data_ptr(), N.stream_of(x))
    N.check(st, "xgen_indexed_modulate")
    return out


def _merge_gpu(back_recv, out_dtype):
    _on_gpu(back_recv)
    q, scale = _merge_meta(back_recv, out_dtype)
    if q.numel() == 0:
        return q, scale
    back_recv = _aligned_flat(back_recv)
    splits, owners, seq, batch, chunk = back_recv.shape
    st = N.lib().xgen_merge_quant(N.dtype_code(out_dtype), back_recv.data_ptr(), splits, owners, seq, batch, chunk,
                                  q.data_ptr(), scale.data_ptr(), N.stream_of(back_recv))
    N.check(st, "xgen_merge_quant")
    return q, scale


_SILU_TABLES: dict[int, torch.Tensor] = {}


def silu_table(device: torch.device) -> torch.Tensor:
    """The device's bf16(silu(g)) table over all 65,536 bf16 patterns (xgen_silu_bf16_table), built on
    first use and kept for the process.  Built on the current stream and waited for once, so any
    stream may read it afterwards."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    t = _SILU_TABLES.get(idx)
    if t is None:
        t = torch.empty(65536, dtype=torch.int16, device=torch.device("cuda", idx))
        stream = torch.cuda.current_stream(t.device)
        N.check(N.lib().xgen_silu_bf16_table(t.data_ptr(), stream.cuda_stream), "xgen_silu_bf16_table")
        stream.synchronize()
        _SILU_TABLES[idx] = t
    return t


def _swiglu_gpu(u, gate_first, out_dtype, scale_mode, return_act):
    _on_gpu(u)
    q, s, act = _swiglu_meta(u, gate_first, out_dtype, scale_mode, return_act)
    if q.numel() == 0:
        return q, s, act
    u = _kernel_rows(u, 8)
    table = silu_table(u.device)
    st = N.lib().xgen_swiglu_quant_lut(
        u.data_ptr(), u.shape[0], u.shape[1], u.shape[2] // 2, u.stride(0), u.stride(1), int(bool(gate_first)),
        N.dtype_code(out_dtype), scale_mode, q.data_ptr(), s.data_ptr(), act.data_ptr() if return_act else None,
        table.data_ptr(), N.stream_of(u))
    N.check(st, "xgen_swiglu_quant_lut")
    return q, s, act


def _mm_gate_gpu(a, w, a_scale, w_scale, bias, residual, gate_table, indices):
    _on_gpu(a, w, a_scale, w_scale, bias, residual, gate_table, indices)
    out = _mm_gate_meta(a, w, a_scale, w_scale, bias, residual, gate_table, indices)
    M, K = a.shape
    Nf = w.shape[0]
    if M == 0:
        return out
    a, w = _kernel_rows(a, 16), _kernel_rows(w, 16)
    a_scale, w_scale = a_scale.contiguous(), w_scale.contiguous()
    bias = None if bias is None else bias.contiguous()
    residual, gate_table = _kernel_rows(residual, 8), _kernel_rows(gate_table, 8)
    indices = indices.contiguous()
    st = N.lib().xgen_w8a8_gate_residual(
        N.dtype_code(a.dtype), a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), M, Nf, K, a_scale.data_ptr(),
        1 if a_scale.numel() == M and M > 1 else 0, w_scale.data_ptr(), 1 if w_scale.numel() == Nf and Nf > 1 else 0,
        N.ptr(bias), N.DTYPE_NONE if bias is None else N.dtype_code(bias.dtype), residual.data_ptr(),
        residual.stride(0), gate_table.data_ptr(), gate_table.stride(0), gate_table.shape[0], indices.data_ptr(),
        indices.shape[0], out.data_ptr(), out.stride(0), N.stream_of(a))
    N.check(st, "xgen_w8a8_gate_residual")
    return out


_IMPLS = {
    "quantize_rows": (_quantize_rows_gpu, _quantize_rows_meta),
    "abs_peak": (_peak_gpu, _peak_meta),
    "fp8_tensor_scale": (_tensor_scale_gpu, _peak_meta),
    "fp8_pack": (_pack_gpu, _pack_meta),
    "norm_affine_quant": (_norm_gpu, _norm_meta),
    "scaled_mm": (_mm_gpu, _mm_meta),
    "gate_residual": (_gate_gpu, _gate_meta),
    "indexed_modulate": (_modulate_gpu, _modulate_meta),
    "merge_quant": (_merge_gpu, _merge_meta),
    "swiglu_quant": (_swiglu_gpu, _swiglu_meta),
    "scaled_mm_gate_residual": (_mm_gate_gpu, _mm_gate_meta),
}


def register() -> None:
    """Defines the xgen_amd operators (idempotent; does not load the HIP library)."""
    global _LIB
    if _LIB is not None:
        return
    lib = torch.library.Library(NAMESPACE, "DEF")
    for name, schema in SCHEMAS.items():
        lib.define(schema)
        gpu, meta = _IMPLS[name]
        lib.impl(name, gpu, "CUDA")
        lib.impl(name, meta, "Meta")
    _LIB = lib


register()
xops = getattr(torch.ops, NAMESPACE)
