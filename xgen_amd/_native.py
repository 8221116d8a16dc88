"""Loads libxgen_amd.so once per process and declares its C ABI (include/xgen_amd.h).

The library is loaded after torch so that it binds to the HIP runtime torch
uses (both link libamdhip64.so.7).  A missing or unloadable library raises
RuntimeError: there is no other implementation of these operators.
Library-path override: XGEN_AMD_LIBRARY (cf. the reference's H3_*_LIBRARY
overrides, x_base/x_base/operator/npu_fusion/nq2.py:10-15).
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

_lock = threading.Lock()
_lib = None

# dtype codes, include/xgen_amd.h
DTYPE_BF16, DTYPE_F16, DTYPE_F32, DTYPE_E4M3, DTYPE_I8, DTYPE_I32, DTYPE_NONE = 0, 1, 2, 3, 4, 5, -1
NORM_LAYER, NORM_RMS, NORM_SCALE_ONE_PLUS = 0, 1, 0x100
ACT_NONE, ACT_GELU_TANH = 0, 1
OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3

_TORCH_DTYPE = {
    torch.bfloat16: DTYPE_BF16,
    torch.float16: DTYPE_F16,
    torch.float32: DTYPE_F32,
    torch.float8_e4m3fn: DTYPE_E4M3,
    torch.int8: DTYPE_I8,
    torch.int32: DTYPE_I32,
}

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_ptr = ctypes.c_void_p
_c_float = ctypes.c_float
_c_size = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/xgen_amd.h
SIGNATURES = {
    "xgen_abi_version": (_c_int, []),
    "xgen_status_string": (ctypes.c_char_p, [_c_int]),
    "xgen_last_error": (ctypes.c_char_p, []),
    "xgen_quantize_rows": (_c_int, [_c_int, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr, _c_i64, _c_ptr, _c_ptr]),
    "xgen_quantize_rows_gelu": (_c_int, [_c_int, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr, _c_i64, _c_ptr, _c_ptr]),
    "xgen_abs_peak_workspace_bytes": (_c_size, [_c_i64]),
    "xgen_abs_peak": (_c_int, [_c_int, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "xgen_fp8_tensor_scale": (_c_int, [_c_int, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_size, _c_ptr]),
    "xgen_fp8_tensor_scale_noalloc": (_c_int, [_c_int, _c_ptr, _c_i64, _c_ptr, _c_ptr]),
    "xgen_fp8_pack": (_c_int, [_c_int, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr]),
    "xgen_norm_affine_quant": (_c_int, [
        _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr, _c_int, _c_float,
        _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]),
    "xgen_scaled_mm_fp8": (_c_int, [
        _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
        _c_ptr, _c_int, _c_int, _c_ptr, _c_int, _c_i64, _c_ptr, _c_ptr]),
    "xgen_scaled_mm_fp8_exact": (_c_int, [
        _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
        _c_ptr, _c_int, _c_int, _c_ptr, _c_int, _c_i64, _c_ptr, _c_ptr]),
    "xgen_quant_matmul_int8": (_c_int, [
        _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
        _c_ptr, _c_int, _c_int, _c_ptr, _c_int, _c_i64, _c_ptr, _c_ptr]),
    "xgen_gate_residual": (_c_int, [
        _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64,
        _c_ptr, _c_ptr]),
    "xgen_swiglu_quant": (_c_int, [
        _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr]),
    "xgen_silu_bf16_table": (_c_int, [_c_ptr, _c_ptr]),
    "xgen_swiglu_quant_lut": (_c_int, [
        _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
        _c_ptr]),
    "xgen_w8a8_gate_residual": (_c_int, [
        _c_int, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64,
        _c_ptr, _c_int, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr]),
    "xgen_adaln_one_plus": (_c_int, [_c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr]),
    "xgen_fp8_wire_peer_padding": (_c_i64, [_c_int, _c_i64, _c_i64, _c_int]),
    "xgen_fp8_wire_encode": (_c_int, [
        _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr,
        _c_ptr]),
    "xgen_fp8_wire_decode": (_c_int, [
        _c_int, _c_int, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr]),
    "xgen_phaa_pack_qkv": (_c_int, [
        _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr,
        _c_ptr, _c_ptr]),
    "xgen_phaa_pack_back": (_c_int, [_c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr]),
    "xgen_phaa_merge_back": (_c_int, [_c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr]),
    "xgen_merge_quant": (_c_int, [_c_int, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr]),
    "xgen_indexed_modulate": (_c_int, [
        _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int,
        _c_ptr, _c_ptr]),
    "xgen_fp8_wire_encode_masked": (_c_int, [
        _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr,
        _c_ptr]),
    "xgen_fp8_wire_decode_strided": (_c_int, [
        _c_int, _c_int, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr,
        _c_ptr]),
}


def library_path() -> Path:
    default = Path(__file__).resolve().parent / "_lib" / "libxgen_amd.so"
    return Path(os.environ.get("XGEN_AMD_LIBRARY", default)).resolve()


def lib() -> ctypes.CDLL:
    """The loaded library (loaded on first use, once per process, under a lock)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = library_path()
            if not path.is_file():
                raise RuntimeError(
                    f"xgen_amd native library not found at {path}; build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'`")
            handle = ctypes.CDLL(str(path))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            if handle.xgen_abi_version() != 1:
                raise RuntimeError(f"{path}: unexpected ABI version {handle.xgen_abi_version()}")
            _lib = handle
    return _lib


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_DTYPE[dtype]
    except KeyError:
        raise ValueError(f"dtype {dtype} has no xgen_amd code") from None


def check(status: int, fn: str) -> None:
    if status != OK:
        L = lib()
        raise RuntimeError(f"{fn}: {L.xgen_status_string(status).decode()}: {L.xgen_last_error().decode()}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream
