"""The C ABI: every symbol include/xgen_amd.h declares is exported by the built
library and declared to ctypes; argument validation fails before any HIP call
(no GPU needed)."""
import ctypes
import re

import pytest

from xgen_amd import _native as N

HEADER = N.Path(__file__).resolve().parents[1] / "include" / "xgen_amd.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|int64_t|size_t|const char \*)\s*(xgen_\w+)\(", text, re.M)))


def test_header_declares_the_path():
    names = declared_functions()
    for required in ("xgen_quantize_rows", "xgen_abs_peak", "xgen_fp8_tensor_scale", "xgen_fp8_pack",
                     "xgen_norm_affine_quant", "xgen_scaled_mm_fp8", "xgen_quant_matmul_int8"):
        assert required in names


def test_library_exports_every_declared_symbol(built_library):
    raw = ctypes.CDLL(str(built_library))
    for name in declared_functions():
        assert hasattr(raw, name), name


def test_ctypes_signatures_cover_the_header():
    assert set(N.SIGNATURES) == set(declared_functions())


def test_status_strings(built_library):
    L = N.lib()
    assert L.xgen_abi_version() == 1
    assert L.xgen_status_string(N.OK) == b"ok"
    assert L.xgen_status_string(N.ERR_UNSUPPORTED) == b"unsupported shape or layout"


_STRIDES = (N._c_i64 * 12)(384, 128, 128, 128, 384, 128, 128, 128, 384, 128, 128, 128)


@pytest.mark.parametrize("call,status,needle", [
    (lambda L: L.xgen_quantize_rows(9, 16, 4, 64, 64, N.DTYPE_E4M3, 16, 64, 16, None), N.ERR_INVALID_ARGUMENT, b"input dtype"),
    (lambda L: L.xgen_quantize_rows(N.DTYPE_BF16, 16, 4, 64, 32, N.DTYPE_E4M3, 16, 64, 16, None), N.ERR_INVALID_ARGUMENT, b"bad shape"),
    (lambda L: L.xgen_quantize_rows(N.DTYPE_BF16, None, 4, 64, 64, N.DTYPE_I8, 16, 64, 16, None), N.ERR_INVALID_ARGUMENT, b"null"),
    (lambda L: L.xgen_fp8_pack(N.DTYPE_BF16, 8, 64, 16, 16, None), N.ERR_UNSUPPORTED, b"aligned"),
    (lambda L: L.xgen_abs_peak(N.DTYPE_BF16, 16, 4096, 16, 16, 0, None), N.ERR_INVALID_ARGUMENT, b"workspace"),
    (lambda L: L.xgen_scaled_mm_fp8(16, 8, 16, 32, 4, 16, 32, 16, 1, 16, 1, None, N.DTYPE_NONE, 0, 16, N.DTYPE_BF16, 16, None, None),
     N.ERR_INVALID_ARGUMENT, b"leading"),
    (lambda L: L.xgen_scaled_mm_fp8(16, 48, 16, 48, 4, 16, 17, 16, 1, 16, 1, None, N.DTYPE_NONE, 0, 16, N.DTYPE_BF16, 16, None, None),
     N.ERR_UNSUPPORTED, b"multiples of 16"),
    (lambda L: L.xgen_quant_matmul_int8(16, 32, 16, 32, 4, 16, 32, 16, 2, 16, 1, None, N.DTYPE_NONE, 0, 16, N.DTYPE_BF16, 16, None, None),
     N.ERR_INVALID_ARGUMENT, b"stride"),
    (lambda L: L.xgen_quant_matmul_int8(16, 32, 16, 32, 4, 16, 32, 16, 1, 16, 1, None, N.DTYPE_NONE, 7, 16, N.DTYPE_BF16, 16, None, None),
     N.ERR_INVALID_ARGUMENT, b"activation"),
    (lambda L: L.xgen_norm_affine_quant(16, 1, 4, 9000, 9000, 9000, N.NORM_LAYER, None, N.DTYPE_NONE, 1e-6,
                                        16, 9000, 16, 9000, 20, 16, N.DTYPE_E4M3, 16, 16, None, None),
     N.ERR_UNSUPPORTED, b"exceeds"),
    (lambda L: L.xgen_norm_affine_quant(16, 1, 4, 64, 64, 64, 5, None, N.DTYPE_NONE, 1e-6,
                                        16, 64, 16, 64, 20, 16, N.DTYPE_E4M3, 16, 16, None, None),
     N.ERR_INVALID_ARGUMENT, b"norm kind"),
    (lambda L: L.xgen_norm_affine_quant(16, 1, 4, 64, 64, 64, N.NORM_RMS, 16, N.DTYPE_NONE, 1e-6,
                                        16, 64, 16, 64, 20, 16, N.DTYPE_E4M3, 16, 16, None, None),
     N.ERR_INVALID_ARGUMENT, b"disagree"),
    (lambda L: L.xgen_norm_affine_quant(16, 1, 4, 64, 64, 64, 2 | N.NORM_SCALE_ONE_PLUS, None, N.DTYPE_NONE, 1e-6,
                                        16, 64, 16, 64, 20, 16, N.DTYPE_E4M3, 16, 16, None, None),
     N.ERR_INVALID_ARGUMENT, b"norm kind"),
    (lambda L: L.xgen_adaln_one_plus(16, 4, 64, 32, 16, 64, None), N.ERR_INVALID_ARGUMENT, b"bad shape"),
    (lambda L: L.xgen_silu_bf16_table(None, None), N.ERR_INVALID_ARGUMENT, b"null"),
    (lambda L: L.xgen_silu_bf16_table(8, None), N.ERR_UNSUPPORTED, b"aligned"),
    (lambda L: L.xgen_swiglu_quant_lut(16, 1, 4, 64, 128, 128, 0, N.DTYPE_E4M3, 1, 16, 16, None, None, None),
     N.ERR_INVALID_ARGUMENT, b"null silu table"),
    (lambda L: L.xgen_swiglu_quant_lut(16, 1, 4, 64, 128, 128, 0, N.DTYPE_E4M3, 1, 16, 16, None, 8, None),
     N.ERR_UNSUPPORTED, b"silu table must be 16-byte aligned"),
    (lambda L: L.xgen_adaln_one_plus(None, 4, 64, 64, 16, 64, None), N.ERR_INVALID_ARGUMENT, b"null"),
    (lambda L: L.xgen_adaln_one_plus(16, 4, 60, 64, 16, 64, None), N.ERR_UNSUPPORTED, b"multiples of 8"),
    (lambda L: L.xgen_fp8_wire_encode(N.DTYPE_BF16, 2, 16, 16, 16, _STRIDES, 2, 3, 1, 1, 128, 0, 16, None),
     N.ERR_INVALID_ARGUMENT, b"streams"),
    (lambda L: L.xgen_fp8_wire_encode(N.DTYPE_BF16, 1, 16, None, None, _STRIDES, 2, 3, 1, 1, 66, 0, 16, None),
     N.ERR_INVALID_ARGUMENT, b"multiple of 4"),
    (lambda L: L.xgen_fp8_wire_encode(N.DTYPE_I8, 1, 16, None, None, _STRIDES, 2, 3, 1, 1, 64, 0, 16, None),
     N.ERR_INVALID_ARGUMENT, b"input dtype"),
    (lambda L: L.xgen_fp8_wire_encode(N.DTYPE_BF16, 1, 16, None, None, _STRIDES, 2, 3, 1, 1, 64, 6, 16, None),
     N.ERR_INVALID_ARGUMENT, b"peer_padding"),
    (lambda L: L.xgen_fp8_wire_encode(N.DTYPE_BF16, 1, 16, None, None, _STRIDES, 2, 3, 1, 1, 2048, 0, 16, None),
     N.ERR_UNSUPPORTED, b"exceeds"),
    (lambda L: L.xgen_fp8_wire_encode(N.DTYPE_BF16, 1, 17, None, None, _STRIDES, 2, 3, 1, 1, 64, 0, 16, None),
     N.ERR_UNSUPPORTED, b"element-aligned"),
    (lambda L: L.xgen_fp8_wire_decode(N.DTYPE_BF16, 3, 16, 2, 3, 64, 0, 16, None, 16, None),
     N.ERR_INVALID_ARGUMENT, b"null"),
    (lambda L: L.xgen_fp8_wire_decode(N.DTYPE_BF16, 1, 16, 2, 1 << 31, 64, 0, 16, None, None, None),
     N.ERR_UNSUPPORTED, b"2^30"),
    (lambda L: L.xgen_fp8_wire_encode_masked(N.DTYPE_BF16, 1, 16, None, None, _STRIDES, 2, 3, 1, 1, 64, -1, 16, None),
     N.ERR_INVALID_ARGUMENT, b"negative shape"),
    (lambda L: L.xgen_fp8_wire_encode_masked(N.DTYPE_BF16, 1, 16, None, None, None, 2, 3, 1, 1, 64, 4, 16, None),
     N.ERR_INVALID_ARGUMENT, b"null"),
    (lambda L: L.xgen_fp8_wire_decode_strided(N.DTYPE_BF16, 1, 16, 2, 3, 1, 1, 64, None, 6, 16, None, None, None),
     N.ERR_INVALID_ARGUMENT, b"null"),
    (lambda L: L.xgen_fp8_wire_decode_strided(N.DTYPE_BF16, 1, 16, 2, 3, 1, 1, 64, (N._c_i64 * 4)(64, -64, 0, 0), 6,
                                              16, None, None, None), N.ERR_INVALID_ARGUMENT, b"negative stride"),
    (lambda L: L.xgen_fp8_wire_decode_strided(N.DTYPE_I8, 1, 16, 2, 3, 1, 1, 64, (N._c_i64 * 4)(192, 64, 0, 0), 6,
                                              16, None, None, None), N.ERR_INVALID_ARGUMENT, b"output dtype"),
    (lambda L: L.xgen_fp8_wire_decode_strided(N.DTYPE_BF16, 1, 16, 2, 1 << 31, 1, 1, 64, (N._c_i64 * 4)(0, 64, 0, 0),
                                              6, 16, None, None, None), N.ERR_UNSUPPORTED, b"peer rows"),
    (lambda L: L.xgen_phaa_pack_qkv(16, 16, 16, 17, 4, 7, 2, 128, 7168, 7168, 100, 16, 16, 16, None),
     N.ERR_INVALID_ARGUMENT, b"row stride"),
    (lambda L: L.xgen_phaa_pack_qkv(16, 16, None, 17, 4, 7, 2, 128, 7168, 7168, 7168, 16, 16, 16, None),
     N.ERR_INVALID_ARGUMENT, b"null"),
    (lambda L: L.xgen_phaa_pack_qkv(16, 16, 16, 17, 4, 7, 2, 128, 7168, 7172, 7168, 16, 16, 16, None),
     N.ERR_UNSUPPORTED, b"multiples of 8"),
    (lambda L: L.xgen_phaa_pack_back(16, 2, 69, 128, 128, 256, 68, 16, None), N.ERR_INVALID_ARGUMENT,
     b"bad geometry"),
    (lambda L: L.xgen_phaa_pack_back(16, 2, 68, 100, 128, 256, 68, 16, None), N.ERR_UNSUPPORTED, b"multiples of 8"),
    (lambda L: L.xgen_phaa_merge_back(16, 7, 4, -1, 1, 256, 16, None), N.ERR_INVALID_ARGUMENT, b"bad geometry"),
    (lambda L: L.xgen_phaa_merge_back(16, 7, 4, 17, 1, 252, 16, None), N.ERR_UNSUPPORTED, b"multiple of 8"),
    (lambda L: L.xgen_phaa_merge_back(16, 7, 4, 1 << 20, 1 << 10, 256, 16, None), N.ERR_UNSUPPORTED,
     b"2^31 16-byte units"),
    (lambda L: L.xgen_merge_quant(N.DTYPE_BF16, 16, 7, 4, 17, 1, 256, 16, 16, None), N.ERR_INVALID_ARGUMENT,
     b"output dtype"),
    (lambda L: L.xgen_merge_quant(N.DTYPE_I8, 16, 0, 4, 17, 1, 256, 16, 16, None), N.ERR_INVALID_ARGUMENT,
     b"bad geometry"),
    (lambda L: L.xgen_merge_quant(N.DTYPE_I8, 16, 7, 4, 17, 1, 252, 16, 16, None), N.ERR_UNSUPPORTED,
     b"multiple of 8"),
    (lambda L: L.xgen_merge_quant(N.DTYPE_I8, 16, 9, 8, 17, 1, 256, 16, 16, None), N.ERR_UNSUPPORTED, b"16384"),
    (lambda L: L.xgen_merge_quant(N.DTYPE_I8, 16, 7, 4, 1 << 20, 1 << 12, 256, 16, 16, None), N.ERR_UNSUPPORTED,
     b"2^31"),
    (lambda L: L.xgen_merge_quant(N.DTYPE_I8, None, 7, 4, 17, 1, 256, 16, 16, None), N.ERR_INVALID_ARGUMENT,
     b"null"),
    (lambda L: L.xgen_merge_quant(N.DTYPE_I8, 16, 7, 4, 17, 1, 256, 12, 16, None), N.ERR_UNSUPPORTED, b"aligned"),
    (lambda L: L.xgen_indexed_modulate(16, 0, 64, 16, 64, 16, 64, 0, 16, 1, 4, 64, 0, 16, None),
     N.ERR_INVALID_ARGUMENT, b"bad shape"),
    (lambda L: L.xgen_indexed_modulate(16, 0, 32, 16, 64, 16, 64, 3, 16, 1, 4, 64, 0, 16, None),
     N.ERR_INVALID_ARGUMENT, b"row strides"),
    (lambda L: L.xgen_indexed_modulate(16, 0, 64, None, 64, 16, 64, 3, 16, 1, 4, 64, 0, 16, None),
     N.ERR_INVALID_ARGUMENT, b"null"),
    (lambda L: L.xgen_indexed_modulate(16, 0, 68, 16, 68, 16, 68, 3, 16, 1, 4, 60, 1, 16, None),
     N.ERR_UNSUPPORTED, b"multiples of 8"),
    (lambda L: L.xgen_indexed_modulate(24, 0, 64, 16, 64, 16, 64, 3, 16, 1, 4, 64, 1, 16, None),
     N.ERR_UNSUPPORTED, b"aligned"),
])
def test_validation_fails_before_launch(built_library, call, status, needle):
    L = N.lib()
    assert call(L) == status
    assert needle in L.xgen_last_error()


def test_empty_inputs_are_no_ops(built_library):
    L = N.lib()
    assert L.xgen_quantize_rows(N.DTYPE_BF16, None, 0, 64, 64, N.DTYPE_E4M3, None, 64, None, None) == N.OK
    assert L.xgen_scaled_mm_fp8(None, 32, None, 32, 0, 16, 32, None, 1, None, 1, None, N.DTYPE_NONE, 0,
                                None, N.DTYPE_BF16, 16, None, None) == N.OK
    assert L.xgen_fp8_wire_encode(N.DTYPE_BF16, 3, None, None, None, None, 2, 0, 1, 3, 128, 0, None, None) == N.OK
    assert L.xgen_fp8_wire_decode(N.DTYPE_F32, 1, None, 4, 0, 64, 0, None, None, None, None) == N.OK
    assert L.xgen_fp8_wire_encode_masked(N.DTYPE_BF16, 1, None, None, None, None, 2, 0, 1, 3, 128, 0, None,
                                         None) == N.OK
    assert L.xgen_fp8_wire_decode_strided(N.DTYPE_BF16, 3, None, 2, 5, 0, 3, 128, (N._c_i64 * 4)(0, 0, 0, 0), 0,
                                          None, None, None, None) == N.OK
    assert L.xgen_indexed_modulate(None, 0, 64, None, 64, None, 64, 3, None, 2, 0, 64, 0, None, None) == N.OK
    assert L.xgen_merge_quant(N.DTYPE_I8, None, 7, 4, 0, 1, 256, None, None, None) == N.OK
    assert L.xgen_phaa_pack_qkv(None, None, None, 0, 4, 7, 2, 128, 7168, 7168, 7168, None, None, None, None) == N.OK
    assert L.xgen_phaa_pack_back(None, 2, 0, 128, 128, 256, 0, None, None) == N.OK
    assert L.xgen_phaa_merge_back(None, 7, 4, 0, 1, 256, None, None) == N.OK
    assert L.xgen_last_error() == b""


def test_wire_peer_padding(built_library):
    L = N.lib()
    # peer_bytes = streams * peer_rows * (width + 4); padding = (-peer_bytes) mod 16
    assert L.xgen_fp8_wire_peer_padding(1, 17 * 3, 128, 1) == (-(17 * 3 * 132)) % 16 == 4
    assert L.xgen_fp8_wire_peer_padding(3, 20 * 2 * 3, 128, 1) == 0
    assert L.xgen_fp8_wire_peer_padding(3, 17, 128, 0) == 0
    for streams in (1, 3):
        for rows in range(1, 9):
            for width in (4, 8, 64, 68, 96, 128):
                pad = L.xgen_fp8_wire_peer_padding(streams, rows, width, 1)
                assert pad in (0, 4, 8, 12) and (streams * rows * (width + 4) + pad) % 16 == 0
