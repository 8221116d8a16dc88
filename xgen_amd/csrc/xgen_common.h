// Shared device helpers and host-side argument checking for the xgen_amd kernels.
// gfx950 (CDNA4) only: wave64, hardware bf16 and OCP e4m3fn conversions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "xgen_amd.h"

namespace xgen {

// ----------------------------------------------------------------------------
// host side: error reporting (defined in abi.hip)
// ----------------------------------------------------------------------------
int fail(int status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int ok();
// Maps the result of the launch just made to XGEN_OK / XGEN_ERR_HIP.
int launch_status(const char *what);
// Compute units of the current device (cached per device; 256 on MI355X).
int device_cu_count();
// Workgroups of `threads` threads of `kernel` resident on one CU at once (>= 1).
template <typename K>
int resident_blocks_per_cu(K kernel, int threads) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess || n < 1) n = 1;
  return n;
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool is_input_dtype(int dt) { return dt == XGEN_DTYPE_BF16 || dt == XGEN_DTYPE_F16; }
inline bool is_quant_dtype(int dt) { return dt == XGEN_DTYPE_E4M3 || dt == XGEN_DTYPE_I8; }

// ----------------------------------------------------------------------------
// device side
// ----------------------------------------------------------------------------
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Raw buffer resources (gfx9, 32-bit dword format): a load at an offset past
// the resource's byte count returns zeros and such a store is dropped, so lanes
// with nothing to move take the offset kOutOfRange instead of a branch.
constexpr int kBufferFlags = 0x00020000;
constexpr uint32_t kOutOfRange = 0x80000000u;
// Cache policy of a buffer access (gfx940 family): non-temporal.
constexpr int kCachePolicyNT = 2;
// MI355X's last-level (memory-side) cache.  A streaming call whose reads and
// writes exceed it reads its input non-temporally: measured on the per-token
// quantizer, ordinary loads are ~5% faster while the footprint fits (96-168 MB
// inputs; equal at 192 MB), non-temporal loads 14-16% faster beyond it
// (288-384 MB inputs).  A likely reason: the streamed input then stops
// evicting the call's own output lines from that cache.
constexpr int64_t kLastLevelCacheBytes = 256ll << 20;

constexpr float kE4M3Max = 448.0f;
// torch.finfo(torch.float32).tiny, the clamp floor of the FP8 scale (h3_fp8.py:11).
constexpr float kFltMin = 1.17549435082228750797e-38f;
// fl32(1/127): the INT8 scale multiplier (f2bc_kernel.asc:97).
constexpr float kInv127 = 1.0f / 127.0f;

// --- 16-bit float element access on packed dwords --------------------------
// Input element type tag: BF16 or F16, two elements per dword (element 0 in
// the low half).
template <int DT>
struct Half2;

template <>
struct Half2<XGEN_DTYPE_BF16> {
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  // |x| bit patterns of both halves; as unsigned 16-bit integers they order
  // like |x| with NaN above +inf, so an integer max propagates NaN.
  static __device__ __forceinline__ u16x2 absbits(uint32_t w) {
    return __builtin_bit_cast(u16x2, w & 0x7fff7fffu);
  }
  static __device__ __forceinline__ float from_absbits(uint32_t b) { return __uint_as_float(b << 16); }
};

template <>
struct Half2<XGEN_DTYPE_F16> {
  static __device__ __forceinline__ float lo(uint32_t w) {
    return (float)__builtin_bit_cast(f16x2, w).x;
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return (float)__builtin_bit_cast(f16x2, w).y;
  }
  static __device__ __forceinline__ u16x2 absbits(uint32_t w) {
    return __builtin_bit_cast(u16x2, w & 0x7fff7fffu);
  }
  static __device__ __forceinline__ float from_absbits(uint32_t b) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
  }
};

__device__ __forceinline__ u16x2 max_u16x2(u16x2 a, u16x2 b) {
  return __builtin_elementwise_max(a, b);
}

// Round-to-nearest-even fp32 -> bf16, two at a time (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// GELU with the tanh approximation (the GEMM epilogue's and the requant's: one definition, so
// both give the same bits), via tanh(z) = 2*sigmoid(2z) - 1:
// 0.5*x*(1 + tanh(z)) = x / (1 + exp(-2z)),  z = sqrt(2/pi) * (x + 0.044715 x^3).
__device__ __forceinline__ float gelu_tanh(float x) {
  // -2 z log2(e) = x (c0 + c1 x^2): the exponent of exp(-2z) in base 2
  constexpr float kC0 = (float)(-2.0 * 1.4426950408889634 * 0.7978845608028654);
  constexpr float kC1 = (float)(-2.0 * 1.4426950408889634 * 0.7978845608028654 * 0.044715);
  const float t = __builtin_amdgcn_exp2f(x * __builtin_fmaf(kC1, x * x, kC0));
  return x * __builtin_amdgcn_rcpf(1.0f + t);
}

// fp32 rounded to bf16 precision (RNE), returned as fp32: one
// v_cvt_pk_bf16_f32 with the value in the high half and +0 in the low half, so
// the word is the rounded value's fp32 bit pattern.
__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float(pack_bf16x2(0.0f, x));
}

// Gated residual of one 16-byte chunk (8 bf16 values each of residual r,
// branch y and gate t): bf16(r + bf16(y * t)), multiply, round, add, round.
__device__ __forceinline__ void round_bf16x2(float &a, float &b);
__device__ __forceinline__ u32x4 gate_residual8(const u32x4 &r, const u32x4 &y, const u32x4 &t);

// Rounds two floats to bf16 (RNE) with one conversion.
__device__ __forceinline__ void round_bf16x2(float &a, float &b) {
  const uint32_t w = pack_bf16x2(a, b);
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
}

__device__ __forceinline__ u32x4 gate_residual8(const u32x4 &r, const u32x4 &y, const u32x4 &t) {
  const uint32_t rw[4] = {r.x, r.y, r.z, r.w}, yw[4] = {y.x, y.y, y.z, y.w}, tw[4] = {t.x, t.y, t.z, t.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float p0 = __uint_as_float(yw[i] << 16) * __uint_as_float(tw[i] << 16);
    float p1 = __uint_as_float(yw[i] & 0xffff0000u) * __uint_as_float(tw[i] & 0xffff0000u);
    round_bf16x2(p0, p1);
    o[i] = pack_bf16x2(__uint_as_float(rw[i] << 16) + p0, __uint_as_float(rw[i] & 0xffff0000u) + p1);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// --- OCP e4m3fn packing -----------------------------------------------------
// v_cvt_pk_fp8_f32 rounds to nearest even into e4m3fn (gfx950: OCP format).
// Inputs here are always finite and within [-448, 448].
__device__ __forceinline__ uint32_t pack_e4m3x4(float a, float b, float c, float d) {
  // the first conversion's preserved high word is overwritten by the second:
  // any register serves as its input (a's, which it consumes anyway; no v_mov 0)
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __float_as_int(a), false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// Saturating clamp of a finite value to [-448, 448] (v_med3_f32).
__device__ __forceinline__ float clamp448(float v) {
  return __builtin_amdgcn_fmed3f(v, -kE4M3Max, kE4M3Max);
}

// The row quantizers' x / s in two operations: 1/s is carried as r_hi + r_lo
// (r_hi = 1/s rounded toward zero, r_lo = RN((1 - s*r_hi) * r_hi) >= 0, together
// about 46 bits) and q = RN(x*r_hi + RN(x*r_lo)).  For a finite scale the e4m3
// byte equals that of IEEE x / s for every (bf16|f16 x, amax) pair a row
// quantizer can see, both signs, at the row quantizers' scale floor FLT_MIN and
// at the wire codec's 1e-12 (exhaustive oracle checks); r_lo >= 0 keeps
// x = -0 at -0 (-0 * r_lo + -0 * r_hi), and a negative
// quotient that rounds to zero in e4m3 is encoded -0 by v_cvt_pk_fp8_f32, as
// IEEE x / s gives it.
__device__ __forceinline__ float div_by_row_scale(float x, float r_hi, float r_lo) {
  return __builtin_fmaf(x, r_hi, x * r_lo);
}

// INT8 lane value: rint_half_even(x * alpha) as a byte.
__device__ __forceinline__ uint32_t q_i8(float x, float alpha) {
  float y = __builtin_rintf(x * alpha);
  return (uint32_t)(int32_t)y & 0xffu;
}
// Four lane values as bytes, for finite products |x * alpha| <= 127.5 (the
// row quantizer's, alpha = fl(127 / amax)): y = fl(x * alpha) plus 1.5 * 2^23
// is rounded once, to the nearest integer with ties to even, and the sum's low
// mantissa byte is rint(y) in two's complement (the sum lies in [2^23, 2^24));
// v_perm_b32 gathers the four low bytes.  The product and the sum stay two
// roundings (no FMA contraction), as rint(fl(x * alpha)) requires.
__device__ __forceinline__ uint32_t pack_i8x4(float a, float b, float c, float d, float alpha) {
#pragma clang fp contract(off)
  constexpr float kRintMagic = 12582912.0f;  // 1.5 * 2^23
  const uint32_t za = __float_as_uint(a * alpha + kRintMagic), zb = __float_as_uint(b * alpha + kRintMagic);
  const uint32_t zc = __float_as_uint(c * alpha + kRintMagic), zd = __float_as_uint(d * alpha + kRintMagic);
  return __builtin_amdgcn_perm(zb, za, 0x0c0c0400u) | __builtin_amdgcn_perm(zd, zc, 0x04000c0cu);
}

// --- wave64 reductions ---------------------------------------------------------
// Wave64 reductions with DPP lane shuffles (no LDS round trips): quad
// permutes [1,0,3,2] and [2,3,0,1], half-row and row mirrors give every lane
// its 16-lane row's result; row_bcast15 / row_bcast31 (gfx9) fold rows 0-1
// into 1 and 0-2 into 3; lane 63 then holds the wave's result, read back as a
// wave-uniform value.
constexpr int kDppQuad1032 = 0xB1, kDppQuad2301 = 0x4E, kDppRowMirror = 0x140, kDppRowHalfMirror = 0x141,
              kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, 0xf, false);
}
__device__ __forceinline__ uint32_t max_u32(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max_u32(v, dpp_u32<kDppQuad1032>(0, v));
  v = max_u32(v, dpp_u32<kDppQuad2301>(0, v));
  v = max_u32(v, dpp_u32<kDppRowHalfMirror>(0, v));
  v = max_u32(v, dpp_u32<kDppRowMirror>(0, v));
  v = max_u32(v, dpp_u32<kDppRowBcast15, 0xa>(0, v));
  v = max_u32(v, dpp_u32<kDppRowBcast31, 0xc>(0, v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ float wave_sum_f32(float v) {
  auto sh = [](float x, auto ctrl_tag) {
    return __uint_as_float(dpp_u32<decltype(ctrl_tag)::value>(0, __float_as_uint(x)));
  };
  v += sh(v, std::integral_constant<int, kDppQuad1032>{});
  v += sh(v, std::integral_constant<int, kDppQuad2301>{});
  v += sh(v, std::integral_constant<int, kDppRowHalfMirror>{});
  v += sh(v, std::integral_constant<int, kDppRowMirror>{});
  v += __uint_as_float(dpp_u32<kDppRowBcast15, 0xa>(0, __float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppRowBcast31, 0xc>(0, __float_as_uint(v)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// NaN results are stored as the canonical quiet NaN 0x7fc00000 (division
// and conversions may produce other payloads).
__device__ __forceinline__ float canonical_nan(float v) { return v == v ? v : __builtin_nanf(""); }

// Per-row quantization parameters derived from the row's max |x| (as fp32).
struct RowQuant {
  float s;       // stored scale
  float mul;     // FP8: 1/s rounded toward zero (r_hi of div_by_row_scale); INT8: alpha = RN(127/amax)
  float mul_lo;  // FP8: r_lo of div_by_row_scale; INT8: unused (0)
  bool finite;   // FP8: scale finite (fast division valid)
};

// The FP8 parameters of a finite scale s >= FLT_MIN (or of a non-finite one:
// finite = false).
__device__ __forceinline__ RowQuant fp8_scale_params(float s) {
  RowQuant p;
  p.s = canonical_nan(s);
  p.finite = __builtin_isfinite(s);
  // r_hi = 1/s rounded toward zero.  v_rcp_f32 is within one ulp of 1/s (a
  // positive normal for a finite s >= FLT_MIN) and the residual 1 - s*r of an
  // FMA is exact: a negative one means r > 1/s (one ulp down); otherwise r goes
  // one ulp up when that value is still <= 1/s.
  float r = __builtin_amdgcn_rcpf(s);
  float e = __builtin_fmaf(-s, r, 1.0f);
  if (e < 0.0f) {
    r = __uint_as_float(__float_as_uint(r) - 1u);
    e = __builtin_fmaf(-s, r, 1.0f);
  } else {
    const float r1 = __uint_as_float(__float_as_uint(r) + 1u);
    const float e1 = __builtin_fmaf(-s, r1, 1.0f);
    if (e1 >= 0.0f) r = r1, e = e1;
  }
  p.mul = r;
  p.mul_lo = e * r;
  return p;
}

// 1/448 as r_hi + r_lo (r_hi rounded toward zero, r_lo = RN((1 - 448 r_hi) r_hi)),
// the division by the row scale's constant in div_by_row_scale's form.
constexpr float kInv448Hi = 0x1.249248p-9f, kInv448Lo = 0x1.249248p-33f;

// max(amax / 448, FLT_MIN) for a 16-bit amax (bf16 or f16 value), the FP8 row
// scale (h3_fp8.py:11 per row): the quotient in two operations, bit-identical to
// IEEE division for every 16-bit amax after the clamp (the oracle's exhaustive
// check); below 2^-90, where amax * r_lo would lose bits to underflow, IEEE
// division (a branch that is uniform wherever a wave quantizes one row).
__device__ __forceinline__ float fp8_row_scale(float amax) {
  float s;
  if (__builtin_expect(amax < 0x1p-90f, 0)) s = amax / kE4M3Max;
  else s = div_by_row_scale(amax, kInv448Hi, kInv448Lo);
  return (s < kFltMin) ? kFltMin : s;  // clamp_min keeps NaN
}

__device__ __forceinline__ RowQuant fp8_row_params(float amax) { return fp8_scale_params(fp8_row_scale(amax)); }

__device__ __forceinline__ RowQuant i8_row_params(float amax) {
  RowQuant p;
  p.s = canonical_nan(amax * kInv127);
  p.mul = 127.0f / amax;
  p.mul_lo = 0.0f;
  // amax == 0 or subnormal (alpha = inf), inf or NaN: products may be non-finite -> slow path.
  p.finite = amax > 0.0f && __builtin_isfinite(amax) && __builtin_isfinite(p.mul);
  return p;
}

// Slow per-element INT8 path (zero, subnormal or non-finite amax): a non-finite
// product gives 0, so a zero row quantizes to zeros (swiglu_quant_kernel.asc:72-75).
__device__ __forceinline__ uint32_t i8_slow_byte(float x, float alpha) {
  float y = x * alpha;
  y = __builtin_isfinite(y) ? __builtin_rintf(y) : 0.0f;
  return (uint32_t)(int32_t)y & 0xffu;
}

// Slow per-element FP8 path for rows whose scale is inf or NaN: IEEE division;
// NaN results are written as the canonical e4m3fn NaN 0x7f.
__device__ __forceinline__ uint32_t e4m3_slow_byte(float x, float s) {
  float v = x / s;
  if (v != v) return 0x7fu;
  return pack_e4m3x4(clamp448(v), 0.0f, 0.0f, 0.0f) & 0xffu;
}

// Quantizes 8 values (bf16/f16 values as fp32) into 8 bytes.  No clamp is
// needed on the E4M3 fast path: |x| <= amax and s = RN(amax / 448) bound the
// quotient by 448 (1 + 2^-22), below 464, and v_cvt_pk_fp8_f32 rounds such
// values to 448 (checked on the GPU for every bf16 amax).
template <int OUT>
__device__ __forceinline__ u32x2 quant8(const float (&v)[8], const RowQuant &p) {
  u32x2 r;
  if constexpr (OUT == XGEN_DTYPE_E4M3) {
    if (p.finite) {
      float q[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = div_by_row_scale(v[i], p.mul, p.mul_lo);
      r.x = pack_e4m3x4(q[0], q[1], q[2], q[3]);
      r.y = pack_e4m3x4(q[4], q[5], q[6], q[7]);
    } else {
      uint32_t b[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) b[i] = e4m3_slow_byte(v[i], p.s);
      r.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
      r.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    }
  } else {
    if (p.finite) {
      r.x = pack_i8x4(v[0], v[1], v[2], v[3], p.mul);
      r.y = pack_i8x4(v[4], v[5], v[6], v[7], p.mul);
    } else {
      uint32_t b[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) b[i] = i8_slow_byte(v[i], p.mul);
      r.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
      r.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    }
  }
  return r;
}

// Unpacks a 16-byte chunk of 8 bf16/f16 values to fp32.
template <int DT>
__device__ __forceinline__ void unpack8(const u32x4 &c, float (&v)[8]) {
  v[0] = Half2<DT>::lo(c.x);
  v[1] = Half2<DT>::hi(c.x);
  v[2] = Half2<DT>::lo(c.y);
  v[3] = Half2<DT>::hi(c.y);
  v[4] = Half2<DT>::lo(c.z);
  v[5] = Half2<DT>::hi(c.z);
  v[6] = Half2<DT>::lo(c.w);
  v[7] = Half2<DT>::hi(c.w);
}

template <int DT>
__device__ __forceinline__ u16x2 absmax_chunk(const u32x4 &c, u16x2 m) {
  m = max_u16x2(m, Half2<DT>::absbits(c.x));
  m = max_u16x2(m, Half2<DT>::absbits(c.y));
  m = max_u16x2(m, Half2<DT>::absbits(c.z));
  m = max_u16x2(m, Half2<DT>::absbits(c.w));
  return m;
}

__device__ __forceinline__ uint32_t hmax_u16x2(u16x2 m) {
  return m.x > m.y ? (uint32_t)m.x : (uint32_t)m.y;
}

}  // namespace xgen
