/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle's C restatement of the reference
 * quantizers.  Only tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline may load it, and only as a checker.  Nothing in xgen_amd uses it.
 *
 *  oracle_e4m3_encode        OCP e4m3fn round-to-nearest-even from the format's
 *                            definition (1-4-3 bits, bias 7, no inf, NaN 0x7f,
 *                            max 448); values above 464 overflow to NaN (464
 *                            itself ties to the even 448).  This is
 *                            the conversion `.to(torch.float8_e4m3fn)` performs
 *                            at x_base/x_base/operator/h3_fp8.py:12.
 *  oracle_quant_rows_fp8     quantize_per_tensor (h3_fp8.py:9-12) per row:
 *                            s = max(amax / 448, FLT_MIN); q = e4m3(clamp(x / s, +-448)).
 *  oracle_quant_rows_int8    the per-row int8 quantizer the reference restates in
 *                            npu_fusion/f2bc/op_kernel/f2bc_kernel.asc:89-107:
 *                            s = amax * fl(1/127); alpha = fl(127 / amax);
 *                            q = rint_half_even(fl(x * alpha)); a non-finite
 *                            product (NaN, or inf when 127 / amax overflows for
 *                            a subnormal amax) -> 0, as for a flushed zero row.
 *  oracle_check_fast_division   exhaustive check, for every (x, amax) pair of
 *                            16-bit inputs the row quantizers can see, that the
 *                            HIP row quantizers' division by the row scale
 *                            (r_hi = 1/s rounded toward zero, r_lo =
 *                            RN((1 - s*r_hi) * r_hi), q = RN(x*r_hi + RN(x*r_lo)))
 *                            gives the same e4m3 byte as IEEE x / s.
 *  oracle_check_scale_division  exhaustive check, for every 16-bit amax, that the
 *                            row scale amax / 448 computed in two operations
 *                            (amax * r_hi + RN(amax * r_lo) with r_hi, r_lo of 448)
 *                            is the IEEE quotient bit for bit.
 *  oracle_check_wire_division   the same check for the FP8 wire codec's scale
 *                            s = max(amax / 448, 1e-12) (phaa/fp8_transport.py:52),
 *                            whose kernels always take the fast division.
 *
 * NaN convention: any NaN byte is written as 0x7f (canonical positive NaN).
 * Build: oracle/build.py (gcc -O2, no fast-math: float division and fmaf are
 * IEEE correctly rounded).
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#define FMT_BF16 0
#define FMT_F16 1

static float f32_of_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t bits_of_f32(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* IEEE binary16 -> float, from the format's definition. */
static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) & 1u;
  const int e = (h >> 10) & 31;
  const uint32_t m = h & 1023u;
  float v;
  if (e == 31) v = m ? NAN : INFINITY;
  else if (e == 0) v = ldexpf((float)m, -24);
  else v = ldexpf((float)(m | 1024u), e - 25);
  return sign ? -v : v;
}

float oracle_half_to_f32(int fmt, uint16_t h) {
  return fmt == FMT_BF16 ? f32_of_bits((uint32_t)h << 16) : f16_to_f32(h);
}

uint8_t oracle_e4m3_encode(float v) {
  if (isnan(v)) return 0x7f;
  const uint8_t sign = (bits_of_f32(v) >> 31) ? 0x80 : 0x00;
  const float a = fabsf(v);
  /* 464 is the midpoint of 448 (mantissa 110) and the NaN code's 480 (111): a
   * tie goes to the even 448; anything above overflows (no inf) -> NaN. */
  if (a > 464.0f) return 0x7f | sign;
  if (a < 0.015625f) {                 /* below 2^-6: subnormal grid k * 2^-9 */
    const float k = nearbyintf(a * 512.0f); /* exact scaling, RNE */
    return sign | (uint8_t)k;           /* k == 8 encodes 2^-6 exactly */
  }
  int ex;
  const float f = frexpf(a, &ex); /* a = f * 2^ex, f in [0.5, 1) */
  int E = ex - 1;                 /* a in [2^E, 2^(E+1)) */
  const float frac = (f * 2.0f - 1.0f) * 8.0f; /* exact: mantissa in eighths */
  int m = (int)nearbyintf(frac);
  if (m == 8) {
    m = 0;
    E += 1;
  }
  return sign | (uint8_t)(((E + 7) << 3) | m);
}

float oracle_e4m3_decode(uint8_t b) {
  const int E = (b >> 3) & 15, m = b & 7;
  float v;
  if (E == 15 && m == 7) return NAN;
  if (E == 0) v = ldexpf((float)m, -9);
  else v = ldexpf(1.0f + (float)m / 8.0f, E - 7);
  return (b & 0x80) ? -v : v;
}

void oracle_e4m3_encode_array(const float *v, int64_t n, uint8_t *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_e4m3_encode(v[i]);
}

/* NaN-propagating max |x| of a row, as float. */
static float row_amax(int fmt, const uint16_t *x, int64_t cols) {
  float amax = 0.0f;
  for (int64_t c = 0; c < cols; ++c) {
    const float a = fabsf(oracle_half_to_f32(fmt, x[c]));
    if (isnan(a)) return NAN;
    if (a > amax) amax = a;
  }
  return amax;
}

void oracle_quant_rows_fp8(int fmt, const uint16_t *x, int64_t rows, int64_t cols, uint8_t *q,
                           float *scale) {
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t *xr = x + r * cols;
    float s = row_amax(fmt, xr, cols) / 448.0f;
    if (s < FLT_MIN) s = FLT_MIN; /* clamp_min(finfo.tiny), NaN kept */
    scale[r] = s;
    for (int64_t c = 0; c < cols; ++c) {
      float v = oracle_half_to_f32(fmt, xr[c]) / s;
      if (!isnan(v)) v = v > 448.0f ? 448.0f : (v < -448.0f ? -448.0f : v);
      q[r * cols + c] = oracle_e4m3_encode(v);
    }
  }
}

void oracle_quant_rows_int8(int fmt, const uint16_t *x, int64_t rows, int64_t cols, int8_t *q,
                            float *scale) {
  const float inv127 = 1.0f / 127.0f;
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t *xr = x + r * cols;
    const float amax = row_amax(fmt, xr, cols);
    const float alpha = 127.0f / amax;
    scale[r] = amax * inv127;
    for (int64_t c = 0; c < cols; ++c) {
      const float y = oracle_half_to_f32(fmt, xr[c]) * alpha;
      q[r * cols + c] = isfinite(y) ? (int8_t)nearbyintf(y) : 0;
    }
  }
}

/* The row quantizers' reciprocal pair: r_hi = RN(1/s), one ulp down when
 * s * RN(1/s) > 1 (so r_hi <= 1/s), and r_lo = RN((1 - s*r_hi) * r_hi) >= 0
 * (the residual is exact with an FMA). */
static void row_reciprocal(float s, float *r_hi, float *r_lo) {
  float r = 1.0f / s;
  float e = fmaf(-s, r, 1.0f);
  if (e < 0.0f) {
    r = nextafterf(r, 0.0f);
    e = fmaf(-s, r, 1.0f);
  }
  *r_hi = r;
  *r_lo = e * r;
}

static float row_div(float x, float r_hi, float r_lo) {
  const float t = x * r_lo;
  return fmaf(x, r_hi, t);
}

/* Every positive finite amax bit pattern in [amax_lo, amax_hi] and every
 * finite x with |x| <= amax of format fmt (both signs, so signed zeros and
 * underflowing negative quotients are covered): count of e4m3 bytes that differ
 * between IEEE x / s and the HIP row quantizers' division row_div. */
int64_t oracle_check_fast_division(int fmt, uint32_t amax_lo, uint32_t amax_hi) {
  int64_t bad = 0;
  for (uint32_t ab = amax_lo; ab <= amax_hi; ++ab) {
    const float amax = oracle_half_to_f32(fmt, (uint16_t)ab);
    if (!(amax > 0.0f) || isinf(amax) || isnan(amax)) continue;
    float s = amax / 448.0f;
    if (s < FLT_MIN) s = FLT_MIN;
    float r_hi, r_lo;
    row_reciprocal(s, &r_hi, &r_lo);
    for (uint32_t mag = 0; mag <= ab; ++mag) {
      for (uint32_t sign = 0; sign <= 0x8000u; sign += 0x8000u) {
        const float x = oracle_half_to_f32(fmt, (uint16_t)(mag | sign));
        float ref = x / s;
        float got = row_div(x, r_hi, r_lo);
        ref = ref > 448.0f ? 448.0f : (ref < -448.0f ? -448.0f : ref);
        got = got > 448.0f ? 448.0f : (got < -448.0f ? -448.0f : got);
        if (oracle_e4m3_encode(ref) != oracle_e4m3_encode(got)) ++bad;
      }
    }
  }
  return bad;
}

/* Row scale max(amax / 448, FLT_MIN) as the HIP kernels form it: for amax >=
 * 2^-90 the quotient in two operations, q = row_div(amax, r_hi, r_lo) with
 * r_hi, r_lo = row_reciprocal(448) (r_hi = 1/448 rounded toward zero); below
 * 2^-90 (where amax * r_lo would lose bits to underflow) IEEE division; then
 * the clamp (NaN stays NaN).  Every 16-bit pattern of format fmt (both signs,
 * zeros, subnormals, infinities and NaN): count of patterns whose float32 bits
 * differ from the IEEE form (NaN compares as NaN).  *r_hi_out / *r_lo_out
 * receive the constants. */
int64_t oracle_check_scale_division(int fmt, float *r_hi_out, float *r_lo_out) {
  float r_hi, r_lo;
  row_reciprocal(448.0f, &r_hi, &r_lo);
  *r_hi_out = r_hi;
  *r_lo_out = r_lo;
  int64_t bad = 0;
  for (uint32_t ab = 0; ab <= 0xffffu; ++ab) {
    const float amax = oracle_half_to_f32(fmt, (uint16_t)ab);
    float ref = amax / 448.0f, got = amax < 0x1p-90f ? amax / 448.0f : row_div(amax, r_hi, r_lo);
    ref = ref < FLT_MIN ? FLT_MIN : ref;
    got = got < FLT_MIN ? FLT_MIN : got;
    if (isnan(ref) ? !isnan(got) : bits_of_f32(ref) != bits_of_f32(got)) ++bad;
  }
  return bad;
}

/* Wire codec scale rule: every positive finite amax bit pattern in
 * [amax_lo, amax_hi] and every x with |x| <= amax (both signs); count of e4m3
 * bytes that differ between IEEE x / s and the kernels' row_div at the wire's
 * scale s = max(amax / 448, 1e-12). */
int64_t oracle_check_wire_division(int fmt, uint32_t amax_lo, uint32_t amax_hi) {
  int64_t bad = 0;
  for (uint32_t ab = amax_lo; ab <= amax_hi; ++ab) {
    const float amax = oracle_half_to_f32(fmt, (uint16_t)ab);
    if (!(amax > 0.0f) || isinf(amax) || isnan(amax)) continue;
    float s = amax / 448.0f;
    if (s < 1.0e-12f) s = 1.0e-12f;
    float r_hi, r_lo;
    row_reciprocal(s, &r_hi, &r_lo);
    for (uint32_t mag = 0; mag <= ab; ++mag) {
      for (uint32_t sign = 0; sign <= 0x8000u; sign += 0x8000u) {
        const float x = oracle_half_to_f32(fmt, (uint16_t)(mag | sign));
        float ref = x / s;
        float got = row_div(x, r_hi, r_lo);
        ref = ref > 448.0f ? 448.0f : (ref < -448.0f ? -448.0f : ref);
        got = got > 448.0f ? 448.0f : (got < -448.0f ? -448.0f : got);
        if (oracle_e4m3_encode(ref) != oracle_e4m3_encode(got)) ++bad;
      }
    }
  }
  return bad;
}
