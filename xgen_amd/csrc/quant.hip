// Dynamic quantizers for the W8A8 linear path (gfx950).
//
//  * xgen_quantize_rows  — per-row FP8 e4m3fn (the arithmetic of
//    x_base/x_base/operator/h3_fp8.py:9-12 applied per row) or per-row INT8
//    (npu_dynamic_quant as restated in npu_fusion/f2bc/op_kernel/f2bc_kernel.asc:89-107).
//  * xgen_quantize_rows_gelu — the same of dtype(gelu_tanh(x)): the FFN's GELU
//    (x_diffusers/x_diffusers/framework/transformer/hunyuan.py:358, diffusers
//    FeedForward "gelu-approximate") and the down-projection's input quantization
//    in one pass over the hidden activation.
//  * xgen_abs_peak / xgen_fp8_tensor_scale / xgen_fp8_pack — the per-tensor
//    activation quantizer of x_base/x_base/operator/h3_fp8_quant.py:9-25 and
//    h3_abs_peak.py:14-25.
//
// Row kernel layout: each row is read once into registers as 16-byte chunks
// (8 elements), consecutive lanes on consecutive chunks; the row's NaN-
// propagating max |x| is an integer max over the 16-bit magnitudes, reduced
// across the wave with cross-lane shuffles (and across the row's waves through
// LDS); the row is then quantized from registers and written as 8-byte chunks.
#include <mutex>

#include "xgen_common.h"

namespace xgen {

namespace {

constexpr int kThreads = 256;  // 4 waves per workgroup

// dtype(gelu_tanh(x)) of the 8 values of a chunk, in place (a chunk of zeros
// stays zeros: gelu_tanh(0) = 0)
template <int DT>
__device__ __forceinline__ u32x4 gelu_chunk(const u32x4 &c) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = gelu_tanh(Half2<DT>::lo(w[i])), hi = gelu_tanh(Half2<DT>::hi(w[i]));
    o[i] = DT == XGEN_DTYPE_BF16 ? pack_bf16x2(lo, hi) : pack_f16x2(lo, hi);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// the 16-bit pattern of dtype(gelu_tanh(x)) for a 16-bit input pattern.  The
// empty asm keeps the product an f32 value: without it the f16 rounding of
// x * r (x an f16 widened to f32) is selected as v_fma_mixlo_f16 x, r, +0,
// which turns a -0 product (x = -0, or x far below 0 where r = 0) into +0.
template <int DT>
__device__ __forceinline__ uint32_t gelu_bits(uint32_t b) {
  float g = gelu_tanh(Half2<DT>::lo(b));
  asm volatile("" : "+v"(g));
  return (DT == XGEN_DTYPE_BF16 ? pack_bf16x2(g, 0.0f) : pack_f16x2(g, 0.0f)) & 0xffffu;
}

// WPR waves per row, CH chunks of 8 elements per lane: one row covers up to
// 512 * WPR * CH elements.  Requires cols % 8 == 0 and 16-byte aligned rows.
//
// Streaming: a grid of a few workgroups per CU walks the rows (4 / WPR rows
// per workgroup per step); each wave loads its next row before it reduces and
// stores the current one, so loads stay in flight through the reduction.
// gfx9 counts loads and stores with one in-order counter, so the loop's memory
// accesses are all unconditional and the same on every path: rows go through
// per-row buffer resources (chunks past a row's end load zeros, their stores
// are dropped), rows past the end redo the last row (writing the same bytes as
// its owner), and the first row is peeled so that the loop is entered as it is
// repeated; the compiler's wait counts then name exactly the loads a step
// needs.  The wave index is made wave-uniform, so row addresses are
// scalar-unit work.  NT: the input is read non-temporally (calls larger than
// the last-level cache).  ACT: XGEN_ACT_GELU_TANH quantizes dtype(gelu_tanh(x)),
// applied to the row in registers.
template <int DT, int OUT, int WPR, int CH, bool NT, int ACT>
__global__ __launch_bounds__(kThreads) void quant_rows_vec_kernel(
    const uint8_t *__restrict__ x, int64_t rows, int cols, int64_t ldx_bytes,
    uint8_t *__restrict__ q, int64_t ldq, float *__restrict__ scale) {
  constexpr int kRowsPerBlock = 4 / WPR;
  __shared__ uint32_t red[2][4];  // cross-wave max, double-buffered by step parity
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int row_in_block = wave / WPR;
  const int lane_in_row = (wave % WPR) * 64 + lane;
  const int nchunks = cols >> 3;
  const int64_t step = (int64_t)gridDim.x * kRowsPerBlock;
  // byte offset of chunk j of this lane in an input row (kOutOfRange past the end)
  auto in_off = [&](int j) -> uint32_t {
    const int ci = lane_in_row + j * 64 * WPR;
    return ci < nchunks ? (uint32_t)ci * 16u : kOutOfRange;
  };
  auto clamp_row = [&](int64_t row) { return row < rows ? row : rows - 1; };
  auto load_row = [&](int64_t row, u32x4 (&c)[CH]) {
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(x + clamp_row(row) * ldx_bytes), (short)0, cols * 2, kBufferFlags);
#pragma unroll
    for (int j = 0; j < CH; ++j) c[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, in_off(j), 0, NT ? kCachePolicyNT : 0);
  };

  u32x4 c[CH], cn[CH];
  // one row: issue the next row's read, reduce, quantize from registers, store
  auto row_step = [&](int64_t base, int parity) {
    const int64_t row = clamp_row(base + row_in_block);
    __builtin_amdgcn_sched_barrier(0);
    load_row(base + step + row_in_block, cn);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (ACT == XGEN_ACT_GELU_TANH) {
#pragma unroll
      for (int j = 0; j < CH; ++j) c[j] = gelu_chunk<DT>(c[j]);
    }
    u16x2 m = {0, 0};
#pragma unroll
    for (int j = 0; j < CH; ++j) m = absmax_chunk<DT>(c[j], m);
    uint32_t amax_bits = wave_max_u32(hmax_u16x2(m));
    if constexpr (WPR > 1) {
      if (lane == 0) red[parity][wave] = amax_bits;
      __syncthreads();
      const int w0 = row_in_block * WPR;
#pragma unroll
      for (int i = 0; i < WPR; ++i) amax_bits = amax_bits > red[parity][w0 + i] ? amax_bits : red[parity][w0 + i];
    }
    const float amax = Half2<DT>::from_absbits(amax_bits);
    const RowQuant p = (OUT == XGEN_DTYPE_E4M3) ? fp8_row_params(amax) : i8_row_params(amax);
    const __amdgpu_buffer_rsrc_t rq =
        __builtin_amdgcn_make_buffer_rsrc(q + row * ldq, (short)0, cols, kBufferFlags);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      float v[8];
      unpack8<DT>(c[j], v);
      // a chunk past the end: its offset stays past the row's bytes, the store is dropped
      __builtin_amdgcn_raw_buffer_store_b64(quant8<OUT>(v, p), rq, in_off(j) >> 1, 0, 0);
    }
    scale[row] = p.s;  // every lane of the row: the same value
#pragma unroll
    for (int j = 0; j < CH; ++j) c[j] = cn[j];
  };

  int64_t base = (int64_t)blockIdx.x * kRowsPerBlock;  // uniform over the workgroup
  load_row(base + row_in_block, c);
  if (base >= rows) return;
  row_step(base, 0);
  base += step;
  for (int parity = 1; base < rows; base += step, parity ^= 1) row_step(base, parity);
}

// Any width / alignment: one workgroup per row, two passes over global memory.
template <int DT, int OUT, int ACT>
__global__ __launch_bounds__(kThreads) void quant_rows_generic_kernel(
    const uint16_t *__restrict__ x, int64_t rows, int64_t cols, int64_t ldx,
    uint8_t *__restrict__ q, int64_t ldq, float *__restrict__ scale) {
  const int64_t row = blockIdx.x;
  const uint16_t *xr = x + row * ldx;
  uint32_t mb = 0;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    uint32_t b = (ACT == XGEN_ACT_GELU_TANH ? gelu_bits<DT>(xr[c]) : xr[c]) & 0x7fffu;
    mb = mb > b ? mb : b;
  }
  mb = wave_max_u32(mb);
  __shared__ uint32_t red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mb;
  __syncthreads();
  mb = red[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) mb = mb > red[i] ? mb : red[i];
  const float amax = Half2<DT>::from_absbits(mb);
  const RowQuant p = (OUT == XGEN_DTYPE_E4M3) ? fp8_row_params(amax) : i8_row_params(amax);
  uint8_t *qr = q + row * ldq;
  for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
    const uint32_t w = ACT == XGEN_ACT_GELU_TANH ? gelu_bits<DT>(xr[c]) : xr[c];
    const float v = Half2<DT>::lo(w);
    uint32_t b;
    if constexpr (OUT == XGEN_DTYPE_E4M3) {
      b = p.finite ? (pack_e4m3x4(div_by_row_scale(v, p.mul, p.mul_lo), 0.f, 0.f, 0.f) & 0xffu)
                   : e4m3_slow_byte(v, p.s);
    } else {
      b = p.finite ? q_i8(v, p.mul) : i8_slow_byte(v, p.mul);
    }
    qr[c] = (uint8_t)b;
  }
  if (threadIdx.x == 0) scale[row] = p.s;
}

template <int DT, int OUT, int WPR, int CH, bool NT, int ACT>
void launch_vec_policy(const void *x, int64_t rows, int64_t cols, int64_t ldx, void *q, int64_t ldq,
                       float *scale, hipStream_t stream) {
  constexpr int kRowsPerBlock = 4 / WPR;
  // as many workgroups as are resident at once (a streaming grid must not queue)
  static const int per_cu = resident_blocks_per_cu(quant_rows_vec_kernel<DT, OUT, WPR, CH, NT, ACT>, kThreads);
  const int64_t need = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  const int64_t blocks = need < cap ? need : cap;
  quant_rows_vec_kernel<DT, OUT, WPR, CH, NT, ACT><<<dim3((unsigned)blocks), dim3(kThreads), 0, stream>>>(
      static_cast<const uint8_t *>(x), rows, (int)cols, ldx * 2, static_cast<uint8_t *>(q), ldq, scale);
}

template <int DT, int OUT, int ACT, int WPR, int CH>
void launch_vec(const void *x, int64_t rows, int64_t cols, int64_t ldx, void *q, int64_t ldq,
                float *scale, hipStream_t stream) {
  if (rows * cols * 3 > kLastLevelCacheBytes)  // 2 bytes read + 1 written per element
    launch_vec_policy<DT, OUT, WPR, CH, true, ACT>(x, rows, cols, ldx, q, ldq, scale, stream);
  else
    launch_vec_policy<DT, OUT, WPR, CH, false, ACT>(x, rows, cols, ldx, q, ldq, scale, stream);
}

template <int DT, int OUT, int ACT>
int quantize_rows_typed(const void *x, int64_t rows, int64_t cols, int64_t ldx, void *q,
                        int64_t ldq, float *scale, hipStream_t stream) {
  const bool vec = (cols % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) && aligned16(x) &&
                   ((reinterpret_cast<uintptr_t>(q) & 7u) == 0);
  // (waves per row, chunks per lane) covering the row with at most 4 chunks
  // (32 values) per lane where 4 waves suffice (register budget of the
  // streaming kernel, which holds the current and the next row).
  if (vec && cols <= 512 * 2) {
    launch_vec<DT, OUT, ACT, 1, 2>(x, rows, cols, ldx, q, ldq, scale, stream);
  } else if (vec && cols <= 512 * 4) {
    launch_vec<DT, OUT, ACT, 1, 4>(x, rows, cols, ldx, q, ldq, scale, stream);
  } else if (vec && cols <= 1024 * 3) {
    launch_vec<DT, OUT, ACT, 2, 3>(x, rows, cols, ldx, q, ldq, scale, stream);
  } else if (vec && cols <= 1024 * 4) {
    launch_vec<DT, OUT, ACT, 2, 4>(x, rows, cols, ldx, q, ldq, scale, stream);
  } else if (vec && cols <= 2048 * 3) {
    launch_vec<DT, OUT, ACT, 4, 3>(x, rows, cols, ldx, q, ldq, scale, stream);
  } else if (vec && cols <= 2048 * 4) {
    launch_vec<DT, OUT, ACT, 4, 4>(x, rows, cols, ldx, q, ldq, scale, stream);
  } else if (vec && cols <= 2048 * 6) {
    launch_vec<DT, OUT, ACT, 4, 6>(x, rows, cols, ldx, q, ldq, scale, stream);
  } else if (vec && cols <= 2048 * 8) {
    launch_vec<DT, OUT, ACT, 4, 8>(x, rows, cols, ldx, q, ldq, scale, stream);
  } else {
    quant_rows_generic_kernel<DT, OUT, ACT><<<dim3((unsigned)rows), dim3(kThreads), 0, stream>>>(
        static_cast<const uint16_t *>(x), rows, cols, ldx, static_cast<uint8_t *>(q), ldq, scale);
  }
  return XGEN_OK;
}

// ---------------------------------------------------------------------------
// per-tensor path
// ---------------------------------------------------------------------------
constexpr int kPeakBlocksMax = 1024;

// Grid-stride NaN-propagating max |x| -> one partial (as 16-bit magnitude bits)
// per workgroup.
template <int DT>
__global__ __launch_bounds__(kThreads) void abs_peak_partial_kernel(
    const uint8_t *__restrict__ x, int64_t numel, uint32_t *__restrict__ partial) {
  const int64_t nchunks = numel >> 3;
  u16x2 m = {0, 0};
  for (int64_t ci = (int64_t)blockIdx.x * kThreads + threadIdx.x; ci < nchunks;
       ci += (int64_t)gridDim.x * kThreads) {
    const u32x4 c = *reinterpret_cast<const u32x4 *>(x + ci * 16);
    m = absmax_chunk<DT>(c, m);
  }
  uint32_t mb = hmax_u16x2(m);
  // tail elements (numel % 8) handled by the first workgroup
  if (blockIdx.x == 0) {
    const uint16_t *xs = reinterpret_cast<const uint16_t *>(x);
    for (int64_t i = (nchunks << 3) + threadIdx.x; i < numel; i += kThreads) {
      const uint32_t b = xs[i] & 0x7fffu;
      mb = mb > b ? mb : b;
    }
  }
  mb = wave_max_u32(mb);
  __shared__ uint32_t red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mb;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = red[0];
    for (int i = 1; i < 4; ++i) r = r > red[i] ? r : red[i];
    partial[blockIdx.x] = r;
  }
}

// One workgroup: reduce the partials; write the peak (mode 0) or the FP8
// per-tensor scale max(peak / 448, FLT_MIN) (mode 1).
template <int DT>
__global__ __launch_bounds__(kThreads) void abs_peak_final_kernel(const uint32_t *__restrict__ partial,
                                                                  int n, float *__restrict__ out,
                                                                  int mode) {
  uint32_t mb = 0;
  for (int i = threadIdx.x; i < n; i += kThreads) mb = mb > partial[i] ? mb : partial[i];
  mb = wave_max_u32(mb);
  __shared__ uint32_t red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mb;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = red[0];
    for (int i = 1; i < 4; ++i) r = r > red[i] ? r : red[i];
    const float peak = Half2<DT>::from_absbits(r);
    out[0] = mode == 0 ? canonical_nan(peak) : fp8_row_params(peak).s;
  }
}

// True when s is a scale the per-tensor scale kernel produces from an input
// value a: max(RN(a / 448), FLT_MIN) (a MAX over several such scales is one of
// them).  a is recovered as s * 448 rounded to the input type: s is within half
// an fp32 ulp of a / 448, far inside half a bf16 / f16 ulp of a.
template <int DT>
__device__ __forceinline__ bool peak_form_scale(float s) {
  if (!(s >= kFltMin) || !__builtin_isfinite(s)) return false;
  if (s == kFltMin) return true;
  float a;
  if constexpr (DT == XGEN_DTYPE_BF16) a = Half2<DT>::lo(pack_bf16x2(s * kE4M3Max, 0.0f) & 0xffffu);
  else a = (float)(_Float16)(s * kE4M3Max);
  return __builtin_isfinite(a) && fp8_row_params(a).s == s;
}

// q[i] = e4m3(clamp(x[i] / scale[0])) over a contiguous tensor.  For a scale of
// the per-tensor kernel's form the division takes the row quantizers' two
// operations, whose e4m3 byte equals IEEE division's for every input value not
// above the peak a behind the scale (the oracle's exhaustive check over all
// (x, a) pairs); larger values give quotients above 448 either way, which the
// clamp maps to 448.  Any other scale, and chunks holding a NaN or an infinity,
// use IEEE division (NaN -> 0x7f, +-Inf -> +-448): the two-operation form
// computes fma(x, r, x * r_lo), which is NaN for an infinite x when r_lo = 0
// (a power-of-two scale such as 1.0 or FLT_MIN).
template <int DT>
__global__ __launch_bounds__(kThreads) void fp8_pack_kernel(const uint8_t *__restrict__ x,
                                                            int64_t numel,
                                                            const float *__restrict__ scale,
                                                            uint8_t *__restrict__ q) {
  const float s = scale[0];
  const bool fast = peak_form_scale<DT>(s);
  const RowQuant p = fp8_scale_params(s);
  // a 16-bit magnitude at or above infinity's is an infinity or a NaN
  constexpr uint32_t kInfBits = DT == XGEN_DTYPE_BF16 ? 0x7f80u : 0x7c00u;
  const int64_t nchunks = numel >> 3;
  for (int64_t ci = (int64_t)blockIdx.x * kThreads + threadIdx.x; ci < nchunks;
       ci += (int64_t)gridDim.x * kThreads) {
    const u32x4 c = *reinterpret_cast<const u32x4 *>(x + ci * 16);
    float v[8];
    unpack8<DT>(c, v);
    u32x2 r;
    if (fast && hmax_u16x2(absmax_chunk<DT>(c, u16x2{0, 0})) < kInfBits) {
      float qv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) qv[i] = clamp448(div_by_row_scale(v[i], p.mul, p.mul_lo));
      r.x = pack_e4m3x4(qv[0], qv[1], qv[2], qv[3]);
      r.y = pack_e4m3x4(qv[4], qv[5], qv[6], qv[7]);
    } else {
      uint32_t b[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) b[i] = e4m3_slow_byte(v[i], s);
      r.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
      r.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    }
    *reinterpret_cast<u32x2 *>(q + ci * 8) = r;
  }
  if (blockIdx.x == 0) {
    const uint16_t *xs = reinterpret_cast<const uint16_t *>(x);
    for (int64_t i = (nchunks << 3) + threadIdx.x; i < numel; i += kThreads) {
      const float v = Half2<DT>::lo(xs[i]);
      q[i] = (uint8_t)e4m3_slow_byte(v, s);
    }
  }
}

int peak_blocks(int64_t numel) {
  const int64_t chunks = numel >> 3;
  int64_t b = (chunks + kThreads * 8 - 1) / (kThreads * 8);
  if (b < 1) b = 1;
  if (b > kPeakBlocksMax) b = kPeakBlocksMax;
  return (int)b;
}

template <int DT>
int abs_peak_typed(const void *x, int64_t numel, float *out, int mode, void *ws, hipStream_t stream) {
  const int nb = peak_blocks(numel);
  uint32_t *partial = static_cast<uint32_t *>(ws);
  abs_peak_partial_kernel<DT><<<dim3(nb), dim3(kThreads), 0, stream>>>(
      static_cast<const uint8_t *>(x), numel, partial);
  int st = launch_status("xgen_abs_peak(partial)");
  if (st != XGEN_OK) return st;
  abs_peak_final_kernel<DT><<<dim3(1), dim3(kThreads), 0, stream>>>(partial, nb, out, mode);
  return launch_status("xgen_abs_peak(final)");
}

int check_peak_args(const char *fn, int in_dtype, const void *x, int64_t numel, const void *out,
                    void *ws, size_t ws_bytes) {
  if (!is_input_dtype(in_dtype)) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: input dtype must be BF16 or F16", fn);
  if (numel <= 0) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: numel must be positive", fn);
  if (!x || !out || !ws) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (!aligned16(x)) return fail(XGEN_ERR_UNSUPPORTED, "%s: input must be 16-byte aligned", fn);
  if (ws_bytes < xgen_abs_peak_workspace_bytes(numel))
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: workspace too small (%zu < %zu bytes)", fn, ws_bytes,
                xgen_abs_peak_workspace_bytes(numel));
  return XGEN_OK;
}

}  // namespace

}  // namespace xgen

using namespace xgen;

namespace xgen {
namespace {
template <int ACT>
int quantize_rows_entry(const char *fn, int in_dtype, const void *x, int64_t rows, int64_t cols, int64_t ldx,
                        int out_dtype, void *q, int64_t ldq, float *scale, hipStream_t stream) {
  if (!is_input_dtype(in_dtype)) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: input dtype must be BF16 or F16", fn);
  if (!is_quant_dtype(out_dtype)) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: output dtype must be E4M3 or I8", fn);
  if (rows < 0 || cols <= 0 || ldx < cols || ldq < cols)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad shape rows=%lld cols=%lld ldx=%lld ldq=%lld", fn,
                (long long)rows, (long long)cols, (long long)ldx, (long long)ldq);
  if (rows > 0x7fffffffLL) return fail(XGEN_ERR_UNSUPPORTED, "%s: too many rows", fn);
  if (rows == 0) return ok();
  if (!x || !q || !scale) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (in_dtype == XGEN_DTYPE_BF16) {
    if (out_dtype == XGEN_DTYPE_E4M3)
      quantize_rows_typed<XGEN_DTYPE_BF16, XGEN_DTYPE_E4M3, ACT>(x, rows, cols, ldx, q, ldq, scale, stream);
    else
      quantize_rows_typed<XGEN_DTYPE_BF16, XGEN_DTYPE_I8, ACT>(x, rows, cols, ldx, q, ldq, scale, stream);
  } else {
    if (out_dtype == XGEN_DTYPE_E4M3)
      quantize_rows_typed<XGEN_DTYPE_F16, XGEN_DTYPE_E4M3, ACT>(x, rows, cols, ldx, q, ldq, scale, stream);
    else
      quantize_rows_typed<XGEN_DTYPE_F16, XGEN_DTYPE_I8, ACT>(x, rows, cols, ldx, q, ldq, scale, stream);
  }
  return launch_status(fn);
}
}  // namespace
}  // namespace xgen

extern "C" int xgen_quantize_rows(int in_dtype, const void *x, int64_t rows, int64_t cols,
                                  int64_t ldx, int out_dtype, void *q, int64_t ldq, float *scale,
                                  hipStream_t stream) {
  return quantize_rows_entry<XGEN_ACT_NONE>("xgen_quantize_rows", in_dtype, x, rows, cols, ldx, out_dtype, q, ldq,
                                            scale, stream);
}

extern "C" int xgen_quantize_rows_gelu(int in_dtype, const void *x, int64_t rows, int64_t cols,
                                       int64_t ldx, int out_dtype, void *q, int64_t ldq, float *scale,
                                       hipStream_t stream) {
  return quantize_rows_entry<XGEN_ACT_GELU_TANH>("xgen_quantize_rows_gelu", in_dtype, x, rows, cols, ldx, out_dtype,
                                                 q, ldq, scale, stream);
}

extern "C" size_t xgen_abs_peak_workspace_bytes(int64_t numel) {
  return (size_t)peak_blocks(numel < 0 ? 0 : numel) * sizeof(uint32_t);
}

extern "C" int xgen_abs_peak(int in_dtype, const void *x, int64_t numel, float *peak,
                             void *workspace, size_t workspace_bytes, hipStream_t stream) {
  int st = check_peak_args("xgen_abs_peak", in_dtype, x, numel, peak, workspace, workspace_bytes);
  if (st != XGEN_OK) return st;
  return in_dtype == XGEN_DTYPE_BF16 ? abs_peak_typed<XGEN_DTYPE_BF16>(x, numel, peak, 0, workspace, stream)
                                     : abs_peak_typed<XGEN_DTYPE_F16>(x, numel, peak, 0, workspace, stream);
}

extern "C" int xgen_fp8_tensor_scale(int in_dtype, const void *x, int64_t numel, float *scale,
                                     void *workspace, size_t workspace_bytes, hipStream_t stream) {
  int st = check_peak_args("xgen_fp8_tensor_scale", in_dtype, x, numel, scale, workspace, workspace_bytes);
  if (st != XGEN_OK) return st;
  return in_dtype == XGEN_DTYPE_BF16 ? abs_peak_typed<XGEN_DTYPE_BF16>(x, numel, scale, 1, workspace, stream)
                                     : abs_peak_typed<XGEN_DTYPE_F16>(x, numel, scale, 1, workspace, stream);
}

// Scratch of the allocation-free per-tensor scale: the per-workgroup partial
// maxima (at most kPeakBlocksMax of them, 4 KB).  Each GPU holds its own copy
// for the life of the process.  Host code never passes the name itself to a
// kernel (on the host it is a stand-in, not a device address): it uses the
// address hipGetSymbolAddress returns on each device, resolved once per device.
static __device__ __align__(256) uint32_t scratch[kPeakBlocksMax];
constexpr size_t kScratchBytes = sizeof(scratch);

namespace xgen {
namespace {

// Device address of `scratch` on the current device (resolved on the first call there).
int scratch_on_current_device(const char *fn, void **out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void *addr[kMaxDevices];
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(XGEN_ERR_HIP, "%s: no current HIP device (or device index above %d)", fn, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(XGEN_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev,
                  hipGetErrorString(e));
    addr[dev] = p;
  }
  *out = addr[dev];
  return XGEN_OK;
}

}  // namespace
}  // namespace xgen

extern "C" int xgen_fp8_tensor_scale_noalloc(int in_dtype, const void *x, int64_t numel, float *scale,
                                             hipStream_t stream) {
  const char *fn = "xgen_fp8_tensor_scale_noalloc";
  void *ws = nullptr;
  int st = scratch_on_current_device(fn, &ws);
  if (st != XGEN_OK) return st;
  // the partials a call needs never exceed the scratch (peak_blocks caps them), but check anyway
  if (numel > 0 && xgen_abs_peak_workspace_bytes(numel) > kScratchBytes)
    return fail(XGEN_ERR_UNSUPPORTED, "%s: %zu bytes of partial maxima exceed the %zu-byte scratch", fn,
                xgen_abs_peak_workspace_bytes(numel), kScratchBytes);
  st = check_peak_args(fn, in_dtype, x, numel, scale, ws, kScratchBytes);
  if (st != XGEN_OK) return st;
  // every partial the final reduction reads is written by this call first: nothing to clear
  return in_dtype == XGEN_DTYPE_BF16 ? abs_peak_typed<XGEN_DTYPE_BF16>(x, numel, scale, 1, ws, stream)
                                     : abs_peak_typed<XGEN_DTYPE_F16>(x, numel, scale, 1, ws, stream);
}

extern "C" int xgen_fp8_pack(int in_dtype, const void *x, int64_t numel, const float *scale, void *q,
                             hipStream_t stream) {
  const char *fn = "xgen_fp8_pack";
  if (!is_input_dtype(in_dtype)) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: input dtype must be BF16 or F16", fn);
  if (numel < 0) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: numel must be non-negative", fn);
  if (numel == 0) return ok();
  if (!x || !scale || !q) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (!aligned16(x) || (reinterpret_cast<uintptr_t>(q) & 7u))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: input must be 16-byte and output 8-byte aligned", fn);
  int64_t blocks = ((numel >> 3) + kThreads - 1) / kThreads;
  if (blocks < 1) blocks = 1;
  if (blocks > 8192) blocks = 8192;
  if (in_dtype == XGEN_DTYPE_BF16)
    fp8_pack_kernel<XGEN_DTYPE_BF16><<<dim3((unsigned)blocks), dim3(kThreads), 0, stream>>>(
        static_cast<const uint8_t *>(x), numel, scale, static_cast<uint8_t *>(q));
  else
    fp8_pack_kernel<XGEN_DTYPE_F16><<<dim3((unsigned)blocks), dim3(kThreads), 0, stream>>>(
        static_cast<const uint8_t *>(x), numel, scale, static_cast<uint8_t *>(q));
  return launch_status(fn);
}
