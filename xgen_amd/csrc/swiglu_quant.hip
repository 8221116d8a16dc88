// SwiGLU + per-row dynamic quantization (gfx950): the H3 FFN's activation and
// the requantization before its down-projection in one HBM pass.
//
//   u = [hidden | gate] (gate_first = 0, npu_fusion/f1b/op_kernel/swiglu_quant_reuse_kernel.asc:36-58)
//     or [gate | hidden] (gate_first = 1, x_base/x_base/operator/h3_swiglu.py:15-29), each F wide:
//   a = bf16(silu(gate)),  silu(g) = g / (1 + exp(-g))  (IEEE division)
//   v = bf16(hidden * a)
//   (q, s) = per-row quantization of v: E4M3 as xgen_quantize_rows, or I8 with
//            scale_mode 1: s = amax * fl(1/127); 0: s = 1 / fl(127 / amax)
//            (swiglu_quant_reuse_kernel.asc:80-89)
//
// Layout: streaming rows like the per-token quantizer — WPR waves per row,
// CH chunks of 8 outputs per lane; each wave loads its next row's hidden and
// gate chunks before it reduces and stores the current row; v stays in
// registers between the activation and the quantization.
#include "xgen_common.h"

namespace xgen {

namespace {

constexpr int kThreads = 256;

struct SwigluArgs {
  const uint8_t *u;
  int64_t sb, sr;  // bytes
  int64_t seq, rows;
  int half;        // F
  int gate_first;
  int scale_mode;  // I8 only
  uint8_t *q;
  float *scale;
  uint8_t *act;    // optional bf16 [rows, F]
};

// silu(g) = g / (1 + exp(-g)) as the reference computes it: IEEE division and
// the device library's accurate exponential (no fast-math in this build).
// (The hardware exp2 + reciprocal form measured 17% faster at H3 geometry but
// moves a share of the bf16 results by up to 2 ulps.)
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <int OUT, int WPR, int CH>
__global__ __launch_bounds__(kThreads) void swiglu_quant_kernel(SwigluArgs a) {
  constexpr int kRowsPerBlock = 4 / WPR;
  __shared__ uint32_t red[2][4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row_in_block = wave / WPR;
  const int lane_in_row = (wave % WPR) * 64 + lane;
  const int nchunks = a.half >> 3;
  const int64_t step = (int64_t)gridDim.x * kRowsPerBlock;
  const int hoff = a.gate_first ? a.half * 2 : 0, goff = a.gate_first ? 0 : a.half * 2;  // bytes

  auto load_row = [&](int64_t row, u32x4 (&h)[CH], u32x4 (&g)[CH]) {
    const bool ok = row < a.rows;
    const int64_t r = ok ? row : 0;
    const uint8_t *ur = a.u + (r / a.seq) * a.sb + (r % a.seq) * a.sr;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int ci = lane_in_row + j * 64 * WPR;
      const bool in = ok && ci < nchunks;
      h[j] = in ? *reinterpret_cast<const u32x4 *>(ur + hoff + (int64_t)ci * 16) : u32x4{0, 0, 0, 0};
      g[j] = in ? *reinterpret_cast<const u32x4 *>(ur + goff + (int64_t)ci * 16) : u32x4{0, 0, 0, 0};
    }
  };

  u32x4 h[CH], g[CH];
  int parity = 0;
  int64_t base = (int64_t)blockIdx.x * kRowsPerBlock;
  load_row(base + row_in_block, h, g);
  for (; base < a.rows; base += step, parity ^= 1) {
    const int64_t row = base + row_in_block;
    u32x4 hn[CH], gn[CH];
    load_row(row + step, hn, gn);

    // v = bf16(hidden * bf16(silu(gate))), kept packed in h
    u16x2 m = {0, 0};
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const uint32_t hw[4] = {h[j].x, h[j].y, h[j].z, h[j].w}, gw[4] = {g[j].x, g[j].y, g[j].z, g[j].w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a0 = silu(Half2<XGEN_DTYPE_BF16>::lo(gw[i])), a1 = silu(Half2<XGEN_DTYPE_BF16>::hi(gw[i]));
        round_bf16x2(a0, a1);
        o[i] = pack_bf16x2(Half2<XGEN_DTYPE_BF16>::lo(hw[i]) * a0, Half2<XGEN_DTYPE_BF16>::hi(hw[i]) * a1);
      }
      h[j] = u32x4{o[0], o[1], o[2], o[3]};
      // chunks past the row's end hold bf16(0 * silu(0)) = 0: no effect on the max
      m = absmax_chunk<XGEN_DTYPE_BF16>(h[j], m);
    }
    uint32_t amax_bits = wave_max_u32(hmax_u16x2(m));
    if constexpr (WPR > 1) {
      if (lane == 0) red[parity][wave] = amax_bits;
      __syncthreads();
      const int w0 = row_in_block * WPR;
#pragma unroll
      for (int i = 0; i < WPR; ++i) amax_bits = max_u32(amax_bits, red[parity][w0 + i]);
    }
    if (row < a.rows) {
      const float amax = Half2<XGEN_DTYPE_BF16>::from_absbits(amax_bits);
      RowQuant p = (OUT == XGEN_DTYPE_E4M3) ? fp8_row_params(amax) : i8_row_params(amax);
      if (OUT == XGEN_DTYPE_I8 && a.scale_mode == 0) p.s = canonical_nan(1.0f / p.mul);
      uint8_t *qr = a.q + row * (int64_t)a.half;
      uint8_t *ar = a.act ? a.act + row * (int64_t)a.half * 2 : nullptr;
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int ci = lane_in_row + j * 64 * WPR;
        if (ci < nchunks) {
          float v[8];
          unpack8<XGEN_DTYPE_BF16>(h[j], v);
          *reinterpret_cast<u32x2 *>(qr + (int64_t)ci * 8) = quant8<OUT>(v, p);
          if (ar) *reinterpret_cast<u32x4 *>(ar + (int64_t)ci * 16) = h[j];
        }
      }
      if (lane_in_row == 0) a.scale[row] = p.s;
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      h[j] = hn[j];
      g[j] = gn[j];
    }
  }
}

template <int OUT, int WPR, int CH>
void launch(const SwigluArgs &a, hipStream_t stream) {
  constexpr int kRowsPerBlock = 4 / WPR;
  static const int per_cu = resident_blocks_per_cu(swiglu_quant_kernel<OUT, WPR, CH>, kThreads);
  const int64_t need = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  swiglu_quant_kernel<OUT, WPR, CH><<<dim3((unsigned)(need < cap ? need : cap)), dim3(kThreads), 0, stream>>>(a);
}

// --- table variant -------------------------------------------------------------
// A bf16 gate g has 65,536 bit patterns, so a = bf16(silu(g)) is a table of
// 128 KB, computed once by silu_table_kernel with the code above (the same
// values by construction).  The table variant copies it into LDS (one 16-wave
// workgroup per CU) and looks a up per element: the exp and the division leave
// the per-element work, which is then a product, two roundings and the
// quantizer.
constexpr int kLutThreads = 1024;
constexpr int kLutEntries = 65536;

__global__ __launch_bounds__(256) void silu_table_kernel(uint16_t *table) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= kLutEntries) return;
  float a0 = silu(__uint_as_float((uint32_t)i << 16)), a1 = 0.0f;
  round_bf16x2(a0, a1);
  table[i] = (uint16_t)(__float_as_uint(a0) >> 16);
}

// NT: u is read non-temporally (calls larger than the last-level cache).
template <int OUT, int WPR, int CH, bool NT>
__global__ __launch_bounds__(kLutThreads) void swiglu_quant_lut_kernel(SwigluArgs a, const uint16_t *table) {
  constexpr int kWaves = kLutThreads / 64;
  constexpr int kRowsPerBlock = kWaves / WPR;
  __shared__ __attribute__((aligned(16))) uint16_t lut[kLutEntries];
  __shared__ uint32_t red[2][kWaves];
  for (int i = threadIdx.x; i < kLutEntries / 8; i += kLutThreads)
    reinterpret_cast<u32x4 *>(lut)[i] = reinterpret_cast<const u32x4 *>(table)[i];
  __syncthreads();

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row_in_block = wave / WPR;
  const int lane_in_row = (wave % WPR) * 64 + lane;
  const int nchunks = a.half >> 3;
  const int64_t step = (int64_t)gridDim.x * kRowsPerBlock;
  const int hoff = a.gate_first ? a.half * 2 : 0, goff = a.gate_first ? 0 : a.half * 2;  // bytes

  auto load16 = [](const uint8_t *ptr) {
    const u32x4 *v = reinterpret_cast<const u32x4 *>(ptr);
    if constexpr (NT) return __builtin_nontemporal_load(v);
    else return *v;
  };
  auto load_row = [&](int64_t row, u32x4 (&h)[CH], u32x4 (&g)[CH]) {
    const bool ok = row < a.rows;
    const int64_t r = ok ? row : 0;
    const uint8_t *ur = a.u + (r / a.seq) * a.sb + (r % a.seq) * a.sr;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int ci = lane_in_row + j * 64 * WPR;
      const bool in = ok && ci < nchunks;
      h[j] = in ? load16(ur + hoff + (int64_t)ci * 16) : u32x4{0, 0, 0, 0};
      g[j] = in ? load16(ur + goff + (int64_t)ci * 16) : u32x4{0, 0, 0, 0};
    }
  };

  u32x4 h[CH], g[CH];
  int parity = 0;
  int64_t base = (int64_t)blockIdx.x * kRowsPerBlock;
  load_row(base + row_in_block, h, g);
  for (; base < a.rows; base += step, parity ^= 1) {
    const int64_t row = base + row_in_block;
    u32x4 hn[CH], gn[CH];
    load_row(row + step, hn, gn);

    // v = bf16(hidden * a), a = table[gate bits], kept packed in h
    u16x2 m = {0, 0};
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const uint32_t hw[4] = {h[j].x, h[j].y, h[j].z, h[j].w}, gw[4] = {g[j].x, g[j].y, g[j].z, g[j].w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a0 = __uint_as_float((uint32_t)lut[gw[i] & 0xffffu] << 16);
        const float a1 = __uint_as_float((uint32_t)lut[gw[i] >> 16] << 16);
        o[i] = pack_bf16x2(Half2<XGEN_DTYPE_BF16>::lo(hw[i]) * a0, Half2<XGEN_DTYPE_BF16>::hi(hw[i]) * a1);
      }
      h[j] = u32x4{o[0], o[1], o[2], o[3]};
      // chunks past the row's end hold bf16(0 * table[0]) = 0: no effect on the max
      m = absmax_chunk<XGEN_DTYPE_BF16>(h[j], m);
    }
    uint32_t amax_bits = wave_max_u32(hmax_u16x2(m));
    if constexpr (WPR > 1) {
      if (lane == 0) red[parity][wave] = amax_bits;
      __syncthreads();
      const int w0 = row_in_block * WPR;
#pragma unroll
      for (int i = 0; i < WPR; ++i) amax_bits = max_u32(amax_bits, red[parity][w0 + i]);
    }
    if (row < a.rows) {
      const float amax = Half2<XGEN_DTYPE_BF16>::from_absbits(amax_bits);
      RowQuant p = (OUT == XGEN_DTYPE_E4M3) ? fp8_row_params(amax) : i8_row_params(amax);
      if (OUT == XGEN_DTYPE_I8 && a.scale_mode == 0) p.s = canonical_nan(1.0f / p.mul);
      uint8_t *qr = a.q + row * (int64_t)a.half;
      uint8_t *ar = a.act ? a.act + row * (int64_t)a.half * 2 : nullptr;
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int ci = lane_in_row + j * 64 * WPR;
        if (ci < nchunks) {
          float v[8];
          unpack8<XGEN_DTYPE_BF16>(h[j], v);
          *reinterpret_cast<u32x2 *>(qr + (int64_t)ci * 8) = quant8<OUT>(v, p);
          if (ar) *reinterpret_cast<u32x4 *>(ar + (int64_t)ci * 16) = h[j];
        }
      }
      if (lane_in_row == 0) a.scale[row] = p.s;
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      h[j] = hn[j];
      g[j] = gn[j];
    }
  }
}

template <int OUT, int WPR, int CH>
void launch_lut(const SwigluArgs &a, const uint16_t *table, hipStream_t stream) {
  constexpr int kRowsPerBlock = kLutThreads / 64 / WPR;
  const int64_t need = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const int64_t cap = device_cu_count();  // the 128 KB table: one workgroup per CU
  const dim3 grid((unsigned)(need < cap ? need : cap)), block(kLutThreads);
  if (a.rows * (int64_t)a.half * 5 > kLastLevelCacheBytes)  // 4 bytes read + 1 written per output
    swiglu_quant_lut_kernel<OUT, WPR, CH, true><<<grid, block, 0, stream>>>(a, table);
  else
    swiglu_quant_lut_kernel<OUT, WPR, CH, false><<<grid, block, 0, stream>>>(a, table);
}

// At most 4 chunks of 8 per lane (16 waves of a workgroup share the registers of a CU).
template <int OUT>
void dispatch_lut(const SwigluArgs &a, const uint16_t *table, hipStream_t stream) {
  const int f = a.half;
  if (f <= 2048) launch_lut<OUT, 1, 4>(a, table, stream);
  else if (f <= 4096) launch_lut<OUT, 2, 4>(a, table, stream);
  else if (f <= 8192) launch_lut<OUT, 4, 4>(a, table, stream);
  else launch_lut<OUT, 8, 4>(a, table, stream);
}

template <int OUT>
void dispatch(const SwigluArgs &a, hipStream_t stream) {
  const int f = a.half;
  if (f <= 1024) launch<OUT, 1, 2>(a, stream);
  else if (f <= 2048) launch<OUT, 1, 4>(a, stream);
  else if (f <= 3072) launch<OUT, 2, 3>(a, stream);
  else if (f <= 4096) launch<OUT, 2, 4>(a, stream);
  else if (f <= 6144) launch<OUT, 4, 3>(a, stream);
  else if (f <= 8192) launch<OUT, 4, 4>(a, stream);
  else if (f <= 12288) launch<OUT, 4, 6>(a, stream);
  else if (f <= 14336) launch<OUT, 4, 7>(a, stream);  // H3's FFN: F = 14,336
  else launch<OUT, 4, 8>(a, stream);
}

}  // namespace

}  // namespace xgen

using namespace xgen;

namespace {

int swiglu_entry(const char *fn, const void *u, int64_t batch, int64_t seq, int64_t half_width,
                 int64_t u_stride_batch, int64_t u_stride_seq, int gate_first, int out_dtype, int scale_mode,
                 void *q, float *scale, void *act_out, const void *silu_table, hipStream_t stream) {
  if (!is_quant_dtype(out_dtype)) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: output dtype must be E4M3 or I8", fn);
  if (scale_mode != 0 && scale_mode != 1) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: scale mode must be 0 or 1", fn);
  if (gate_first != 0 && gate_first != 1) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: gate_first must be 0 or 1", fn);
  if (batch < 0 || seq < 0 || half_width <= 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad shape batch=%lld seq=%lld F=%lld", fn, (long long)batch,
                (long long)seq, (long long)half_width);
  if (half_width > XGEN_SWIGLU_MAX_HALF)
    return fail(XGEN_ERR_UNSUPPORTED, "%s: F=%lld exceeds %d", fn, (long long)half_width, XGEN_SWIGLU_MAX_HALF);
  if (u_stride_seq < 2 * half_width || u_stride_batch < 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: row stride must be >= 2F", fn);
  const int64_t rows = batch * seq;
  if (rows == 0) return ok();
  if (!u || !q || !scale) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (half_width % 8 || u_stride_seq % 8 || u_stride_batch % 8 || !aligned16(u) ||
      (reinterpret_cast<uintptr_t>(q) & 7u) || (act_out && !aligned16(act_out)))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: F and strides must be multiples of 8 elements, u and act_out 16-byte "
                "and q 8-byte aligned", fn);
  SwigluArgs a;
  a.u = static_cast<const uint8_t *>(u);
  a.sb = u_stride_batch * 2;
  a.sr = u_stride_seq * 2;
  a.seq = seq;
  a.rows = rows;
  a.half = (int)half_width;
  a.gate_first = gate_first;
  a.scale_mode = scale_mode;
  a.q = static_cast<uint8_t *>(q);
  a.scale = scale;
  a.act = static_cast<uint8_t *>(act_out);
  if (silu_table) {
    if (!aligned16(silu_table)) return fail(XGEN_ERR_UNSUPPORTED, "%s: silu table must be 16-byte aligned", fn);
    const uint16_t *t = static_cast<const uint16_t *>(silu_table);
    if (out_dtype == XGEN_DTYPE_E4M3) dispatch_lut<XGEN_DTYPE_E4M3>(a, t, stream);
    else dispatch_lut<XGEN_DTYPE_I8>(a, t, stream);
  } else {
    if (out_dtype == XGEN_DTYPE_E4M3) dispatch<XGEN_DTYPE_E4M3>(a, stream);
    else dispatch<XGEN_DTYPE_I8>(a, stream);
  }
  return launch_status(fn);
}

}  // namespace

extern "C" int xgen_swiglu_quant(const void *u, int64_t batch, int64_t seq, int64_t half_width,
                                 int64_t u_stride_batch, int64_t u_stride_seq, int gate_first, int out_dtype,
                                 int scale_mode, void *q, float *scale, void *act_out, hipStream_t stream) {
  return swiglu_entry("xgen_swiglu_quant", u, batch, seq, half_width, u_stride_batch, u_stride_seq, gate_first,
                      out_dtype, scale_mode, q, scale, act_out, nullptr, stream);
}

extern "C" int xgen_silu_bf16_table(void *table, hipStream_t stream) {
  const char *fn = "xgen_silu_bf16_table";
  if (!table) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (!aligned16(table)) return fail(XGEN_ERR_UNSUPPORTED, "%s: table must be 16-byte aligned", fn);
  silu_table_kernel<<<dim3(kLutEntries / 256), dim3(256), 0, stream>>>(static_cast<uint16_t *>(table));
  return launch_status(fn);
}

extern "C" int xgen_swiglu_quant_lut(const void *u, int64_t batch, int64_t seq, int64_t half_width,
                                     int64_t u_stride_batch, int64_t u_stride_seq, int gate_first, int out_dtype,
                                     int scale_mode, void *q, float *scale, void *act_out, const void *silu_table,
                                     hipStream_t stream) {
  if (!silu_table) return fail(XGEN_ERR_INVALID_ARGUMENT, "xgen_swiglu_quant_lut: null silu table");
  return swiglu_entry("xgen_swiglu_quant_lut", u, batch, seq, half_width, u_stride_batch, u_stride_seq,
                      gate_first, out_dtype, scale_mode, q, scale, act_out, silu_table, stream);
}
