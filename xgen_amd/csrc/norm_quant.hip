// Fused normalisation + AdaLN-table modulation + per-row quantization (gfx950).
//
// Replaces torch.ops.h3_phaa_nq2.fused (npu_fusion/f2_nq2/op_extension/nq2_queued.asc:53-61,
// kernel npu_fusion/f2bc/op_kernel/f2bc_kernel.asc:57-107) and, with LayerNorm,
// the eager front end of x_diffusers/x_diffusers/framework/transformer/hunyuan.py:390-393:
//
//   n = bf16(norm(x) [* weight]);  f = bf16(1 + scale[g]);
//   m = bf16(bf16(n * f) + shift[g]);  (q, s) = quantize_row(m)
//
// with every intermediate rounded to bf16 as the eager bf16 ops round it
// (x_base/x_base/operator/h3_indexed_affine.py:22-28).
//
// Layout: one to four waves per row (at most 4 chunks of 8 per lane).  The row
// stays in registers from the single HBM read to the single quantized write;
// mean / variance / max |m| are wave reductions (plus an LDS exchange when a
// row spans two waves).  The two table rows come from L2 (the table is small).
#include "fastdiv.h"
#include "xgen_common.h"

namespace xgen {

namespace {

constexpr int kThreads = 256;

struct NormArgs {
  const uint8_t *x;
  FastDiv seq;       // row r = b * seq + s
  int64_t rows;
  int width;
  int64_t xsb_bytes, xss_bytes;
  const void *weight;
  int weight_dtype;  // XGEN_DTYPE_NONE / BF16 / F32
  float eps;
  const uint8_t *scale_tab;
  int64_t scale_stride_bytes;
  const uint8_t *shift_tab;
  int64_t shift_stride_bytes;
  int64_t table_rows;
  const int64_t *indices;
  uint8_t *q;
  float *token_scale;
  uint8_t *normed;  // optional bf16 [rows, width]
};

template <int WPR>
__device__ __forceinline__ float row_sum(float v, int wave, int lane, float *red) {
  v = wave_sum_f32(v);
  if constexpr (WPR > 1) {
    __syncthreads();  // red[] reuse
    if (lane == 0) red[wave] = v;
    __syncthreads();
    const int w0 = (wave / WPR) * WPR;
    v = red[w0];
#pragma unroll
    for (int i = 1; i < WPR; ++i) v += red[w0 + i];
  }
  return v;
}

template <int WPR>
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v, int wave, int lane, uint32_t *red) {
  v = wave_max_u32(v);
  if constexpr (WPR > 1) {
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    const int w0 = (wave / WPR) * WPR;
    v = red[w0];
#pragma unroll
    for (int i = 1; i < WPR; ++i) v = v > red[w0 + i] ? v : red[w0 + i];
  }
  return v;
}

__device__ __forceinline__ void load_weight8(const void *w, int dtype, int ci, float (&wv)[8]) {
  if (dtype == XGEN_DTYPE_BF16) {
    const u32x4 c = *reinterpret_cast<const u32x4 *>(static_cast<const uint8_t *>(w) + (int64_t)ci * 16);
    unpack8<XGEN_DTYPE_BF16>(c, wv);
  } else {
    const f32x4 *p = reinterpret_cast<const f32x4 *>(static_cast<const uint8_t *>(w) + (int64_t)ci * 32);
    const f32x4 a = p[0], b = p[1];
    wv[0] = a.x; wv[1] = a.y; wv[2] = a.z; wv[3] = a.w;
    wv[4] = b.x; wv[5] = b.y; wv[6] = b.z; wv[7] = b.w;
  }
}

// Streaming: a grid of as many workgroups as are resident walks the rows
// (4 / WPR rows per workgroup per step; the walk is uniform over the
// workgroup, so the cross-wave reductions stay in step); each wave loads its
// next row and table index before it works on the current row.
// FULL: the row is exactly CH chunks per lane (width == 512 * WPR * CH), so
// no chunk needs a bounds check.
// NORM: XGEN_NORM_LAYER or XGEN_NORM_RMS, plus XGEN_NORM_SCALE_ONE_PLUS when
// the scale table already holds bf16(1 + scale).
template <int NORM, int OUT, int WPR, int CH, bool FULL>
__global__ __launch_bounds__(kThreads) void norm_affine_quant_kernel(NormArgs a) {
  constexpr bool kOnePlus = (NORM & XGEN_NORM_SCALE_ONE_PLUS) != 0;
  constexpr int kNorm = NORM & ~XGEN_NORM_SCALE_ONE_PLUS;
  constexpr int kRowsPerBlock = 4 / WPR;
  __shared__ float red_f[4];
  __shared__ uint32_t red_u[4];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int lane_in_row = (wave % WPR) * 64 + lane;
  const int nchunks = a.width >> 3;
  const int64_t step = (int64_t)gridDim.x * kRowsPerBlock;
  auto chunk_ok = [&](int j) { return FULL || lane_in_row + j * 64 * WPR < nchunks; };

  // one read of a row (zeros past the last row) and its table index
  auto load_row = [&](int64_t row, u32x4 (&c)[CH], int64_t &g) {
    const bool ok = row < a.rows;
    const uint32_t r = ok ? (uint32_t)row : 0u;
    const uint32_t b = fast_div(r, a.seq), s = r - b * a.seq.d;
    const uint8_t *xr = a.x + (int64_t)b * a.xsb_bytes + (int64_t)s * a.xss_bytes;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int ci = lane_in_row + j * 64 * WPR;
      c[j] = (ok && chunk_ok(j)) ? *reinterpret_cast<const u32x4 *>(xr + (int64_t)ci * 16) : u32x4{0, 0, 0, 0};
    }
    g = ok ? a.indices[s] : 0;
  };

  u32x4 c[CH];
  int64_t g;
  int64_t base = (int64_t)blockIdx.x * kRowsPerBlock;
  load_row(base + wave / WPR, c, g);
  for (; base < a.rows; base += step) {
    const int64_t row = base + wave / WPR;
    const bool row_ok = row < a.rows;
    u32x4 cn[CH];
    int64_t gn;
    load_row(row + step, cn, gn);
    const bool g_ok = g >= 0 && g < a.table_rows;

    // statistics (fp32, two passes over the packed row; chunks past the row's
    // end are zeros and must stay out of the variance)
    // the row as fp32, unpacked once for the statistics and the normalisation
    float xv[CH][8];
#pragma unroll
    for (int j = 0; j < CH; ++j) unpack8<XGEN_DTYPE_BF16>(c[j], xv[j]);
    float rstd, nmr = 0.0f;  // n = x * rstd + nmr
    if constexpr (kNorm == XGEN_NORM_LAYER) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < CH; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc += xv[j][i];
      const float mean = row_sum<WPR>(acc, wave, lane, red_f) / (float)a.width;
      float acc2 = 0.0f;
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        if (chunk_ok(j)) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float d = xv[j][i] - mean;
            acc2 = __builtin_fmaf(d, d, acc2);
          }
        }
      }
      const float var = row_sum<WPR>(acc2, wave, lane, red_f) / (float)a.width;
      rstd = 1.0f / __builtin_sqrtf(var + a.eps);
      nmr = -mean * rstd;
    } else {
      float acc2 = 0.0f;
#pragma unroll
      for (int j = 0; j < CH; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc2 = __builtin_fmaf(xv[j][i], xv[j][i], acc2);
      const float ms = row_sum<WPR>(acc2, wave, lane, red_f) / (float)a.width;
      rstd = 1.0f / __builtin_sqrtf(ms + a.eps);
    }

    // normalise, modulate with the table row, keep m as packed bf16 (in c);
    // bf16 roundings two at a time (one conversion per pair)
    u16x2 am = {0, 0};
    if (row_ok && g_ok) {  // uniform over the wave (one row per wave)
      const uint8_t *sr = a.scale_tab + g * a.scale_stride_bytes;
      const uint8_t *tr = a.shift_tab + g * a.shift_stride_bytes;
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int ci = lane_in_row + j * 64 * WPR;
        if (chunk_ok(j)) {
          const u32x4 scw = *reinterpret_cast<const u32x4 *>(sr + (int64_t)ci * 16);
          const u32x4 shw = *reinterpret_cast<const u32x4 *>(tr + (int64_t)ci * 16);
          float n[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) n[i] = __builtin_fmaf(xv[j][i], rstd, nmr);
          if (a.weight_dtype != XGEN_DTYPE_NONE) {
            float wv[8];
            load_weight8(a.weight, a.weight_dtype, ci, wv);
#pragma unroll
            for (int i = 0; i < 8; ++i) n[i] *= wv[i];
          }
          const uint32_t scp[4] = {scw.x, scw.y, scw.z, scw.w}, shp[4] = {shw.x, shw.y, shw.z, shw.w};
          uint32_t pk[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float n0 = n[2 * i], n1 = n[2 * i + 1];
            round_bf16x2(n0, n1);
            float f0 = Half2<XGEN_DTYPE_BF16>::lo(scp[i]), f1 = Half2<XGEN_DTYPE_BF16>::hi(scp[i]);
            if constexpr (!kOnePlus) {
              f0 += 1.0f, f1 += 1.0f;
              round_bf16x2(f0, f1);
            }
            float p0 = n0 * f0, p1 = n1 * f1;
            round_bf16x2(p0, p1);
            pk[i] = pack_bf16x2(p0 + Half2<XGEN_DTYPE_BF16>::lo(shp[i]), p1 + Half2<XGEN_DTYPE_BF16>::hi(shp[i]));
          }
          c[j] = u32x4{pk[0], pk[1], pk[2], pk[3]};
          am = absmax_chunk<XGEN_DTYPE_BF16>(c[j], am);
        } else {
          c[j] = u32x4{0, 0, 0, 0};
        }
      }
    }
    const uint32_t amax_bits = row_max_u32<WPR>(hmax_u16x2(am), wave, lane, red_u);

    // quantize from registers
    if (row_ok) {
      uint8_t *qr = a.q + row * (int64_t)a.width;
      const float amax = Half2<XGEN_DTYPE_BF16>::from_absbits(amax_bits);
      const RowQuant p = (OUT == XGEN_DTYPE_E4M3) ? fp8_row_params(amax) : i8_row_params(amax);
      if (g_ok) {
        uint8_t *nr = a.normed ? a.normed + row * (int64_t)a.width * 2 : nullptr;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
          const int ci = lane_in_row + j * 64 * WPR;
          if (chunk_ok(j)) {
            float v[8];
            unpack8<XGEN_DTYPE_BF16>(c[j], v);
            *reinterpret_cast<u32x2 *>(qr + (int64_t)ci * 8) = quant8<OUT>(c[j], v, p);
            if (nr) *reinterpret_cast<u32x4 *>(nr + (int64_t)ci * 16) = c[j];
          }
        }
        if (lane_in_row == 0) a.token_scale[row] = p.s;
      } else {  // index outside the table: a poisoned row (NaN scale; NaN bytes or zeros)
        const u32x2 bad = (OUT == XGEN_DTYPE_E4M3) ? u32x2{0x7f7f7f7fu, 0x7f7f7f7fu} : u32x2{0u, 0u};
        uint8_t *nr = a.normed ? a.normed + row * (int64_t)a.width * 2 : nullptr;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
          const int ci = lane_in_row + j * 64 * WPR;
          if (chunk_ok(j)) {
            *reinterpret_cast<u32x2 *>(qr + (int64_t)ci * 8) = bad;
            if (nr) *reinterpret_cast<u32x4 *>(nr + (int64_t)ci * 16) = u32x4{0, 0, 0, 0};
          }
        }
        if (lane_in_row == 0) a.token_scale[row] = __builtin_nanf("");
      }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) c[j] = cn[j];
    g = gn;
  }
}

template <int NORM, int OUT, int WPR, int CH, bool FULL>
void launch_kernel(const NormArgs &a, hipStream_t stream) {
  constexpr int kRowsPerBlock = 4 / WPR;
  static const int per_cu = resident_blocks_per_cu(norm_affine_quant_kernel<NORM, OUT, WPR, CH, FULL>, kThreads);
  const int64_t need = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  norm_affine_quant_kernel<NORM, OUT, WPR, CH, FULL>
      <<<dim3((unsigned)(need < cap ? need : cap)), dim3(kThreads), 0, stream>>>(a);
}

template <int NORM, int OUT, int WPR, int CH>
void launch(const NormArgs &a, hipStream_t stream) {
  if (a.width == 512 * WPR * CH) launch_kernel<NORM, OUT, WPR, CH, true>(a, stream);
  else launch_kernel<NORM, OUT, WPR, CH, false>(a, stream);
}

// Waves per row and chunks per lane by width: at most 4 chunks (32 values) per
// lane keeps a wave's registers at occupancy >= 3; the row's reductions are
// DPP shuffles plus one LDS exchange between the row's waves.
template <int NORM, int OUT>
void dispatch_width(const NormArgs &a, hipStream_t stream) {
  const int w = a.width;
  if (w <= 1024) launch<NORM, OUT, 1, 2>(a, stream);
  else if (w <= 2048) launch<NORM, OUT, 2, 2>(a, stream);
  else if (w <= 3072) launch<NORM, OUT, 2, 3>(a, stream);
  else if (w <= 4096) launch<NORM, OUT, 2, 4>(a, stream);
  else if (w <= 6144) launch<NORM, OUT, 4, 3>(a, stream);
  else launch<NORM, OUT, 4, 4>(a, stream);
}

}  // namespace

}  // namespace xgen

using namespace xgen;

extern "C" int xgen_norm_affine_quant(const void *x, int64_t batch, int64_t seq, int64_t width,
                                      int64_t x_stride_batch, int64_t x_stride_seq, int norm_kind,
                                      const void *norm_weight, int norm_weight_dtype, float eps,
                                      const void *scale_table, int64_t scale_row_stride,
                                      const void *shift_table, int64_t shift_row_stride,
                                      int64_t table_rows, const int64_t *indices, int out_dtype,
                                      void *q, float *token_scale, void *normed_out,
                                      hipStream_t stream) {
  const char *fn = "xgen_norm_affine_quant";
  const int norm_base = norm_kind & ~XGEN_NORM_SCALE_ONE_PLUS;
  if (norm_base != XGEN_NORM_LAYER && norm_base != XGEN_NORM_RMS)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: unknown norm kind %d", fn, norm_kind);
  if (!is_quant_dtype(out_dtype)) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: output dtype must be E4M3 or I8", fn);
  if (norm_weight_dtype != XGEN_DTYPE_NONE && norm_weight_dtype != XGEN_DTYPE_BF16 &&
      norm_weight_dtype != XGEN_DTYPE_F32)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: norm weight dtype must be NONE, BF16 or F32", fn);
  if ((norm_weight_dtype == XGEN_DTYPE_NONE) != (norm_weight == nullptr))
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: norm weight pointer and dtype disagree", fn);
  if (batch < 0 || seq < 0 || width <= 0 || table_rows <= 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad shape batch=%lld seq=%lld width=%lld tables=%lld", fn,
                (long long)batch, (long long)seq, (long long)width, (long long)table_rows);
  if (!(eps > 0.0f && eps < 1.0f)) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: eps must be in (0, 1)", fn);
  if (width > XGEN_NORM_MAX_WIDTH)
    return fail(XGEN_ERR_UNSUPPORTED, "%s: width %lld exceeds %d", fn, (long long)width, XGEN_NORM_MAX_WIDTH);
  if (x_stride_seq < width || scale_row_stride < width || shift_row_stride < width)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: row strides must be >= width", fn);
  const int64_t rows = batch * seq;
  if (rows == 0) return ok();
  if (!x || !scale_table || !shift_table || !indices || !q || !token_scale)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (width % 8 || x_stride_seq % 8 || x_stride_batch % 8 || scale_row_stride % 8 || shift_row_stride % 8 ||
      !aligned16(x) || !aligned16(scale_table) || !aligned16(shift_table) || !aligned16(q) ||
      (normed_out && !aligned16(normed_out)) || (norm_weight && !aligned16(norm_weight)))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: width and row strides must be multiples of 8 elements and "
                "buffers 16-byte aligned", fn);
  // row indices (plus one grid step of prefetch) stay below 2^31
  if (rows > 0x3fffffffLL) return fail(XGEN_ERR_UNSUPPORTED, "%s: too many rows", fn);

  NormArgs a;
  a.x = static_cast<const uint8_t *>(x);
  a.seq = make_fastdiv((uint32_t)seq);
  a.rows = rows;
  a.width = (int)width;
  a.xsb_bytes = x_stride_batch * 2;
  a.xss_bytes = x_stride_seq * 2;
  a.weight = norm_weight;
  a.weight_dtype = norm_weight_dtype;
  a.eps = eps;
  a.scale_tab = static_cast<const uint8_t *>(scale_table);
  a.scale_stride_bytes = scale_row_stride * 2;
  a.shift_tab = static_cast<const uint8_t *>(shift_table);
  a.shift_stride_bytes = shift_row_stride * 2;
  a.table_rows = table_rows;
  a.indices = indices;
  a.q = static_cast<uint8_t *>(q);
  a.token_scale = token_scale;
  a.normed = static_cast<uint8_t *>(normed_out);
  constexpr int kP = XGEN_NORM_SCALE_ONE_PLUS;
  const bool e4m3 = out_dtype == XGEN_DTYPE_E4M3;
  switch (norm_kind) {
    case XGEN_NORM_LAYER:
      if (e4m3) dispatch_width<XGEN_NORM_LAYER, XGEN_DTYPE_E4M3>(a, stream);
      else dispatch_width<XGEN_NORM_LAYER, XGEN_DTYPE_I8>(a, stream);
      break;
    case XGEN_NORM_RMS:
      if (e4m3) dispatch_width<XGEN_NORM_RMS, XGEN_DTYPE_E4M3>(a, stream);
      else dispatch_width<XGEN_NORM_RMS, XGEN_DTYPE_I8>(a, stream);
      break;
    case XGEN_NORM_LAYER | kP:
      if (e4m3) dispatch_width<XGEN_NORM_LAYER | kP, XGEN_DTYPE_E4M3>(a, stream);
      else dispatch_width<XGEN_NORM_LAYER | kP, XGEN_DTYPE_I8>(a, stream);
      break;
    default:
      if (e4m3) dispatch_width<XGEN_NORM_RMS | kP, XGEN_DTYPE_E4M3>(a, stream);
      else dispatch_width<XGEN_NORM_RMS | kP, XGEN_DTYPE_I8>(a, stream);
      break;
  }
  return launch_status(fn);
}

// out[r, c] = bf16(1 + scale[r, c]): the `1.0 + scale` of the eager modulation
// (x_base/x_base/operator/h3_indexed_affine.py:22-28, hunyuan.py:393), computed once per
// table so the fused front end reads it directly (XGEN_NORM_SCALE_ONE_PLUS).
__global__ __launch_bounds__(256) void adaln_one_plus_kernel(const uint8_t *scale, int64_t s_stride_bytes,
                                                             uint8_t *out, int64_t o_stride_bytes, int64_t rows,
                                                             int chunks) {
  const int64_t total = rows * chunks;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / chunks;
    const int c = (int)(i - r * chunks);
    const u32x4 v = *reinterpret_cast<const u32x4 *>(scale + r * s_stride_bytes + (int64_t)c * 16);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = pack_bf16x2(1.0f + Half2<XGEN_DTYPE_BF16>::lo(w[k]), 1.0f + Half2<XGEN_DTYPE_BF16>::hi(w[k]));
    *reinterpret_cast<u32x4 *>(out + r * o_stride_bytes + (int64_t)c * 16) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

extern "C" int xgen_adaln_one_plus(const void *scale_table, int64_t rows, int64_t width, int64_t scale_row_stride,
                                   void *out, int64_t out_row_stride, hipStream_t stream) {
  const char *fn = "xgen_adaln_one_plus";
  if (rows < 0 || width <= 0 || scale_row_stride < width || out_row_stride < width)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad shape rows=%lld width=%lld (row strides must be >= width)", fn,
                (long long)rows, (long long)width);
  if (rows == 0) return ok();
  if (!scale_table || !out) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (width % 8 || scale_row_stride % 8 || out_row_stride % 8 || !aligned16(scale_table) || !aligned16(out))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: width and row strides must be multiples of 8 elements and buffers "
                "16-byte aligned", fn);
  if (width / 8 > 0x7fffffffLL) return fail(XGEN_ERR_UNSUPPORTED, "%s: row too wide", fn);
  const int chunks = (int)(width / 8);
  const int64_t total = rows * chunks;
  const int64_t blocks = (total + 255) / 256;
  adaln_one_plus_kernel<<<dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, stream>>>(
      static_cast<const uint8_t *>(scale_table), scale_row_stride * 2, static_cast<uint8_t *>(out),
      out_row_stride * 2, rows, chunks);
  return launch_status(fn);
}
