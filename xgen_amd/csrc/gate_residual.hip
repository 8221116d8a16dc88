// Gated residual with an indexed gate table (gfx950):
//
//   out[b, s, :] = bf16(residual[b, s, :] + bf16(branch[b, s, :] * gate[indices[s], :]))
//
// multiply, round, add, round — no fused multiply-add, as
// x_base/x_base/operator/npu_fusion/f2a/op_kernel/gate_residual_kernel.asc:57-67 and the eager
// form of x_base/x_base/operator/h3_indexed_affine.py:49 compute it.  Replaces
// torch.ops.h3_phaa_gate_residual.gate_residual (f2a/op_extension/gate_residual_queued.asc:33-35).
//
// The same file holds the other half of the reference's indexed affine
// (x_base/x_base/operator/h3_indexed_affine.py:9-48, `_apply(..., modulation=True)`): the
// AdaLN modulation of already normalised rows,
//
//   out[b, s, :] = bf16(bf16(x[b, s, :] * bf16(1 + scale[indices[s], :])) + shift[indices[s], :])
//
// (scale[g] itself when the table holds the prepared bf16(1 + scale)).
//
// Layout: a streaming grid of waves walks the rows; the lanes of a wave cover
// a row in 16-byte chunks (8 values); the row's table index is read once per
// row.  An index outside the table writes a NaN row (the reference asserts
// and abandons the rest of its block).
#include "xgen_common.h"

namespace xgen {

namespace {

constexpr int kThreads = 256;

struct GateArgs {
  const uint8_t *res;
  int64_t rsb, rss;  // bytes
  const uint8_t *br;
  int64_t bsb, bss;  // bytes
  const uint8_t *gate;
  int64_t gstride;  // bytes
  int64_t gate_rows;
  const int64_t *indices;
  int64_t rows, seq;
  int chunks;  // 16-byte chunks per row
  uint8_t *out;
};

__global__ __launch_bounds__(kThreads) void gate_residual_kernel(GateArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * (kThreads / 64);
  for (int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); row < a.rows; row += waves) {
    const int64_t b = row / a.seq, s = row % a.seq;
    const int64_t g = a.indices[s];
    const bool g_ok = g >= 0 && g < a.gate_rows;
    const uint8_t *rr = a.res + b * a.rsb + s * a.rss;
    const uint8_t *yr = a.br + b * a.bsb + s * a.bss;
    const uint8_t *tr = a.gate + (g_ok ? g : 0) * a.gstride;
    uint8_t *orow = a.out + row * (int64_t)a.chunks * 16;
    for (int c = lane; c < a.chunks; c += 64) {
      u32x4 o;
      if (g_ok) {
        o = gate_residual8(*reinterpret_cast<const u32x4 *>(rr + (int64_t)c * 16),
                           *reinterpret_cast<const u32x4 *>(yr + (int64_t)c * 16),
                           *reinterpret_cast<const u32x4 *>(tr + (int64_t)c * 16));
      } else {
        o = u32x4{0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
      }
      *reinterpret_cast<u32x4 *>(orow + (int64_t)c * 16) = o;
    }
  }
}

struct ModArgs {
  const uint8_t *x;
  int64_t xsb, xss;  // bytes
  const uint8_t *scale, *shift;
  int64_t sstride, tstride;  // bytes
  int64_t table_rows;
  const int64_t *indices;
  int64_t rows, seq;
  int chunks;  // 16-byte chunks per row
  uint8_t *out;
};

// One 16-byte chunk: bf16(bf16(x * f) + shift), f = bf16(1 + scale) (or scale when prepared).
template <bool ONE_PLUS>
__device__ __forceinline__ u32x4 modulate8(const u32x4 &x, const u32x4 &sc, const u32x4 &sh) {
  const uint32_t xw[4] = {x.x, x.y, x.z, x.w}, cw[4] = {sc.x, sc.y, sc.z, sc.w}, hw[4] = {sh.x, sh.y, sh.z, sh.w};
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float f0 = __uint_as_float(cw[i] << 16), f1 = __uint_as_float(cw[i] & 0xffff0000u);
    if constexpr (!ONE_PLUS) {
      f0 += 1.0f, f1 += 1.0f;
      round_bf16x2(f0, f1);
    }
    float p0 = __uint_as_float(xw[i] << 16) * f0, p1 = __uint_as_float(xw[i] & 0xffff0000u) * f1;
    round_bf16x2(p0, p1);
    o[i] = pack_bf16x2(p0 + __uint_as_float(hw[i] << 16), p1 + __uint_as_float(hw[i] & 0xffff0000u));
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

template <bool ONE_PLUS>
__global__ __launch_bounds__(kThreads) void indexed_modulate_kernel(ModArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = (int64_t)gridDim.x * (kThreads / 64);
  for (int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6); row < a.rows; row += waves) {
    const int64_t b = row / a.seq, s = row % a.seq;
    const int64_t g = a.indices[s];
    const bool g_ok = g >= 0 && g < a.table_rows;
    const uint8_t *xr = a.x + b * a.xsb + s * a.xss;
    const uint8_t *fr = a.scale + (g_ok ? g : 0) * a.sstride;
    const uint8_t *hr = a.shift + (g_ok ? g : 0) * a.tstride;
    uint8_t *orow = a.out + row * (int64_t)a.chunks * 16;
    for (int c = lane; c < a.chunks; c += 64) {
      u32x4 o;
      if (g_ok) {
        o = modulate8<ONE_PLUS>(*reinterpret_cast<const u32x4 *>(xr + (int64_t)c * 16),
                                *reinterpret_cast<const u32x4 *>(fr + (int64_t)c * 16),
                                *reinterpret_cast<const u32x4 *>(hr + (int64_t)c * 16));
      } else {
        o = u32x4{0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
      }
      *reinterpret_cast<u32x4 *>(orow + (int64_t)c * 16) = o;
    }
  }
}

}  // namespace

}  // namespace xgen

using namespace xgen;

extern "C" int xgen_gate_residual(const void *residual, int64_t res_stride_batch, int64_t res_stride_seq,
                                  const void *branch, int64_t br_stride_batch, int64_t br_stride_seq,
                                  const void *gate_table, int64_t gate_row_stride, int64_t gate_rows,
                                  const int64_t *indices, int64_t batch, int64_t seq, int64_t width, void *out,
                                  hipStream_t stream) {
  const char *fn = "xgen_gate_residual";
  if (batch < 0 || seq < 0 || width <= 0 || gate_rows <= 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad shape batch=%lld seq=%lld width=%lld gate_rows=%lld", fn,
                (long long)batch, (long long)seq, (long long)width, (long long)gate_rows);
  if (res_stride_seq < width || br_stride_seq < width || gate_row_stride < width || res_stride_batch < 0 ||
      br_stride_batch < 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: row strides must be >= width and batch strides >= 0", fn);
  const int64_t rows = batch * seq;
  if (rows == 0) return ok();
  if (!residual || !branch || !gate_table || !indices || !out)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (width % 8 || res_stride_seq % 8 || res_stride_batch % 8 || br_stride_seq % 8 || br_stride_batch % 8 ||
      gate_row_stride % 8 || !aligned16(residual) || !aligned16(branch) || !aligned16(gate_table) || !aligned16(out))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: width and strides must be multiples of 8 elements and buffers "
                "16-byte aligned", fn);
  if (width / 8 > 0x7fffffffLL) return fail(XGEN_ERR_UNSUPPORTED, "%s: row too wide", fn);
  GateArgs a;
  a.res = static_cast<const uint8_t *>(residual);
  a.rsb = res_stride_batch * 2;
  a.rss = res_stride_seq * 2;
  a.br = static_cast<const uint8_t *>(branch);
  a.bsb = br_stride_batch * 2;
  a.bss = br_stride_seq * 2;
  a.gate = static_cast<const uint8_t *>(gate_table);
  a.gstride = gate_row_stride * 2;
  a.gate_rows = gate_rows;
  a.indices = indices;
  a.rows = rows;
  a.seq = seq;
  a.chunks = (int)(width / 8);
  a.out = static_cast<uint8_t *>(out);
  static const int per_cu = resident_blocks_per_cu(gate_residual_kernel, kThreads);
  const int64_t need = (rows + 3) / 4;
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  gate_residual_kernel<<<dim3((unsigned)(need < cap ? need : cap)), dim3(kThreads), 0, stream>>>(a);
  return launch_status(fn);
}

extern "C" int xgen_indexed_modulate(const void *x, int64_t x_stride_batch, int64_t x_stride_seq,
                                     const void *scale_table, int64_t scale_row_stride, const void *shift_table,
                                     int64_t shift_row_stride, int64_t table_rows, const int64_t *indices,
                                     int64_t batch, int64_t seq, int64_t width, int scale_is_one_plus, void *out,
                                     hipStream_t stream) {
  const char *fn = "xgen_indexed_modulate";
  if (batch < 0 || seq < 0 || width <= 0 || table_rows <= 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad shape batch=%lld seq=%lld width=%lld table_rows=%lld", fn,
                (long long)batch, (long long)seq, (long long)width, (long long)table_rows);
  if (x_stride_seq < width || scale_row_stride < width || shift_row_stride < width || x_stride_batch < 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: row strides must be >= width and batch strides >= 0", fn);
  const int64_t rows = batch * seq;
  if (rows == 0) return ok();
  if (!x || !scale_table || !shift_table || !indices || !out)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (width % 8 || x_stride_seq % 8 || x_stride_batch % 8 || scale_row_stride % 8 || shift_row_stride % 8 ||
      !aligned16(x) || !aligned16(scale_table) || !aligned16(shift_table) || !aligned16(out))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: width and strides must be multiples of 8 elements and buffers "
                "16-byte aligned", fn);
  if (width / 8 > 0x7fffffffLL) return fail(XGEN_ERR_UNSUPPORTED, "%s: row too wide", fn);
  ModArgs a;
  a.x = static_cast<const uint8_t *>(x);
  a.xsb = x_stride_batch * 2;
  a.xss = x_stride_seq * 2;
  a.scale = static_cast<const uint8_t *>(scale_table);
  a.shift = static_cast<const uint8_t *>(shift_table);
  a.sstride = scale_row_stride * 2;
  a.tstride = shift_row_stride * 2;
  a.table_rows = table_rows;
  a.indices = indices;
  a.rows = rows;
  a.seq = seq;
  a.chunks = (int)(width / 8);
  a.out = static_cast<uint8_t *>(out);
  const int64_t need = (rows + 3) / 4;
  if (scale_is_one_plus) {
    static const int per_cu = resident_blocks_per_cu(indexed_modulate_kernel<true>, kThreads);
    const int64_t cap = (int64_t)device_cu_count() * per_cu;
    indexed_modulate_kernel<true><<<dim3((unsigned)(need < cap ? need : cap)), dim3(kThreads), 0, stream>>>(a);
  } else {
    static const int per_cu = resident_blocks_per_cu(indexed_modulate_kernel<false>, kThreads);
    const int64_t cap = (int64_t)device_cu_count() * per_cu;
    indexed_modulate_kernel<false><<<dim3((unsigned)(need < cap ? need : cap)), dim3(kThreads), 0, stream>>>(a);
  }
  return launch_status(fn);
}
