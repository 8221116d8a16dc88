// BF16 layouts of the head-parallel attention's exchange (gfx950): pure byte moves, no arithmetic.
//
// Replaces torch.ops.h3_phaa_layout.{pack, back, merge}
// (x_base/x_base/operator/npu_fusion/f4/op_extension/layout_queued.asc:27-55, kernels
// f4/op_kernel/layout_kernel.asc:33-59; wrapper npu_fusion/phaa_layout.py:13-28):
//
//  * pack  — Q/K/V [1, S, heads, D] (heads contiguous, any row stride) into the all-to-all's send
//            buffers [chunks, owners, S, 1, heads_per_chunk, D]: owner d's chunk c holds heads
//            d * (chunks * heads_per_chunk) + c * heads_per_chunk + i;
//  * back  — the attention output [1, heads, L, D] (any head / position strides) into the return
//            buffer [owners * S, heads * D]: row s holds every head of position s, rows L.. are
//            zero (the padding tokens);
//  * merge — the returned chunks [chunks, owners, S, batch, heads_per_chunk * D] into the
//            out-projection's input [batch, S, owners * chunks * heads_per_chunk * D]
//            (owner-major, chunk-minor columns; the layout xgen_merge_quant quantizes).
//
// One kernel serves all three: the output is written in order as 16-byte units; a unit belongs
// to a run (contiguous in the output, made of `nsub` sub-runs of `sub_units` units that are each
// contiguous in the source); the run index is a mixed-radix number (i0 fastest, i3 slowest)
// whose digits select the source position through byte strides.  Runs from `valid_runs` on are
// written as zeros.  Divisions by the launch's radices are multiply-highs (FastDiv).  Each
// thread moves four units per step (loads first, then stores); blockIdx.y picks the tensor.
// NT: the source is read non-temporally (calls larger than the last-level cache).
#include "fastdiv.h"
#include "xgen_common.h"

namespace xgen {

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

struct LayoutArgs {
  const uint8_t *src[3];
  uint8_t *dst[3];
  int64_t stride[4];   // source bytes per digit i0..i3 of the run index
  int64_t sub_stride;  // source bytes between the sub-runs of a run
  FastDiv sub_units, nsub, n0, n1, n2;
  uint32_t units;       // 16-byte output units per tensor (< 2^31)
  uint32_t valid_runs;  // runs at or past it are zero
};

__device__ __forceinline__ int64_t source_offset(const LayoutArgs &a, uint32_t u, bool &live) {
  const uint32_t sr = fast_div(u, a.sub_units), k = u - sr * a.sub_units.d;  // sub-run, unit in it
  const uint32_t r = fast_div(sr, a.nsub), j = sr - r * a.nsub.d;            // run, sub-run in it
  live = r < a.valid_runs;
  const uint32_t q0 = fast_div(r, a.n0), i0 = r - q0 * a.n0.d;
  const uint32_t q1 = fast_div(q0, a.n1), i1 = q0 - q1 * a.n1.d;
  const uint32_t i3 = fast_div(q1, a.n2), i2 = q1 - i3 * a.n2.d;
  return (int64_t)i0 * a.stride[0] + (int64_t)i1 * a.stride[1] + (int64_t)i2 * a.stride[2] +
         (int64_t)i3 * a.stride[3] + (int64_t)j * a.sub_stride + (int64_t)k * 16;
}

template <bool NT>
__global__ __launch_bounds__(kThreads) void layout_copy_kernel(LayoutArgs a) {
  const uint8_t *src = a.src[blockIdx.y];
  uint8_t *dst = a.dst[blockIdx.y];
  const uint32_t step = gridDim.x * kThreads;
  for (uint32_t u0 = blockIdx.x * kThreads + threadIdx.x; u0 < a.units; u0 += step * kUnroll) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int i = 0; i < kUnroll; ++i) {
      const uint32_t u = u0 + i * step;  // < 2^31 + 2^31: no wrap in 32 bits
      bool live = false;
      const int64_t off = u < a.units ? source_offset(a, u, live) : 0;
      const u32x4 *p = reinterpret_cast<const u32x4 *>(src + off);
      if constexpr (NT) v[i] = (u < a.units && live) ? __builtin_nontemporal_load(p) : u32x4{0u, 0u, 0u, 0u};
      else v[i] = (u < a.units && live) ? *p : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < kUnroll; ++i) {
      const uint32_t u = u0 + i * step;
      if (u < a.units) *reinterpret_cast<u32x4 *>(dst + (int64_t)u * 16) = v[i];
    }
  }
}

template <bool NT>
void launch_layout_policy(LayoutArgs &a, int tensors, hipStream_t stream) {
  static const int per_cu = resident_blocks_per_cu(layout_copy_kernel<NT>, kThreads);
  const int64_t cap = (int64_t)device_cu_count() * per_cu / tensors + 1;
  const int64_t need = ((int64_t)a.units + kThreads * kUnroll - 1) / (kThreads * kUnroll);
  const int64_t blocks = need < cap ? need : cap;
  layout_copy_kernel<NT><<<dim3((unsigned)blocks, (unsigned)tensors), dim3(kThreads), 0, stream>>>(a);
}

// A call moving more than the last-level cache holds (read + written) reads non-temporally.
int launch_layout(const char *fn, LayoutArgs &a, int tensors, hipStream_t stream) {
  if ((int64_t)a.units * 16 * 2 * tensors > kLastLevelCacheBytes) launch_layout_policy<true>(a, tensors, stream);
  else launch_layout_policy<false>(a, tensors, stream);
  return launch_status(fn);
}

bool fits_units(int64_t bytes) { return bytes / 16 < 0x7fffffffLL; }

}  // namespace

}  // namespace xgen

using namespace xgen;

extern "C" int xgen_phaa_pack_qkv(const void *q, const void *k, const void *v, int64_t seq, int64_t owners,
                                  int64_t chunks, int64_t heads_per_chunk, int64_t head_dim, int64_t q_row_stride,
                                  int64_t k_row_stride, int64_t v_row_stride, void *q_send, void *k_send,
                                  void *v_send, hipStream_t stream) {
  const char *fn = "xgen_phaa_pack_qkv";
  if (seq < 0 || owners < 1 || chunks < 1 || heads_per_chunk < 1 || head_dim < 1)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad geometry seq=%lld owners=%lld chunks=%lld heads_per_chunk=%lld "
                "head_dim=%lld", fn, (long long)seq, (long long)owners, (long long)chunks, (long long)heads_per_chunk,
                (long long)head_dim);
  const int64_t heads = owners * chunks * heads_per_chunk, run_bytes = heads_per_chunk * head_dim * 2;
  const int64_t strides[3] = {q_row_stride, k_row_stride, v_row_stride};
  for (int64_t st : strides)
    if (st < heads * head_dim)
      return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: row stride %lld below heads * head_dim = %lld", fn, (long long)st,
                  (long long)(heads * head_dim));
  if (seq == 0) return ok();
  const void *srcs[3] = {q, k, v};
  void *dsts[3] = {q_send, k_send, v_send};
  for (int z = 0; z < 3; ++z) {
    if (!srcs[z] || !dsts[z]) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    if (!aligned16(srcs[z]) || !aligned16(dsts[z]) || strides[z] % 8)
      return fail(XGEN_ERR_UNSUPPORTED, "%s: buffers must be 16-byte aligned and row strides multiples of 8", fn);
  }
  if (run_bytes % 16) return fail(XGEN_ERR_UNSUPPORTED, "%s: heads_per_chunk * head_dim must be a multiple of 8", fn);
  if (seq > 0x7fffffffLL || !fits_units(seq * heads * head_dim * 2))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: a tensor of %lld x %lld values exceeds 2^31 16-byte units", fn,
                (long long)seq, (long long)(heads * head_dim));
  LayoutArgs a;
  for (int z = 0; z < 3; ++z) a.src[z] = static_cast<const uint8_t *>(srcs[z]), a.dst[z] = static_cast<uint8_t *>(dsts[z]);
  // output [chunks, owners, seq] runs of one chunk's heads: i0 = s, i1 = owner, i2 = chunk
  a.sub_units = make_fastdiv((uint32_t)(run_bytes / 16));
  a.nsub = make_fastdiv(1);
  a.n0 = make_fastdiv((uint32_t)seq);
  a.n1 = make_fastdiv((uint32_t)owners);
  a.n2 = make_fastdiv((uint32_t)chunks);
  a.sub_stride = 0;
  a.units = (uint32_t)(seq * heads * head_dim * 2 / 16);
  a.valid_runs = 0xffffffffu;
  a.stride[1] = chunks * run_bytes;
  a.stride[2] = run_bytes;
  a.stride[3] = 0;
  // the three tensors may differ in row stride: one launch each when they do
  if (q_row_stride == k_row_stride && q_row_stride == v_row_stride) {
    a.stride[0] = q_row_stride * 2;
    return launch_layout(fn, a, 3, stream);
  }
  for (int z = 0; z < 3; ++z) {
    LayoutArgs one = a;
    one.src[0] = a.src[z], one.dst[0] = a.dst[z];
    one.stride[0] = strides[z] * 2;
    const int st = launch_layout(fn, one, 1, stream);
    if (st != XGEN_OK) return st;
  }
  return XGEN_OK;
}

extern "C" int xgen_phaa_pack_back(const void *attn, int64_t heads, int64_t length, int64_t head_dim,
                                   int64_t head_stride, int64_t position_stride, int64_t rows, void *back_send,
                                   hipStream_t stream) {
  const char *fn = "xgen_phaa_pack_back";
  if (heads < 1 || head_dim < 1 || length < 0 || rows < length || head_stride < 0 || position_stride < 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad geometry heads=%lld length=%lld head_dim=%lld rows=%lld", fn,
                (long long)heads, (long long)length, (long long)head_dim, (long long)rows);
  if (rows == 0) return ok();
  if (!back_send || (length > 0 && !attn)) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if ((head_dim * 2) % 16 || head_stride % 8 || position_stride % 8 || (attn && !aligned16(attn)) ||
      !aligned16(back_send))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: head_dim and strides must be multiples of 8 and buffers 16-byte aligned",
                fn);
  if (rows > 0x7fffffffLL || !fits_units(rows * heads * head_dim * 2))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: %lld rows of %lld values exceed 2^31 16-byte units", fn, (long long)rows,
                (long long)(heads * head_dim));
  LayoutArgs a;
  a.src[0] = static_cast<const uint8_t *>(attn);
  a.dst[0] = static_cast<uint8_t *>(back_send);
  // output rows of every head of one position: run = position (i0), sub-run = head
  a.sub_units = make_fastdiv((uint32_t)(head_dim * 2 / 16));
  a.nsub = make_fastdiv((uint32_t)heads);
  a.n0 = make_fastdiv((uint32_t)rows);
  a.n1 = make_fastdiv(1);
  a.n2 = make_fastdiv(1);
  a.stride[0] = position_stride * 2;
  a.stride[1] = a.stride[2] = a.stride[3] = 0;
  a.sub_stride = head_stride * 2;
  a.units = (uint32_t)(rows * heads * head_dim * 2 / 16);
  a.valid_runs = (uint32_t)length;
  return launch_layout(fn, a, 1, stream);
}

extern "C" int xgen_phaa_merge_back(const void *back_recv, int64_t chunks, int64_t owners, int64_t seq,
                                    int64_t batch, int64_t chunk, void *merged, hipStream_t stream) {
  const char *fn = "xgen_phaa_merge_back";
  if (chunks < 1 || owners < 1 || chunk < 1 || seq < 0 || batch < 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad geometry chunks=%lld owners=%lld seq=%lld batch=%lld chunk=%lld",
                fn, (long long)chunks, (long long)owners, (long long)seq, (long long)batch, (long long)chunk);
  if (chunks > 0x7fffffffLL || owners > 0x7fffffffLL || seq > 0x7fffffffLL || batch > 0x7fffffffLL ||
      chunk > 0x7fffffffLL || (seq && batch > 0x7fffffffLL / seq))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: geometry exceeds 2^31 - 1", fn);
  const int64_t rows = seq * batch;
  if (rows == 0) return ok();
  if (!back_recv || !merged) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (chunk % 8 || !aligned16(back_recv) || !aligned16(merged))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: chunk must be a multiple of 8 and buffers 16-byte aligned", fn);
  if (chunks * owners > 0x7fffffffLL / chunk || !fits_units(rows * chunks * owners * chunk * 2))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: %lld rows of %lld values exceed 2^31 16-byte units", fn, (long long)rows,
                (long long)(chunks * owners * chunk));
  LayoutArgs a;
  a.src[0] = static_cast<const uint8_t *>(back_recv);
  a.dst[0] = static_cast<uint8_t *>(merged);
  // output [batch, seq, owners, chunks] runs of one chunk: i0 = chunk c, i1 = owner, i2 = s, i3 = b
  const int64_t cb = chunk * 2;
  a.sub_units = make_fastdiv((uint32_t)(cb / 16));
  a.nsub = make_fastdiv(1);
  a.n0 = make_fastdiv((uint32_t)chunks);
  a.n1 = make_fastdiv((uint32_t)owners);
  a.n2 = make_fastdiv((uint32_t)seq);
  a.stride[0] = owners * seq * batch * cb;
  a.stride[1] = seq * batch * cb;
  a.stride[2] = batch * cb;
  a.stride[3] = cb;
  a.sub_stride = 0;
  a.units = (uint32_t)(rows * chunks * owners * cb / 16);
  a.valid_runs = 0xffffffffu;
  return launch_layout(fn, a, 1, stream);
}
