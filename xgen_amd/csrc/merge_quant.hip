// Merge of the head-parallel attention's returned chunks + per-row quantization (gfx950).
//
// The out-projection's input arrives from the all-to-all as
// back_recv [splits, owners, seq, batch, chunk] (bf16, contiguous): the
// attention output of chunk c of owner o's heads.  A token's row of the
// out-projection's input is owner-major, chunk-minor:
//
//   row (b, s) = b * seq + s,  column (o * splits + c) * chunk + j  <-  back_recv[c, o, s, b, j]
//
// and the row is quantized per token as the path's other row quantizers do
// (INT8: npu_dynamic_quant as restated in f2bc_kernel.asc:89-107, scale mode 1;
// FP8 e4m3fn: h3_fp8.py:9-12 per row).  Replaces
// torch.ops.h3_phaa_merge_quant.fused (x_base/x_base/operator/npu_fusion/
// f4_merge_quant/op_extension/merge_quant_queued.asc:9-28, its kernel
// op_kernel/merge_quant_kernel.asc:20-87 at splits 7, owners 4, batch 1,
// chunk 256).
//
// Layout: one workgroup per row (a grid-stride loop over rows); thread t holds
// the row's 16-byte chunks t, t + 256, ...  Where each chunk comes from does
// not depend on the row, so a thread's source offsets are formed once; a row
// adds its (s, b) position.  A wave's 64 chunks are two 512-byte runs of one
// segment at chunk = 256: coalesced.  The row's max |x| is an integer max of
// the bf16 magnitudes (NaN-propagating), reduced across the wave with lane
// shuffles and across the four waves through LDS; the bytes are written from
// registers.  NT: the input is read non-temporally (calls larger than the
// last-level cache).
#include "xgen_common.h"

namespace xgen {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxChunksPerThread = 8;  // rows up to 256 * 8 * 8 = 16,384 values

struct MergeArgs {
  const uint8_t *x;
  int64_t seg_bytes;  // between consecutive (c, o) segments: seq * batch * chunk * 2
  int64_t pos_bytes;  // between consecutive (s, b) positions: chunk * 2
  uint32_t rows, seq, batch;
  int splits, owners, chunks_per_seg, nchunks;
  uint8_t *q;
  float *scale;
};

template <int OUT, int CH, bool NT>
__global__ __launch_bounds__(kThreads) void merge_quant_kernel(MergeArgs a) {
  __shared__ uint32_t red[2][kThreads / 64];  // cross-wave max, double-buffered by row parity
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t off[CH];
  bool live[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int ci = threadIdx.x + j * kThreads;  // chunk of the output row
    live[j] = ci < a.nchunks;
    const int t = ci / a.chunks_per_seg, w = ci - t * a.chunks_per_seg;
    const int o = t / a.splits, c = t - o * a.splits;
    off[j] = live[j] ? (int64_t)(c * a.owners + o) * a.seg_bytes + (int64_t)w * 16 : 0;
  }
  int parity = 0;
  for (uint32_t row = blockIdx.x; row < a.rows; row += gridDim.x, parity ^= 1) {
    const uint32_t b = row / a.seq, s = row - b * a.seq;
    const uint8_t *base = a.x + ((int64_t)s * a.batch + b) * a.pos_bytes;
    u32x4 v[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const u32x4 *src = reinterpret_cast<const u32x4 *>(base + off[j]);
      if constexpr (NT) v[j] = live[j] ? __builtin_nontemporal_load(src) : u32x4{0u, 0u, 0u, 0u};
      else v[j] = live[j] ? *src : u32x4{0u, 0u, 0u, 0u};
    }
    u16x2 m = {0, 0};
#pragma unroll
    for (int j = 0; j < CH; ++j) m = absmax_chunk<XGEN_DTYPE_BF16>(v[j], m);
    uint32_t amax_bits = wave_max_u32(hmax_u16x2(m));
    if (lane == 0) red[parity][wave] = amax_bits;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kThreads / 64; ++i) amax_bits = amax_bits > red[parity][i] ? amax_bits : red[parity][i];
    const float amax = Half2<XGEN_DTYPE_BF16>::from_absbits(amax_bits);
    const RowQuant p = OUT == XGEN_DTYPE_E4M3 ? fp8_row_params(amax) : i8_row_params(amax);
    uint8_t *qr = a.q + (int64_t)row * a.nchunks * 8;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (live[j]) {
        float f[8];
        unpack8<XGEN_DTYPE_BF16>(v[j], f);
        *reinterpret_cast<u32x2 *>(qr + (int64_t)(threadIdx.x + j * kThreads) * 8) = quant8<OUT>(f, p);
      }
    }
    if (threadIdx.x == 0) a.scale[row] = p.s;
  }
}

template <int OUT, int CH, bool NT>
void launch_merge_policy(const MergeArgs &a, hipStream_t stream) {
  static const int per_cu = resident_blocks_per_cu(merge_quant_kernel<OUT, CH, NT>, kThreads);
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  const int64_t blocks = (int64_t)a.rows < cap ? (int64_t)a.rows : cap;
  merge_quant_kernel<OUT, CH, NT><<<dim3((unsigned)blocks), dim3(kThreads), 0, stream>>>(a);
}

template <int OUT, int CH>
void launch_merge(const MergeArgs &a, hipStream_t stream) {
  // 2 bytes read + 1 written per value: a call beyond the last-level cache reads its input
  // non-temporally (H3 at S = 15,624, 336 MB: 55.2 against 64.1 us with ordinary loads)
  if ((int64_t)a.rows * a.nchunks * 8 * 3 > kLastLevelCacheBytes) launch_merge_policy<OUT, CH, true>(a, stream);
  else launch_merge_policy<OUT, CH, false>(a, stream);
}

template <int OUT>
void launch_merge_out(const MergeArgs &a, hipStream_t stream) {
  if (a.nchunks <= kThreads) launch_merge<OUT, 1>(a, stream);
  else if (a.nchunks <= 2 * kThreads) launch_merge<OUT, 2>(a, stream);
  else if (a.nchunks <= 4 * kThreads) launch_merge<OUT, 4>(a, stream);
  else launch_merge<OUT, 8>(a, stream);
}

}  // namespace

}  // namespace xgen

using namespace xgen;

extern "C" int xgen_merge_quant(int out_dtype, const void *back_recv, int64_t splits, int64_t owners, int64_t seq,
                                int64_t batch, int64_t chunk, void *q, float *scale, hipStream_t stream) {
  const char *fn = "xgen_merge_quant";
  if (!is_quant_dtype(out_dtype))
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: output dtype %d is not e4m3fn or int8", fn, out_dtype);
  if (splits < 1 || owners < 1 || chunk < 1 || seq < 0 || batch < 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad geometry splits=%lld owners=%lld seq=%lld batch=%lld chunk=%lld",
                fn, (long long)splits, (long long)owners, (long long)seq, (long long)batch, (long long)chunk);
  if (chunk % 8)
    return fail(XGEN_ERR_UNSUPPORTED, "%s: chunk must be a multiple of 8 values (got %lld)", fn, (long long)chunk);
  const int64_t max_width = (int64_t)kThreads * kMaxChunksPerThread * 8;
  if (splits > max_width || owners > max_width || chunk > max_width || splits * owners * chunk > max_width)
    return fail(XGEN_ERR_UNSUPPORTED, "%s: row width splits*owners*chunk exceeds %lld", fn, (long long)max_width);
  if (seq > 0x7fffffffLL || batch > 0x7fffffffLL || (seq && batch > 0x7fffffffLL / seq))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: seq*batch exceeds 2^31 - 1 rows", fn);
  const int64_t rows = seq * batch;
  if (rows == 0) return ok();
  if (!back_recv || !q || !scale) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (!aligned16(back_recv) || (reinterpret_cast<uintptr_t>(q) & 7u) || (reinterpret_cast<uintptr_t>(scale) & 3u))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: back_recv must be 16-byte, q 8-byte and scale 4-byte aligned", fn);
  MergeArgs a;
  a.x = static_cast<const uint8_t *>(back_recv);
  a.seg_bytes = seq * batch * chunk * 2;
  a.pos_bytes = chunk * 2;
  a.rows = (uint32_t)rows;
  a.seq = (uint32_t)seq;
  a.batch = (uint32_t)batch;
  a.splits = (int)splits;
  a.owners = (int)owners;
  a.chunks_per_seg = (int)(chunk / 8);
  a.nchunks = (int)(splits * owners * chunk / 8);
  a.q = static_cast<uint8_t *>(q);
  a.scale = scale;
  if (out_dtype == XGEN_DTYPE_E4M3) launch_merge_out<XGEN_DTYPE_E4M3>(a, stream);
  else launch_merge_out<XGEN_DTYPE_I8>(a, stream);
  return launch_status(fn);
}
