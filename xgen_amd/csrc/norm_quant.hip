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
// Layout: one wave per row up to width 3072, two or four beyond (at most 6
// chunks of 8 per lane).  The row stays in registers from the single HBM read
// to the single quantized write; the row sums and max |m| are wave reductions
// (plus an LDS exchange when a row spans several waves).  The two table rows
// come from L2 (the table is small).
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
  const void *weight;  // per-column weight of dtype WT (kernel template), or null
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

// a.lo * b.lo + a.hi * b.hi + c on two packed bf16 pairs (v_dot2c_f32_bf16);
// used only for the row statistics, whose rounding is not bit-specified.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                         false);
}
constexpr uint32_t kBf16OnePair = 0x3f803f80u;

// The one-pass variance E[x^2] - mean^2 loses at most one bit to cancellation
// while mean^2 <= E[x^2] / 2; other rows (including constant rows, and NaN or
// infinite statistics) take the two-pass variance sum((x - mean)^2) / width.
__device__ __forceinline__ bool needs_two_pass(float mean, float ex2) { return !(mean * mean <= 0.5f * ex2); }

// Rows spread over WPR > 1 waves reduce across waves through LDS with one
// barrier per reduction: each reduction of a row step has its own slots, and
// the slots alternate between even and odd steps, so a wave writes a slot again
// two steps later, after a barrier of the step in between that no wave passes
// before it has read the slot.
struct RedSlots {
  float mom[8];    // per wave: sum, then sum of squares
  float var[4];    // per wave: two-pass sum of squares / RMS sum of squares
  uint32_t amax[4];
};

template <int WPR>
__device__ __forceinline__ float row_sum(float v, int wave, int lane, float *red) {
  v = wave_sum_f32(v);
  if constexpr (WPR > 1) {
    if (lane == 0) red[wave] = v;
    __syncthreads();
    const int w0 = (wave / WPR) * WPR;
    v = red[w0];
#pragma unroll
    for (int i = 1; i < WPR; ++i) v += red[w0 + i];
  }
  return v;
}

// Sum and sum of squares of a row, reduced together.  two_pass_here: this row
// needs the two-pass variance; two_pass_any: some row of the workgroup does
// (the same value in every wave, so the second reduction's barrier stays in
// step; each row still uses only its own statistics).
struct RowMoments {
  float s1, s2;
  bool two_pass_here, two_pass_any;
};

template <int WPR>
__device__ __forceinline__ RowMoments row_moments(float s1, float s2, int wave, int lane, float *red,
                                                  float inv_w) {
  s1 = wave_sum_f32(s1);
  s2 = wave_sum_f32(s2);
  RowMoments m;
  if constexpr (WPR == 1) {
    m.s1 = s1, m.s2 = s2;
    m.two_pass_here = m.two_pass_any = needs_two_pass(s1 * inv_w, s2 * inv_w);
  } else {
    if (lane == 0) red[wave] = s1, red[4 + wave] = s2;
    __syncthreads();
    m.two_pass_any = false;
#pragma unroll
    for (int r = 0; r < 4 / WPR; ++r) {
      float t1 = red[r * WPR], t2 = red[4 + r * WPR];
#pragma unroll
      for (int i = 1; i < WPR; ++i) t1 += red[r * WPR + i], t2 += red[4 + r * WPR + i];
      const bool need = needs_two_pass(t1 * inv_w, t2 * inv_w);
      m.two_pass_any |= need;
      if (r == wave / WPR) m.s1 = t1, m.s2 = t2, m.two_pass_here = need;
    }
  }
  return m;
}

template <int WPR>
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v, int wave, int lane, uint32_t *red) {
  v = wave_max_u32(v);
  if constexpr (WPR > 1) {
    if (lane == 0) red[wave] = v;
    __syncthreads();
    const int w0 = (wave / WPR) * WPR;
    v = red[w0];
#pragma unroll
    for (int i = 1; i < WPR; ++i) v = v > red[w0 + i] ? v : red[w0 + i];
  }
  return v;
}

// The 8 weights of one chunk (WT = BF16 or F32) as fp32, read through the
// weight row's buffer resource (zeros past the row's end).
template <int WT>
struct Weight8 {
  static constexpr int kWords = WT == XGEN_DTYPE_F32 ? 8 : 4;
  uint32_t w[kWords];
  // off: byte offset of the chunk's bf16 elements (kOutOfRange past the end)
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (WT == XGEN_DTYPE_F32) {
      const uint32_t o = off == kOutOfRange ? kOutOfRange : off * 2u;
      const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0);
      const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r, o == kOutOfRange ? o : o + 16u, 0, 0);
      w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
    } else if constexpr (WT == XGEN_DTYPE_BF16) {
      const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
      w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w;
    }
  }
  __device__ __forceinline__ float get(int i) const {
    if constexpr (WT == XGEN_DTYPE_F32) return __uint_as_float(w[i]);
    else return (i & 1) ? Half2<XGEN_DTYPE_BF16>::hi(w[i >> 1]) : Half2<XGEN_DTYPE_BF16>::lo(w[i >> 1]);
  }
};

// Streaming: a grid of as many workgroups as are resident walks the rows
// (4 / WPR rows per workgroup per step; the walk is uniform over the
// workgroup, so the cross-wave reductions stay in step).  Software pipeline
// per wave: at the top of a step it issues the next row's table index and x
// read; once the current row's modulation has consumed its table rows it
// issues the next row's table reads into the same registers; so every read
// has about one step of work to hide behind (the weight is read once).
// gfx9 counts loads and stores with one in-order counter, so the loop's memory
// accesses are unconditional and the same on every path: rows go through
// buffer resources (chunks past a row's end load zeros, their stores are
// dropped), rows past the end redo the last row (writing the same bytes as its
// owner), a row whose index is outside the table reads table row 0 and selects
// its poisoned output, and the first row is peeled so that the loop is entered
// as it is repeated; the compiler's wait counts then name exactly the loads a
// step needs.
// NORM: XGEN_NORM_LAYER or XGEN_NORM_RMS, plus XGEN_NORM_SCALE_ONE_PLUS when
// the scale table already holds bf16(1 + scale).  WT: weight dtype (NONE,
// BF16, F32).  NORMED: also store the pre-quantization rows.
template <int NORM, int OUT, int WT, int WPR, int CH, bool NORMED>
__device__ __forceinline__ void norm_rows(const NormArgs &a, RedSlots (&red)[2]) {
  constexpr bool kOnePlus = (NORM & XGEN_NORM_SCALE_ONE_PLUS) != 0;
  constexpr int kNorm = NORM & ~XGEN_NORM_SCALE_ONE_PLUS;
  constexpr int kRowsPerBlock = 4 / WPR;
  // the wave index as a wave-uniform value: row indices and addresses are
  // then computed by the scalar unit
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int lane_in_row = (wave % WPR) * 64 + lane;
  const int64_t step = (int64_t)gridDim.x * kRowsPerBlock;
  const float inv_w = 1.0f / (float)a.width;
  const int row_bytes = a.width * 2;
  const bool full = a.width == 512 * WPR * CH;  // no chunk past the row's end
  auto chunk_ok = [&](int j) { return lane_in_row + j * 64 * WPR < (a.width >> 3); };
  // byte offset of chunk j of this lane in a bf16 row (kOutOfRange past the end)
  auto in_off = [&](int j) -> uint32_t {
    return chunk_ok(j) ? (uint32_t)(lane_in_row + j * 64 * WPR) * 16u : kOutOfRange;
  };
  auto rsrc = [](const void *base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, bytes, kBufferFlags);
  };
  auto clamp_row = [&](int64_t row) -> uint32_t { return (uint32_t)(row < a.rows ? row : a.rows - 1); };
  // row r = b * seq + s: x row address and the token's index position s
  auto x_row = [&](uint32_t r, uint32_t &s) {
    const uint32_t b = fast_div(r, a.seq);
    s = r - b * a.seq.d;
    return a.x + (int64_t)b * a.xsb_bytes + (int64_t)s * a.xss_bytes;
  };
  // table indices through the constant address space: a scalar load (the
  // index is wave-uniform), waited for only where the table rows are read
  const __attribute__((address_space(4))) int64_t *indices =
      (const __attribute__((address_space(4))) int64_t *)a.indices;
  auto load_x = [&](const uint8_t *xr, u32x4 (&c)[CH]) {
    const __amdgpu_buffer_rsrc_t r = rsrc(xr, row_bytes);
#pragma unroll
    for (int j = 0; j < CH; ++j) c[j] = __builtin_amdgcn_raw_buffer_load_b128(r, in_off(j), 0, 0);
  };
  const __amdgpu_buffer_rsrc_t rw =
      rsrc(a.weight, WT == XGEN_DTYPE_NONE ? 0 : a.width * (WT == XGEN_DTYPE_F32 ? 4 : 2));
  // the weight is the same for every row: read once, kept in registers
  Weight8<WT> wt[CH];
  if constexpr (WT != XGEN_DTYPE_NONE) {
#pragma unroll
    for (int j = 0; j < CH; ++j) wt[j].load(rw, in_off(j));
  }
  // table rows of index g (row 0 stands in for an index outside the table)
  u32x4 scw[CH], shw[CH];
  auto load_tables = [&](int64_t g) {
    const int64_t gt = (g >= 0 && g < a.table_rows) ? g : 0;
    const __amdgpu_buffer_rsrc_t rs = rsrc(a.scale_tab + gt * a.scale_stride_bytes, row_bytes);
    const __amdgpu_buffer_rsrc_t rt = rsrc(a.shift_tab + gt * a.shift_stride_bytes, row_bytes);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      scw[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, in_off(j), 0, 0);
      shw[j] = __builtin_amdgcn_raw_buffer_load_b128(rt, in_off(j), 0, 0);
    }
  };

  u32x4 c[CH], cn[CH];
  int64_t g;
  int parity = 0;  // LDS reduction slots of this step
  // one row (base: the workgroup's first row of this step) from x chunks c, loading the next
  // row's into cn (the loop alternates the two buffers: no register copies between rows)
  auto row_step = [&](int64_t base, u32x4 (&c)[CH], u32x4 (&cn)[CH]) {
    const uint32_t row = clamp_row(base + wave / WPR);
    const bool g_ok = g >= 0 && g < a.table_rows;  // uniform over the wave (one row per wave)

    // the next row's index, then its x
    __builtin_amdgcn_sched_barrier(0);
    uint32_t sn;
    const uint8_t *xn = x_row(clamp_row(base + step + wave / WPR), sn);
    const int64_t gn = indices[sn];
    load_x(xn, cn);
    __builtin_amdgcn_sched_barrier(0);

    // statistics in fp32 (chunks past the row's end are zeros)
    float rstd, mean = 0.0f;
    bool two_pass = false;
    if constexpr (kNorm == XGEN_NORM_LAYER) {
      float s1[2] = {0.0f, 0.0f}, s2[2] = {0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const uint32_t w[4] = {c[j].x, c[j].y, c[j].z, c[j].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          s1[k & 1] = dot2_bf16(kBf16OnePair, w[k], s1[k & 1]);
          s2[k & 1] = dot2_bf16(w[k], w[k], s2[k & 1]);
        }
      }
      const RowMoments mo = row_moments<WPR>(s1[0] + s1[1], s2[0] + s2[1], wave, lane, red[parity].mom, inv_w);
      // sum / width: the product with 1 / width plus one FMA correction, exact
      // whenever the quotient is representable (a constant row's mean is its value)
      const float mean0 = mo.s1 * inv_w;
      mean = __builtin_fmaf(__builtin_fmaf(-mean0, (float)a.width, mo.s1), inv_w, mean0);
      float var = __builtin_fmaxf(mo.s2 * inv_w - mean * mean, 0.0f);
      if (mo.two_pass_any) {  // uniform over the workgroup
        float acc2 = 0.0f;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
          if (chunk_ok(j)) {
            float xv[8];
            unpack8<XGEN_DTYPE_BF16>(c[j], xv);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float d = xv[i] - mean;
              acc2 = __builtin_fmaf(d, d, acc2);
            }
          }
        }
        const float var2 = row_sum<WPR>(acc2, wave, lane, red[parity].var) * inv_w;
        if (mo.two_pass_here) var = var2;
      }
      two_pass = mo.two_pass_here;
      rstd = __builtin_amdgcn_rsqf(var + a.eps);
    } else {
      float s2[2] = {0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const uint32_t w[4] = {c[j].x, c[j].y, c[j].z, c[j].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) s2[k & 1] = dot2_bf16(w[k], w[k], s2[k & 1]);
      }
      const float ms = row_sum<WPR>(s2[0] + s2[1], wave, lane, red[parity].var) * inv_w;
      rstd = __builtin_amdgcn_rsqf(ms + a.eps);
    }
    const float neg_mean_rstd = -mean * rstd;

    // normalise and modulate with the table row: m as fp32 values of bf16
    // precision (each bf16 rounding is one v_cvt_pk_bf16_f32 whose other half
    // is zero, so its word is the rounded value's fp32 bits).  LayerNorm rows
    // with an ordinary variance take n = fma(x, rstd, -mean * rstd); rows that
    // took the two-pass variance (a large common offset, constant rows) keep
    // the eager (x - mean) * rstd, whose subtraction is exact there.
    float m[CH][8];
    auto modulate = [&](auto exact_tag) {
      constexpr bool kExact = decltype(exact_tag)::value;
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        // opaque copies: each of the two instances unpacks its own inputs (no
        // common code is hoisted above the branch, where it would stay live)
        u32x4 xj = c[j], sj = scw[j], tj = shw[j];
        asm volatile("" : "+v"(xj), "+v"(sj), "+v"(tj));
        const uint32_t xw[4] = {xj.x, xj.y, xj.z, xj.w};
        const uint32_t scp[4] = {sj.x, sj.y, sj.z, sj.w};
        const uint32_t shp[4] = {tj.x, tj.y, tj.z, tj.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int i = k >> 1;
          auto half = [&](uint32_t w) {
            return (k & 1) ? Half2<XGEN_DTYPE_BF16>::hi(w) : Half2<XGEN_DTYPE_BF16>::lo(w);
          };
          const float x = half(xw[i]);
          float n;
          if constexpr (kNorm == XGEN_NORM_RMS) n = x * rstd;
          else if constexpr (kExact) n = (x - mean) * rstd;
          else n = __builtin_fmaf(x, rstd, neg_mean_rstd);
          if constexpr (WT != XGEN_DTYPE_NONE) n *= wt[j].get(k);
          n = round_bf16(n);
          float f = half(scp[i]);
          if constexpr (!kOnePlus) f = round_bf16(1.0f + f);
          const float pr = round_bf16(n * f);
          float mv = round_bf16(pr + half(shp[i]));
          asm volatile("" : "+v"(mv));  // the rounding stays in this instance (not sunk past the merge)
          m[j][k] = mv;
        }
      }
    };
    if (kNorm == XGEN_NORM_LAYER && two_pass) modulate(std::true_type{});
    else modulate(std::false_type{});
    if (!full) {  // uniform: chunks past the row's end are zeros again (they stay out of the row max)
#pragma unroll
      for (int j = 0; j < CH; ++j)
#pragma unroll
        for (int k = 0; k < 8; ++k) m[j][k] = chunk_ok(j) ? m[j][k] : 0.0f;
    }
    // max |m| (NaN-propagating: v_maximum3_f32), as the bits of a float >= +0 or a NaN
    float am = 0.0f;
#pragma unroll
    for (int j = 0; j < CH; ++j)
#pragma unroll
      for (int k = 0; k < 8; ++k) am = __builtin_elementwise_maximum(am, __builtin_fabsf(m[j][k]));
    // the table rows are consumed: the next row's go into the same registers
    __builtin_amdgcn_sched_barrier(0);
    load_tables(gn);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t amax_bits = row_max_u32<WPR>(__float_as_uint(am) & 0x7fffffffu, wave, lane, red[parity].amax);

    // quantize from registers; a row whose index is outside the table is
    // poisoned: its amax is taken as NaN, so the scale is NaN and the row
    // quantizer's non-finite path writes NaN bytes (E4M3) or zeros (I8); its
    // normed row is zeros
    const float amax = g_ok ? __uint_as_float(amax_bits) : __builtin_nanf("");
    const RowQuant p = (OUT == XGEN_DTYPE_E4M3) ? fp8_row_params(amax) : i8_row_params(amax);
    const __amdgpu_buffer_rsrc_t rq = rsrc(a.q + (int64_t)row * a.width, a.width);
    const __amdgpu_buffer_rsrc_t rn = rsrc(NORMED ? a.normed + (int64_t)row * row_bytes : a.q, NORMED ? row_bytes : 0);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const u32x2 qb = quant8<OUT>(m[j], p);
      // a chunk past the end: its offset stays past the row's bytes, the stores are dropped
      __builtin_amdgcn_raw_buffer_store_b64(qb, rq, in_off(j) >> 1, 0, 0);
      if constexpr (NORMED) {
        uint32_t pk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)  // the high halves of two fp32 words of bf16 precision
          pk[i] = __builtin_amdgcn_perm(__float_as_uint(m[j][2 * i + 1]), __float_as_uint(m[j][2 * i]), 0x07060302u);
        __builtin_amdgcn_raw_buffer_store_b128(g_ok ? u32x4{pk[0], pk[1], pk[2], pk[3]} : u32x4{0, 0, 0, 0}, rn,
                                               in_off(j), 0, 0);
      }
    }
    a.token_scale[row] = p.s;  // every lane of the row: the same value
    g = gn;
    parity ^= 1;
  };

  int64_t base = (int64_t)blockIdx.x * kRowsPerBlock;
  uint32_t s0;
  const uint8_t *x0 = x_row(clamp_row(base + wave / WPR), s0);
  g = indices[s0];
  load_x(x0, c);
  __builtin_amdgcn_sched_barrier(0);
  load_tables(g);
  if (base >= a.rows) return;
  row_step(base, c, cn);  // peeled: the loop is then entered with the pending accesses of a step
  for (base += step; base < a.rows; base += 2 * step) {
    row_step(base, cn, c);
    if (base + step >= a.rows) break;
    row_step(base + step, c, cn);
  }
}

template <int NORM, int OUT, int WT, int WPR, int CH>
__global__ __launch_bounds__(kThreads) void norm_affine_quant_kernel(NormArgs a) {
  __shared__ RedSlots red[2];
  if (a.normed) norm_rows<NORM, OUT, WT, WPR, CH, true>(a, red);
  else norm_rows<NORM, OUT, WT, WPR, CH, false>(a, red);
}

template <int NORM, int OUT, int WT, int WPR, int CH>
void launch(const NormArgs &a, hipStream_t stream) {
  constexpr int kRowsPerBlock = 4 / WPR;
  static const int per_cu = resident_blocks_per_cu(norm_affine_quant_kernel<NORM, OUT, WT, WPR, CH>, kThreads);
  const int64_t need = (a.rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  norm_affine_quant_kernel<NORM, OUT, WT, WPR, CH>
      <<<dim3((unsigned)(need < cap ? need : cap)), dim3(kThreads), 0, stream>>>(a);
}

// Waves per row and chunks per lane by width: up to 3072 one wave per row (no
// barriers; at most 6 chunks = 48 values per lane), wider rows two or four
// waves with one LDS exchange per reduction (measured at d = 5,376: four waves
// of 3 chunks beat two of 6 by 4%).
template <int NORM, int OUT, int WT>
void dispatch_width(const NormArgs &a, hipStream_t stream) {
  const int w = a.width;
  if (w <= 1024) launch<NORM, OUT, WT, 1, 2>(a, stream);
  else if (w <= 2048) launch<NORM, OUT, WT, 1, 4>(a, stream);
  else if (w <= 3072) launch<NORM, OUT, WT, 1, 6>(a, stream);
  else if (w <= 4096) launch<NORM, OUT, WT, 2, 4>(a, stream);
  else if (w <= 6144) launch<NORM, OUT, WT, 4, 3>(a, stream);
  else launch<NORM, OUT, WT, 4, 4>(a, stream);
}

template <int NORM, int OUT>
void dispatch_weight(const NormArgs &a, int weight_dtype, hipStream_t stream) {
  if (weight_dtype == XGEN_DTYPE_BF16) dispatch_width<NORM, OUT, XGEN_DTYPE_BF16>(a, stream);
  else if (weight_dtype == XGEN_DTYPE_F32) dispatch_width<NORM, OUT, XGEN_DTYPE_F32>(a, stream);
  else dispatch_width<NORM, OUT, XGEN_DTYPE_NONE>(a, stream);
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
      if (e4m3) dispatch_weight<XGEN_NORM_LAYER, XGEN_DTYPE_E4M3>(a, norm_weight_dtype, stream);
      else dispatch_weight<XGEN_NORM_LAYER, XGEN_DTYPE_I8>(a, norm_weight_dtype, stream);
      break;
    case XGEN_NORM_RMS:
      if (e4m3) dispatch_weight<XGEN_NORM_RMS, XGEN_DTYPE_E4M3>(a, norm_weight_dtype, stream);
      else dispatch_weight<XGEN_NORM_RMS, XGEN_DTYPE_I8>(a, norm_weight_dtype, stream);
      break;
    case XGEN_NORM_LAYER | kP:
      if (e4m3) dispatch_weight<XGEN_NORM_LAYER | kP, XGEN_DTYPE_E4M3>(a, norm_weight_dtype, stream);
      else dispatch_weight<XGEN_NORM_LAYER | kP, XGEN_DTYPE_I8>(a, norm_weight_dtype, stream);
      break;
    default:
      if (e4m3) dispatch_weight<XGEN_NORM_RMS | kP, XGEN_DTYPE_E4M3>(a, norm_weight_dtype, stream);
      else dispatch_weight<XGEN_NORM_RMS | kP, XGEN_DTYPE_I8>(a, norm_weight_dtype, stream);
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
