// Per-row FP8 wire codec (gfx950) of the head-parallel attention exchange.
//
// Replaces the encode / decode kernels around the byte all-to-all of
// x_base/x_base/phaa/fp8_transport.py:26-78 (launched at :137-144).  Each row
// of `width` values (one head of one token) travels as `width` e4m3fn bytes
// followed by its float32 scale:
//
//   scale = max(max|v| / 448, 1e-12)               (fp32, IEEE division)
//   byte  = e4m3fn_rne(clamp(v / scale, -448, 448))
//   value = bf16|f16|f32(fl32(e4m3(byte) * scale))  (decode)
//
// Wire layout: rows of width + 4 bytes ordered [peer][stream][peer row], i.e.
// wire row = row + (row / peer_rows * (streams - 1) + slot) * peer_rows for row
// `row` of stream `slot` (fp8_transport.py:53), each peer's block followed by
// `peer_padding` zero bytes (fp8_transport.py:55-63, the 16-byte peer
// alignment option).  Source row `row` of a stream is element
// (peer, seq, batch, head) of a [peers, seq, batch, heads, width] view with
// arbitrary strides (fp8_transport.py:36-48); decoded rows are written
// contiguously, row-major (fp8_transport.py:78).
//
// The asynchronous transport's layouts (fp8_async_transport.py:13-80) are the
// same rows with two more degrees of freedom: the encoder treats rows whose
// global sequence index peer * seq + s is at least `valid_seq` as zero rows
// without reading them (the fused return pack of a ragged attention output,
// RETURN_SEQ, :22-27,41-44), and the strided decoder writes row (peer, s,
// batch, head) at any element strides over those four indices, skipping rows
// past `valid_seq` (the direct gather into [batch, heads, seq, width], :67-73,
// and the return layout into [batch, seq, peers * heads, width], :74-78).
//
// Non-finite inputs (which the reference leaves to its min/max lowering): the
// row max propagates NaN (scale NaN, every byte 0x7f, decoded NaN); an inf
// row max gives scale inf, byte 0x7f for +-inf and signed zero for finite values.
//
// Layout on the chip: a persistent grid walks the wire rows in wire order
// (reads of the wire and writes of the decoded rows stay within one moving
// window of memory).  One group of G lanes (a power of two <= 64) handles a
// row, each lane holding C chunks of E consecutive values (chunk j of lane l
// is chunk l + j*G); each group loads its next row while it reduces and
// stores the current one.  A row's (peer, stream,
// row) comes from two multiply-shift divisions; the stream's source base and
// strides from a table in LDS.  The row max is a DPP / ds_swizzle butterfly
// inside the group.
#include "fastdiv.h"
#include "xgen_common.h"

namespace xgen {

namespace {

constexpr int kThreads = 256;
constexpr float kScaleFloor = 1.0e-12f;

// 4-byte aligned dword pair (wire rows are only dword aligned).
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

template <int DT>
struct Elem {
  static constexpr int kBytes = DT == XGEN_DTYPE_F32 ? 4 : 2;
};

// Max over the G lanes of each aligned lane group (every lane gets its group's max).
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v, int lanes) {
  if (lanes >= 2) v = max_u32(v, dpp_u32<kDppQuad1032>(0, v));
  if (lanes >= 4) v = max_u32(v, dpp_u32<kDppQuad2301>(0, v));
  if (lanes >= 8) v = max_u32(v, dpp_u32<kDppRowHalfMirror>(0, v));
  if (lanes >= 16) v = max_u32(v, dpp_u32<kDppRowMirror>(0, v));
  if (lanes >= 32) v = max_u32(v, (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401F));  // lane ^ 16
  if (lanes >= 64)
    v = max_u32((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 32));
  return v;
}

// Accesses through byte addresses, marked as global memory (global_load /
// global_store rather than flat).
#define XGEN_GLOBAL __attribute__((address_space(1)))
// NT: non-temporal load, for inputs streamed once through a call whose
// footprint exceeds the last-level cache.
template <typename T, bool NT = false>
__device__ __forceinline__ T ld_global(const void *p) {
  if constexpr (NT) return __builtin_nontemporal_load((const XGEN_GLOBAL T *)p);
  else return *(const XGEN_GLOBAL T *)p;
}
template <typename T>
__device__ __forceinline__ void st_global(void *p, const T &v) {
  *(XGEN_GLOBAL T *)p = v;
}
// Dword pairs at addresses that are only 4-byte aligned (wire rows).
__device__ __forceinline__ u32x2 ld_global_a4x2(const void *p) { return *(const XGEN_GLOBAL u32x2_a4 *)p; }
__device__ __forceinline__ void st_global_a4x2(void *p, u32x2 v) { *(XGEN_GLOBAL u32x2_a4 *)p = v; }

// Wire geometry: wire row w -> (peer, stream slot, row within the peer's stream block).
struct WireGeom {
  uint32_t total;      // streams * peers * peer_rows
  FastDiv per_peer;    // streams * peer_rows
  FastDiv peer_rows;
  int64_t row_bytes;   // width + 4
  int64_t pad;         // peer_padding
};

struct RowPos {
  uint32_t peer, slot, pr;
};

__device__ __forceinline__ RowPos locate(const WireGeom &g, uint32_t w) {
  RowPos p;
  p.peer = fast_div(w, g.per_peer);
  const uint32_t within = w - p.peer * g.per_peer.d;
  p.slot = fast_div(within, g.peer_rows);
  p.pr = within - p.slot * g.peer_rows.d;
  return p;
}

// Byte offset of wire row w of peer `peer`.
__device__ __forceinline__ int64_t wire_offset(const WireGeom &g, uint32_t w, uint32_t peer) {
  return (int64_t)w * g.row_bytes + (int64_t)peer * g.pad;
}

// --------------------------------------------------------------------------- encode
struct EncodeArgs {
  const uint8_t *src[3];
  int64_t st[3][4];  // bytes: peer, seq, batch, head
  uint8_t *wire;
  WireGeom g;
  FastDiv heads, batch;
  uint32_t seq;        // sequence positions per peer
  uint32_t valid_seq;  // rows with peer * seq + s >= valid_seq encode as zeros
  int width;
  int log2_lanes;
};

// One chunk of E values of input type DT as raw dwords.
template <int DT, int E>
struct Chunk {
  static constexpr int kWords = E * Elem<DT>::kBytes / 4;
  uint32_t w[kWords];
};

template <int DT, int E, bool ALIGNED, bool NT>
__device__ __forceinline__ void load_chunk(const uint8_t *p, Chunk<DT, E> &c) {
  constexpr int kWords = Chunk<DT, E>::kWords;
  if constexpr (ALIGNED) {
    if constexpr (kWords == 2) {
      const u32x2 v = ld_global<u32x2, NT>(p);
      c.w[0] = v.x, c.w[1] = v.y;
    } else {
      const u32x4 v = ld_global<u32x4, NT>(p);
      c.w[0] = v.x, c.w[1] = v.y, c.w[2] = v.z, c.w[3] = v.w;
    }
  } else if constexpr (DT == XGEN_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < kWords; ++i) c.w[i] = ld_global<uint32_t>(p + 4 * i);
  } else {
#pragma unroll
    for (int i = 0; i < kWords; ++i)
      c.w[i] = (uint32_t)ld_global<uint16_t>(p + 4 * i) | ((uint32_t)ld_global<uint16_t>(p + 4 * i + 2) << 16);
  }
}

// max |x| bits of a chunk (16-bit: |bf16|/|f16| bits, ordered like the values; f32: |x| bits).
template <int DT, int E>
__device__ __forceinline__ uint32_t chunk_absmax(const Chunk<DT, E> &c, uint32_t m) {
  if constexpr (DT == XGEN_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < Chunk<DT, E>::kWords; ++i) m = max_u32(m, c.w[i] & 0x7fffffffu);
  } else {
#pragma unroll
    for (int i = 0; i < Chunk<DT, E>::kWords; ++i) {
      const u16x2 a = Half2<DT>::absbits(c.w[i]);
      m = max_u32(m, max_u32(a.x, a.y));
    }
  }
  return m;
}

template <int DT>
__device__ __forceinline__ float absmax_value(uint32_t bits) {
  if constexpr (DT == XGEN_DTYPE_F32) return __uint_as_float(bits);
  else return Half2<DT>::from_absbits(bits);
}

struct WireScale {
  float s, r, r_lo;
  bool fast;
};

template <int DT>
__device__ __forceinline__ WireScale wire_scale(float amax) {
  WireScale q;
  float s = amax / kE4M3Max;
  s = (s < kScaleFloor) ? kScaleFloor : s;  // NaN kept
  q.s = canonical_nan(s);
  // div_by_row_scale gives IEEE's e4m3 byte for every 16-bit (x, amax) pair,
  // also at this scale floor (exhaustive oracle check); f32 inputs divide exactly.
  q.fast = DT != XGEN_DTYPE_F32 && __builtin_isfinite(s);
  float r = 1.0f / s;
  float e = __builtin_fmaf(-s, r, 1.0f);
  if (q.fast && e < 0.0f) {  // r_hi <= 1/s: one ulp down
    r = __uint_as_float(__float_as_uint(r) - 1u);
    e = __builtin_fmaf(-s, r, 1.0f);
  }
  q.r = r;
  q.r_lo = e * r;
  return q;
}

// e4m3 byte of x / s by IEEE division (NaN -> 0x7f).
__device__ __forceinline__ uint32_t wire_byte_exact(float x, float s) {
  const float v = x / s;
  if (v != v) return 0x7fu;
  return pack_e4m3x4(clamp448(v), 0.0f, 0.0f, 0.0f) & 0xffu;
}

// Four values (dword pair w0, w1 of a 16-bit chunk, or four f32 dwords) -> four bytes.
template <int DT>
__device__ __forceinline__ uint32_t quant4(const uint32_t *w, const WireScale &q) {
  float v[4];
  if constexpr (DT == XGEN_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(w[i]);
  } else {
    v[0] = Half2<DT>::lo(w[0]), v[1] = Half2<DT>::hi(w[0]);
    v[2] = Half2<DT>::lo(w[1]), v[3] = Half2<DT>::hi(w[1]);
  }
  if constexpr (DT != XGEN_DTYPE_F32) {
    if (q.fast) {  // |x| <= amax: the quotient stays below 464, which v_cvt_pk_fp8_f32 rounds to 448 at most
      float a[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = div_by_row_scale(v[i], q.r, q.r_lo);
      return pack_e4m3x4(a[0], a[1], a[2], a[3]);
    }
  }
  return wire_byte_exact(v[0], q.s) | (wire_byte_exact(v[1], q.s) << 8) | (wire_byte_exact(v[2], q.s) << 16) |
         (wire_byte_exact(v[3], q.s) << 24);
}

template <int DT, int E, bool ALIGNED, int C, bool NT>
__global__ __launch_bounds__(kThreads) void wire_encode_kernel(EncodeArgs a) {
  constexpr int kEb = Elem<DT>::kBytes;
  constexpr int kWords = Chunk<DT, E>::kWords;
  const int lanes = 1 << a.log2_lanes;
  const int lig = threadIdx.x & (lanes - 1);
  const uint32_t groups = kThreads >> a.log2_lanes;
  const uint32_t step = gridDim.x * groups;

  // per stream: source base, then peer / seq / batch / head strides (bytes)
  __shared__ int64_t tab[3][5];
  if (threadIdx.x < 15) {
    const int s = threadIdx.x / 5, k = threadIdx.x % 5;
    tab[s][k] = k == 0 ? (int64_t)(uintptr_t)a.src[s] : a.st[s][k - 1];
  }
  __syncthreads();

  struct Row {
    Chunk<DT, E> c[C];
    RowPos p;
  };
  // loads wire row w's values (zeros past the end)
  auto load_row = [&](uint32_t w, Row &r) {
    const bool ok = w < a.g.total;
    const RowPos p = locate(a.g, ok ? w : 0);
    r.p = p;
    const int64_t *t = tab[p.slot];
    const uint32_t hb = fast_div(p.pr, a.heads);
    const uint32_t head = p.pr - hb * a.heads.d;
    const uint32_t sq = fast_div(hb, a.batch);
    const uint32_t b = hb - sq * a.batch.d;
    // a row past the valid sequence is a zero row: scale 1e-12, zero bytes
    const bool live = ok && p.peer * a.seq + sq < a.valid_seq;
    const uint8_t *row = reinterpret_cast<const uint8_t *>(t[0] + (int64_t)p.peer * t[1] + (int64_t)sq * t[2] +
                                                           (int64_t)b * t[3] + (int64_t)head * t[4]);
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const int e0 = (lig + j * lanes) * E;
      if (live && e0 < a.width) {
        load_chunk<DT, E, ALIGNED, NT>(row + (int64_t)e0 * kEb, r.c[j]);
      } else {
#pragma unroll
        for (int i = 0; i < kWords; ++i) r.c[j].w[i] = 0;
      }
    }
  };

  uint32_t w = blockIdx.x * groups + (threadIdx.x >> a.log2_lanes);
  Row cur;
  load_row(w, cur);
  for (; w < a.g.total; w += step) {
    Row nxt;
    load_row(w + step, nxt);
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < C; ++j) m = chunk_absmax<DT, E>(cur.c[j], m);
    const WireScale q = wire_scale<DT>(absmax_value<DT>(group_max_u32(m, lanes)));
    uint8_t *row = a.wire + wire_offset(a.g, w, cur.p.peer);
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const int e0 = (lig + j * lanes) * E;
      if (e0 < a.width) {
        // 4 values (kEb dwords of input) -> one dword of e4m3 bytes
        if constexpr (E == 4) {
          st_global(row + e0, quant4<DT>(&cur.c[j].w[0], q));
        } else {
          st_global_a4x2(row + e0, u32x2{quant4<DT>(&cur.c[j].w[0], q), quant4<DT>(&cur.c[j].w[kEb], q)});
        }
      }
    }
    if (lig == 0) {
      st_global(row + a.width, q.s);
      // the first row of a peer's block also zeroes the padding after the block
      if (a.g.pad && cur.p.slot == 0 && cur.p.pr == 0) {
        uint8_t *tail = a.wire + wire_offset(a.g, (cur.p.peer + 1) * a.g.per_peer.d, cur.p.peer);
        for (int i = 0; i < a.g.pad; i += 4) st_global(tail + i, 0u);
      }
    }
    cur = nxt;
  }
}

// --------------------------------------------------------------------------- decode
struct DecodeArgs {
  const uint8_t *wire;
  uint8_t *dst[3];
  WireGeom g;
  int64_t dst_row_bytes;  // width * element size
  // strided form: output byte strides over (peer, seq, batch, head), shared by the streams
  int64_t dst_st[4];
  FastDiv heads, batch;
  uint32_t seq, valid_seq;  // rows with peer * seq + s >= valid_seq are not written
  int width;
  int log2_lanes;
};

// Four decoded values stored in the output dtype (8 or 16 bytes, naturally aligned).
template <int OT>
__device__ __forceinline__ void store4(uint8_t *p, const float (&v)[4]) {
  if constexpr (OT == XGEN_DTYPE_F32) {
    st_global(p, f32x4{v[0], v[1], v[2], v[3]});
  } else if constexpr (OT == XGEN_DTYPE_BF16) {
    st_global(p, u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])});
  } else {
    st_global(p, u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])});
  }
}

template <int OT>
__device__ __forceinline__ void store4_unaligned(uint8_t *p, const float (&v)[4]) {
  if constexpr (OT == XGEN_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) st_global(p + 4 * i, v[i]);
  } else {
    uint32_t w0, w1;
    if constexpr (OT == XGEN_DTYPE_BF16) w0 = pack_bf16x2(v[0], v[1]), w1 = pack_bf16x2(v[2], v[3]);
    else w0 = pack_f16x2(v[0], v[1]), w1 = pack_f16x2(v[2], v[3]);
    st_global(p, (uint16_t)w0);
    st_global(p + 2, (uint16_t)(w0 >> 16));
    st_global(p + 4, (uint16_t)w1);
    st_global(p + 6, (uint16_t)(w1 >> 16));
  }
}

// e4m3fn bytes of a dword -> four exact floats, each times the scale (fp32 product).
__device__ __forceinline__ void decode4(uint32_t b, float s, float (&v)[4]) {
  const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)b, false);
  const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)b, true);
  v[0] = lo.x * s, v[1] = lo.y * s, v[2] = hi.x * s, v[3] = hi.y * s;
}

template <int OT, int E, bool ALIGNED, int C, bool STRIDED>
__global__ __launch_bounds__(kThreads) void wire_decode_kernel(DecodeArgs a) {
  constexpr int kOb = Elem<OT>::kBytes;
  const int lanes = 1 << a.log2_lanes;
  const int lig = threadIdx.x & (lanes - 1);
  const uint32_t groups = kThreads >> a.log2_lanes;
  const uint32_t step = gridDim.x * groups;

  __shared__ int64_t dst_tab[3];
  if (threadIdx.x < 3) dst_tab[threadIdx.x] = (int64_t)(uintptr_t)a.dst[threadIdx.x];
  __syncthreads();

  struct Row {
    uint32_t b[C][E / 4];
    float s;
    RowPos p;
  };
  auto load_row = [&](uint32_t w, Row &r) {
    const bool ok = w < a.g.total;
    r.p = locate(a.g, ok ? w : 0);
    const uint8_t *row = a.wire + wire_offset(a.g, ok ? w : 0, r.p.peer);
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const int e0 = (lig + j * lanes) * E;
      const bool in = ok && e0 < a.width;
      if constexpr (E == 4) {
        r.b[j][0] = in ? ld_global<uint32_t>(row + e0) : 0u;
      } else {
        const u32x2 v = in ? ld_global_a4x2(row + e0) : u32x2{0, 0};
        r.b[j][0] = v.x, r.b[j][1] = v.y;
      }
    }
    r.s = ok ? ld_global<float>(row + a.width) : 0.0f;
  };

  uint32_t w = blockIdx.x * groups + (threadIdx.x >> a.log2_lanes);
  Row cur;
  load_row(w, cur);
  for (; w < a.g.total; w += step) {
    Row nxt;
    load_row(w + step, nxt);
    const RowPos &p = cur.p;
    uint8_t *out = reinterpret_cast<uint8_t *>(dst_tab[p.slot]);
    bool live = true;
    if constexpr (STRIDED) {
      const uint32_t hb = fast_div(p.pr, a.heads);
      const uint32_t head = p.pr - hb * a.heads.d;
      const uint32_t sq = fast_div(hb, a.batch);
      const uint32_t b = hb - sq * a.batch.d;
      live = p.peer * a.seq + sq < a.valid_seq;
      out += (int64_t)p.peer * a.dst_st[0] + (int64_t)sq * a.dst_st[1] + (int64_t)b * a.dst_st[2] +
             (int64_t)head * a.dst_st[3];
    } else {
      out += ((int64_t)p.peer * a.g.peer_rows.d + p.pr) * a.dst_row_bytes;
    }
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const int e0 = (lig + j * lanes) * E;
      if (live && e0 < a.width) {
        if constexpr (E == 8) {  // 16-bit output, 16-byte aligned runs of 8 values
          float v0[4], v1[4];
          decode4(cur.b[j][0], cur.s, v0);
          decode4(cur.b[j][1], cur.s, v1);
          u32x4 o;
          if constexpr (OT == XGEN_DTYPE_BF16)
            o = u32x4{pack_bf16x2(v0[0], v0[1]), pack_bf16x2(v0[2], v0[3]), pack_bf16x2(v1[0], v1[1]),
                      pack_bf16x2(v1[2], v1[3])};
          else
            o = u32x4{pack_f16x2(v0[0], v0[1]), pack_f16x2(v0[2], v0[3]), pack_f16x2(v1[0], v1[1]),
                      pack_f16x2(v1[2], v1[3])};
          st_global(out + (int64_t)e0 * kOb, o);
        } else {
          float v[4];
          decode4(cur.b[j][0], cur.s, v);
          if constexpr (ALIGNED) store4<OT>(out + (int64_t)e0 * kOb, v);
          else store4_unaligned<OT>(out + (int64_t)e0 * kOb, v);
        }
      }
    }
    cur = nxt;
  }
}

// --------------------------------------------------------------------------- launch helpers
struct Shape {
  int E, C, log2_lanes;
};

// A row is ceil(width / E) chunks of E values.  Lanes per row: the power of two
// in [1, 64] covering the chunks in at most c_max (1, 2 or 4) chunks per lane;
// chunk j of lane l is chunk l + j * lanes, so the lanes of a row cover
// consecutive bytes in each access.
Shape pick_shape(int width, int E, int c_max) {
  Shape sh;
  sh.E = E;
  const int chunks = (width + E - 1) / E;
  const int per_lane = (chunks + c_max - 1) / c_max;
  int l = 0;
  while ((1 << l) < per_lane && l < 6) ++l;
  sh.log2_lanes = l;
  const int c = (chunks + (1 << l) - 1) >> l;
  sh.C = c <= 1 ? 1 : (c <= 2 ? 2 : 4);
  return sh;
}

// Chunks per lane, measured at width 128: the encoder is fastest with one
// 16-byte chunk per lane (16 lanes per row), the decoder with two.
constexpr int kEncodeChunks = 1, kDecodeChunks = 2;

// Persistent grid: one resident wave of blocks, or fewer when the rows run out
// (the occupancy of each kernel is queried once).
template <typename KS, typename Args>
void launch_rows(const Args &a, int rows_per_block, hipStream_t stream) {
  static const int per_cu = resident_blocks_per_cu(KS::kernel, kThreads);
  const int64_t need = ((int64_t)a.g.total + rows_per_block - 1) / rows_per_block;
  const int64_t cap = (int64_t)device_cu_count() * per_cu;
  KS::kernel<<<dim3((unsigned)(need < cap ? need : cap)), dim3(kThreads), 0, stream>>>(a);
}

template <template <int, int, bool, int> class K, int T, int E, bool ALIGNED, typename Args>
void launch_c(const Args &a, const Shape &sh, hipStream_t stream) {
  const int rows_per_block = kThreads >> sh.log2_lanes;
  if (sh.C == 1) launch_rows<K<T, E, ALIGNED, 1>>(a, rows_per_block, stream);
  else if (sh.C == 2) launch_rows<K<T, E, ALIGNED, 2>>(a, rows_per_block, stream);
  else launch_rows<K<T, E, ALIGNED, 4>>(a, rows_per_block, stream);
}
template <template <int, int, bool, int> class K, int T, bool ALIGNED, typename Args>
void launch_ec(const Args &a, const Shape &sh, hipStream_t stream) {
  if (sh.E == 8) launch_c<K, T, 8, ALIGNED>(a, sh, stream);
  else launch_c<K, T, 4, ALIGNED>(a, sh, stream);
}
template <int DT, int E, bool ALIGNED, int C>
struct EncodeK {
  static constexpr auto kernel = wire_encode_kernel<DT, E, ALIGNED, C, false>;
};
// Non-temporal input loads: 8% faster (H3 Q/K/V, 288 MB in + 149 MB out) once
// a call's footprint exceeds the last-level cache; the decoder, whose input is
// the smaller side, gains nothing from them.
template <int DT, int E, bool ALIGNED, int C>
struct EncodeNtK {
  static constexpr auto kernel = wire_encode_kernel<DT, E, ALIGNED, C, true>;
};
template <int OT, int E, bool ALIGNED, int C>
struct DecodeK {
  static constexpr auto kernel = wire_decode_kernel<OT, E, ALIGNED, C, false>;
};
template <int OT, int E, bool ALIGNED, int C>
struct DecodeStridedK {
  static constexpr auto kernel = wire_decode_kernel<OT, E, ALIGNED, C, true>;
};

bool is_wire_dtype(int dt) { return dt == XGEN_DTYPE_BF16 || dt == XGEN_DTYPE_F16 || dt == XGEN_DTYPE_F32; }
int64_t elem_bytes(int dt) { return dt == XGEN_DTYPE_F32 ? 4 : 2; }
bool aligned_to(const void *p, int64_t n) { return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)n) == 0; }

// Shared checks of the wire geometry; fills g.
int wire_geometry(const char *fn, int streams, int64_t peers, int64_t peer_rows, int64_t width,
                  int64_t peer_padding, WireGeom &g) {
  if (streams != 1 && streams != 3)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: streams must be 1 or 3 (got %d)", fn, streams);
  if (peers < 1 || peer_rows < 0 || width <= 0 || width % 4)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad geometry peers=%lld peer_rows=%lld width=%lld (width must be "
                "a positive multiple of 4)", fn, (long long)peers, (long long)peer_rows, (long long)width);
  if (peer_padding < 0 || peer_padding >= 16 || peer_padding % 4)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: peer_padding must be 0, 4, 8 or 12 (got %lld)", fn,
                (long long)peer_padding);
  if (width > XGEN_WIRE_MAX_WIDTH)
    return fail(XGEN_ERR_UNSUPPORTED, "%s: width %lld exceeds %d", fn, (long long)width, XGEN_WIRE_MAX_WIDTH);
  // wire row indices plus one grid step of prefetch stay below 2^31
  const int64_t total = (int64_t)streams * peers * peer_rows;
  if (peer_rows > 0x3fffffffLL || total > 0x3fffffffLL)
    return fail(XGEN_ERR_UNSUPPORTED, "%s: %lld wire rows exceed 2^30", fn, (long long)total);
  g.total = (uint32_t)total;
  g.per_peer = make_fastdiv((uint32_t)(streams * peer_rows > 0 ? streams * peer_rows : 1));
  g.peer_rows = make_fastdiv((uint32_t)(peer_rows > 0 ? peer_rows : 1));
  g.row_bytes = width + 4;
  g.pad = peer_padding;
  return XGEN_OK;
}

}  // namespace

}  // namespace xgen

using namespace xgen;

extern "C" int64_t xgen_fp8_wire_peer_padding(int streams, int64_t peer_rows, int64_t width, int align16) {
  if (!align16 || (streams != 1 && streams != 3) || peer_rows < 0 || width < 0) return 0;
  const int64_t peer_bytes = (int64_t)streams * peer_rows * (width + 4);
  return (16 - peer_bytes % 16) % 16;
}

namespace xgen {
namespace {

// (peer, seq, batch, head) row geometry of a call: checks it and sets peer_rows = seq * batch * heads.
int row_geometry(const char *fn, int64_t seq, int64_t batch, int64_t heads, int64_t valid_seq, int64_t &peer_rows) {
  if (seq < 0 || batch < 0 || heads < 0 || valid_seq < 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: negative shape seq=%lld batch=%lld heads=%lld valid_seq=%lld", fn,
                (long long)seq, (long long)batch, (long long)heads, (long long)valid_seq);
  if (seq > 0x7fffffffLL || batch > 0x7fffffffLL || heads > 0x7fffffffLL ||
      (batch && heads && seq > 0x7fffffffLL / batch / heads))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: peer rows exceed 2^31 - 1", fn);
  peer_rows = seq * batch * heads;
  return XGEN_OK;
}

int wire_encode(const char *fn, int in_dtype, int streams, const void *q, const void *k, const void *v,
                const int64_t *strides, int64_t peers, int64_t seq, int64_t batch, int64_t heads, int64_t width,
                int64_t valid_seq, int64_t peer_padding, void *wire, hipStream_t stream) {
  if (!is_wire_dtype(in_dtype)) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: input dtype must be BF16, F16 or F32", fn);
  int64_t peer_rows = 0;
  if (int st = row_geometry(fn, seq, batch, heads, valid_seq, peer_rows)) return st;
  EncodeArgs a;
  if (int st = wire_geometry(fn, streams, peers, peer_rows, width, peer_padding, a.g)) return st;
  if (peer_rows == 0) return ok();
  const void *src[3] = {q, streams == 3 ? k : q, streams == 3 ? v : q};
  if (!wire || !strides || !src[0] || !src[1] || !src[2]) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  const int64_t eb = elem_bytes(in_dtype);
  bool vec16 = width % 8 == 0 && in_dtype != XGEN_DTYPE_F32, vec = true;
  for (int s = 0; s < streams; ++s) {
    for (int d = 0; d < 4; ++d) {
      const int64_t x = strides[s * 4 + d];
      if (x < 0) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: negative stride", fn);
      if (x > (int64_t)1 << 46) return fail(XGEN_ERR_UNSUPPORTED, "%s: stride too large", fn);
      vec16 = vec16 && x % 8 == 0;
      vec = vec && x % 4 == 0;
    }
    vec16 = vec16 && aligned16(src[s]);
    vec = vec && aligned_to(src[s], 4 * eb);
    if (!aligned_to(src[s], eb)) return fail(XGEN_ERR_UNSUPPORTED, "%s: input not element-aligned", fn);
  }
  if (!aligned_to(wire, 4)) return fail(XGEN_ERR_UNSUPPORTED, "%s: wire must be 4-byte aligned", fn);
  for (int s = 0; s < 3; ++s) {
    a.src[s] = static_cast<const uint8_t *>(src[s]);
    for (int d = 0; d < 4; ++d) a.st[s][d] = strides[(s < streams ? s : 0) * 4 + d] * eb;
  }
  a.wire = static_cast<uint8_t *>(wire);
  a.heads = make_fastdiv((uint32_t)heads);
  a.batch = make_fastdiv((uint32_t)batch);
  a.seq = (uint32_t)seq;
  // peers * seq < 2^30 (wire_geometry), so a larger valid_seq masks nothing
  a.valid_seq = (uint32_t)(valid_seq < peers * seq ? valid_seq : peers * seq);
  a.width = (int)width;
  // chunks of 8 values (16-byte loads of 16-bit input) or 4 (16-byte f32 / 8-byte loads)
  const Shape sh = pick_shape((int)width, vec16 ? 8 : 4, kEncodeChunks);
  a.log2_lanes = sh.log2_lanes;
  // bytes read and written by the call
  const bool nt = (int64_t)a.g.total * (width * (eb + 1) + 4) > kLastLevelCacheBytes;
  switch (in_dtype) {
    case XGEN_DTYPE_BF16:
      if (vec && nt) launch_ec<EncodeNtK, XGEN_DTYPE_BF16, true>(a, sh, stream);
      else if (vec) launch_ec<EncodeK, XGEN_DTYPE_BF16, true>(a, sh, stream);
      else launch_ec<EncodeK, XGEN_DTYPE_BF16, false>(a, sh, stream);
      break;
    case XGEN_DTYPE_F16:
      if (vec && nt) launch_ec<EncodeNtK, XGEN_DTYPE_F16, true>(a, sh, stream);
      else if (vec) launch_ec<EncodeK, XGEN_DTYPE_F16, true>(a, sh, stream);
      else launch_ec<EncodeK, XGEN_DTYPE_F16, false>(a, sh, stream);
      break;
    default:
      if (vec && nt) launch_ec<EncodeNtK, XGEN_DTYPE_F32, true>(a, sh, stream);
      else if (vec) launch_ec<EncodeK, XGEN_DTYPE_F32, true>(a, sh, stream);
      else launch_ec<EncodeK, XGEN_DTYPE_F32, false>(a, sh, stream);
      break;
  }
  return launch_status(fn);
}

template <template <int, int, bool, int> class K>
void launch_decode(int out_dtype, bool vec, const DecodeArgs &a, const Shape &sh, hipStream_t stream) {
  switch (out_dtype) {
    case XGEN_DTYPE_BF16:
      if (vec) launch_ec<K, XGEN_DTYPE_BF16, true>(a, sh, stream);
      else launch_ec<K, XGEN_DTYPE_BF16, false>(a, sh, stream);
      break;
    case XGEN_DTYPE_F16:
      if (vec) launch_ec<K, XGEN_DTYPE_F16, true>(a, sh, stream);
      else launch_ec<K, XGEN_DTYPE_F16, false>(a, sh, stream);
      break;
    default:
      if (vec) launch_ec<K, XGEN_DTYPE_F32, true>(a, sh, stream);
      else launch_ec<K, XGEN_DTYPE_F32, false>(a, sh, stream);
      break;
  }
}

// dst_strides: null for contiguous [peers * peer_rows, width] outputs, else 4 element strides over
// (peer, seq, batch, head) with rows past valid_seq skipped.
int wire_decode(const char *fn, int out_dtype, int streams, const void *wire, int64_t peers, int64_t seq,
                int64_t batch, int64_t heads, int64_t width, int64_t peer_padding, const int64_t *dst_strides,
                int64_t valid_seq, void *q, void *k, void *v, hipStream_t stream) {
  if (!is_wire_dtype(out_dtype)) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: output dtype must be BF16, F16 or F32", fn);
  int64_t peer_rows = seq;  // contiguous outputs: (seq, batch, heads) = (peer_rows, 1, 1)
  if (dst_strides)
    if (int st = row_geometry(fn, seq, batch, heads, valid_seq, peer_rows)) return st;
  DecodeArgs a;
  if (int st = wire_geometry(fn, streams, peers, peer_rows, width, peer_padding, a.g)) return st;
  if (peer_rows == 0) return ok();
  void *dst[3] = {q, streams == 3 ? k : q, streams == 3 ? v : q};
  if (!wire || !dst[0] || !dst[1] || !dst[2]) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (!aligned_to(wire, 4)) return fail(XGEN_ERR_UNSUPPORTED, "%s: wire must be 4-byte aligned", fn);
  const int64_t eb = elem_bytes(out_dtype);
  bool vec = true, vec16 = width % 8 == 0 && out_dtype != XGEN_DTYPE_F32;
  for (int s = 0; s < streams; ++s) {
    if (!aligned_to(dst[s], eb)) return fail(XGEN_ERR_UNSUPPORTED, "%s: output not element-aligned", fn);
    vec = vec && aligned_to(dst[s], 4 * eb);
    vec16 = vec16 && aligned16(dst[s]);
  }
  if (dst_strides) {
    for (int d = 0; d < 4; ++d) {
      const int64_t x = dst_strides[d];
      if (x < 0) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: negative stride", fn);
      if (x > (int64_t)1 << 46) return fail(XGEN_ERR_UNSUPPORTED, "%s: stride too large", fn);
      vec16 = vec16 && x % 8 == 0;
      vec = vec && x % 4 == 0;
      a.dst_st[d] = x * eb;
    }
  } else {
    for (int d = 0; d < 4; ++d) a.dst_st[d] = 0;
  }
  a.wire = static_cast<const uint8_t *>(wire);
  for (int s = 0; s < 3; ++s) a.dst[s] = static_cast<uint8_t *>(dst[s]);
  a.dst_row_bytes = width * eb;
  a.heads = make_fastdiv((uint32_t)(heads > 0 ? heads : 1));
  a.batch = make_fastdiv((uint32_t)(batch > 0 ? batch : 1));
  a.seq = (uint32_t)seq;
  a.valid_seq = (uint32_t)(valid_seq < peers * seq ? valid_seq : peers * seq);
  a.width = (int)width;
  // chunks of 8 values (16-byte stores of 16-bit output) or 4 (16-byte f32 / 8-byte stores)
  const Shape sh = pick_shape((int)width, vec16 ? 8 : 4, kDecodeChunks);
  a.log2_lanes = sh.log2_lanes;
  if (dst_strides) launch_decode<DecodeStridedK>(out_dtype, vec, a, sh, stream);
  else launch_decode<DecodeK>(out_dtype, vec, a, sh, stream);
  return launch_status(fn);
}

}  // namespace
}  // namespace xgen

extern "C" int xgen_fp8_wire_encode(int in_dtype, int streams, const void *q, const void *k, const void *v,
                                    const int64_t *strides, int64_t peers, int64_t seq, int64_t batch,
                                    int64_t heads, int64_t width, int64_t peer_padding, void *wire,
                                    hipStream_t stream) {
  return wire_encode("xgen_fp8_wire_encode", in_dtype, streams, q, k, v, strides, peers, seq, batch, heads, width,
                     INT64_MAX, peer_padding, wire, stream);
}

extern "C" int xgen_fp8_wire_encode_masked(int in_dtype, int streams, const void *q, const void *k,
                                           const void *v, const int64_t *strides, int64_t peers, int64_t seq,
                                           int64_t batch, int64_t heads, int64_t width, int64_t valid_seq,
                                           void *wire, hipStream_t stream) {
  return wire_encode("xgen_fp8_wire_encode_masked", in_dtype, streams, q, k, v, strides, peers, seq, batch, heads,
                     width, valid_seq, 0, wire, stream);
}

extern "C" int xgen_fp8_wire_decode(int out_dtype, int streams, const void *wire, int64_t peers,
                                    int64_t peer_rows, int64_t width, int64_t peer_padding, void *q, void *k,
                                    void *v, hipStream_t stream) {
  // contiguous outputs: the rows as one sequence axis
  return wire_decode("xgen_fp8_wire_decode", out_dtype, streams, wire, peers, peer_rows, 1, 1, width, peer_padding,
                     nullptr, INT64_MAX, q, k, v, stream);
}

extern "C" int xgen_fp8_wire_decode_strided(int out_dtype, int streams, const void *wire, int64_t peers,
                                            int64_t seq, int64_t batch, int64_t heads, int64_t width,
                                            const int64_t *dst_strides, int64_t valid_seq, void *q, void *k,
                                            void *v, hipStream_t stream) {
  if (!dst_strides) return fail(XGEN_ERR_INVALID_ARGUMENT, "xgen_fp8_wire_decode_strided: null pointer");
  return wire_decode("xgen_fp8_wire_decode_strided", out_dtype, streams, wire, peers, seq, batch, heads, width, 0,
                     dst_strides, valid_seq, q, k, v, stream);
}
