// W8A8 GEMM with fused per-token x per-channel dequant, bias and optional
// GELU-tanh epilogue, on gfx950 matrix cores.
//
//   FP8      : v_mfma_f32_32x32x64_f8f6f4 (e4m3fn x e4m3fn -> fp32)
//              replaces torch._scaled_mm at x_base/x_base/operator/h3_fp8.py:63-66
//   FP8 exact: the same e4m3fn operands, converted to bf16 (exactly) after the
//              LDS reads and multiplied by v_mfma_f32_32x32x16_bf16: exact
//              products summed in fp32, the accumulation _scaled_mm's
//              use_fast_accum=False asks for (h3_fp8.py:63-66), at twice the
//              matrix-core time of the FP8 instructions, plus the conversions
//   INT8     : v_mfma_i32_32x32x32_i8      (int8 x int8 -> exact int32)
//              replaces torch_npu.npu_quant_matmul at x_base/x_base/operator/matmul.py:63-64
//
// The FP8 instructions (all shapes, measured on gfx950) do not sum like IEEE
// fp32: within each group of 8 consecutive K the products are truncated toward
// zero to a multiple of 2^(E - 13), E the largest exponent sum e(a) + e(w) of
// the group, so the result can differ from the exactly rounded sum by up to
// ~2^-13 of the group's largest product.  The FP8-exact kind avoids that sum.
//
// out[m, n] = act(cvt(acc[m, n] * (sa[m] * sw[n]) + bias[n])),  acc = sum_k a[m,k] w[n,k]
//
// Tiling (every kind): a 256x256 output tile per workgroup of 4 waves, one per
// SIMD, each owning a 128x128 block (4x4 MFMA fragments, accumulators in
// AGPRs).  K advances in pairs of 64-byte sub-stages: bounds-checked buffer
// loads on the LDS-DMA path (no VGPR staging; rows past M/N and the K tail
// read as zero) move 128 bytes of K per row into a ring of two 64 KB pair
// slots, one pair ahead, one barrier per pair.
//
// The MFMA's A operand is the weight tile and its B operand the activation
// tile, so each lane's accumulator column is one token and its 4 consecutive
// accumulator rows are 4 consecutive output features: the epilogue writes 8
// contiguous bytes per lane per group.
//
// Workgroup -> tile mapping: the dispatcher places consecutive workgroup ids
// on the 8 XCDs round-robin; ids are remapped so each XCD owns a contiguous
// range of tiles, walked in groups of 8 tile-rows, so concurrently running
// tiles on one XCD share activation rows and weight columns in its L2.
#include "fastdiv.h"
#include "xgen_common.h"

namespace xgen {

namespace {

constexpr int BK = 64;  // K bytes per pipeline stage
// Output tiles of 256 x 256, one persistent workgroup per CU.
constexpr int kTileM = 256, kTileN = 256;

struct GemmArgs {
  const uint8_t *a;
  const uint8_t *w;
  int lda, ldw;  // bytes
  int M, N, K;
  const float *sa;
  int sa_stride;
  const float *sw;
  int sw_stride;
  const void *bias;
  int bias_dtype;
  void *out;
  int64_t ldo;  // elements
  void *acc_out;
  int tiles_m, tiles_n, per_xcd;
  int group_m;  // tile-rows per group of the tile order
  int kt4;      // stages per tile of the one-wave-per-SIMD kernel (a multiple of 4)
  uint32_t out_bytes;  // bytes of the output rows: (M - 1) * ldo * 2 + N * 2
  uint32_t a_bytes, w_bytes;
  // gated residual epilogue (GATED kernels only)
  const uint8_t *residual;
  int64_t ld_residual;  // elements
  const uint8_t *gate;
  int64_t gate_stride;  // elements
  int64_t gate_rows;
  const int64_t *indices;
  uint32_t seq, seq_magic, seq_shift;  // m % seq = m - ((mulhi(m, magic) + m) >> shift) * seq
  uint32_t residual_bytes, gate_bytes;  // (M - 1) * ld_residual * 2 + N * 2, (gate_rows - 1) * gate_stride * 2 + N * 2
};

// Operand kinds of the kernel template.
enum Kind { kInt8 = 0, kFp8 = 1, kFp8Exact = 2 };

// Operand traits per kind: accumulator and fragment types (one fragment = 32
// rows of one 64-byte K step, as the fragment reads deliver them), MFMA steps per
// 64-byte K step, 16-byte LDS reads per fragment, accumulator to float.
template <int KIND>
struct Mfma;

template <>
struct Mfma<kFp8> {
  typedef f32x16 acc_t;
  typedef i32x8 frag_t;
  static constexpr int kSteps = BK / 64;  // 32x32x64: one step per stage
  static constexpr int kReads = 2;        // ds_read_b128 per fragment
  static __device__ __forceinline__ float to_f32(float v) { return v; }
};

// The exact kind reads the FP8 kind's fragments and multiplies them as bf16.
// The conversion is exact (bf16 holds every e4m3fn value, subnormals included).
template <>
struct Mfma<kFp8Exact> {
  typedef f32x16 acc_t;
  typedef i32x8 frag_t;
  static constexpr int kSteps = 1;
  static constexpr int kReads = 2;
  static __device__ __forceinline__ bf16x8 widen(int lo, int hi) {
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    return bf16x8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
  }
  static __device__ __forceinline__ float to_f32(float v) { return v; }
};

template <>
struct Mfma<kInt8> {
  typedef i32x16 acc_t;
  typedef i32x4 frag_t;
  static constexpr int kSteps = BK / 32;  // 32x32x32: two steps per stage
  static constexpr int kReads = 1;        // ds_read_b128 per fragment
  static __device__ __forceinline__ float to_f32(int v) { return (float)v; }
};

// One 16-byte-per-lane buffer load on the LDS-DMA path: lane l's 16 bytes land
// at lds + 16 * l.  (A plain device function: called directly from the kernel
// template, the device-only builtin would keep the host pass from emitting the
// kernel's launch stub.)
__device__ __forceinline__ void dma_load16(__amdgpu_buffer_rsrc_t rsrc, uint8_t *lds, uint32_t offset) {
  typedef __attribute__((address_space(3))) void *lds_ptr_t;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)lds, 16, offset, 0, 0, 0);
}

// Workgroup barrier that orders LDS accesses without waiting for the vector
// memory counter: __syncthreads' fence would also wait for the DMA loads still
// in flight for later stages.  The empty asm statements keep the compiler from
// moving memory accesses across it; the caller waits lgkmcnt for its own LDS
// accesses first.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt constraining only the vector-memory counter (gfx9 encoding: vmcnt
// in bits [3:0] and [15:14]; expcnt [6:4] and lgkmcnt [11:8] left at max).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// v rounded to the output dtype, as the stored output is rounded.  For f16 the
// empty asm keeps v an f32 value: the fma producing it would otherwise be
// selected with the f16 rounding as one v_fma_mixlo_f16 (one rounding of the
// exact a*b+c, where the store rounds the f32 result).
template <int OUT_DT>
__device__ __forceinline__ float round_out(float v) {
  if constexpr (OUT_DT == XGEN_DTYPE_BF16) {
    return round_bf16(v);
  } else {
    asm volatile("" : "+v"(v));
    return (float)(_Float16)v;
  }
}
template <int OUT_DT>
__device__ __forceinline__ uint32_t pack_out(float a, float b) {
  if constexpr (OUT_DT == XGEN_DTYPE_BF16) return pack_bf16x2(a, b);
  else return pack_f16x2(a, b);
}

// Output tile -> (m0, n0): tiles are walked in groups of group_m tile-rows.
template <int BM, int BN>
__device__ __forceinline__ void tile_origin(int pid, int tiles_m, int tiles_n, int group_m, int &m0, int &n0) {
  const int group_size = group_m * tiles_n;
  const int group = pid / group_size;
  const int first_m = group * group_m;
  const int gm = min(tiles_m - first_m, group_m);
  const int in_group = pid - group * group_size;
  m0 = (first_m + in_group % gm) * BM;
  n0 = (in_group / gm) * BN;
}

// One persistent workgroup per CU (a multiple of the 8 XCDs), never more than
// the tiles need.  The tiles of XCD x (workgroups x, x+8, ... run there) are the
// contiguous range [x*per_xcd, (x+1)*per_xcd), dealt round-robin to that XCD's
// workgroups, so the tiles running at once on one XCD are neighbours in its L2.
dim3 gemm_grid(const GemmArgs &a) {
  const int ntiles = a.tiles_m * a.tiles_n;
  int wgs = device_cu_count() / 8 * 8;
  const int need = ((ntiles + 7) / 8) * 8;
  if (wgs > need) wgs = need;
  if (wgs < 8) wgs = 8;
  return dim3((unsigned)wgs);
}

// ---------------------------------------------------------------------------
// The kernel: one wave per SIMD.  Four waves (2 x 2) share a 256 x 256 output
// tile; each wave owns a 128 x 128 block, 4 x 4 MFMA fragments whose 256
// accumulators live in AGPRs, and issues 16 MFMAs (FP8; 32 for INT8, 64 bf16
// ones for the exact kind) per 64-byte K stage from its own instruction stream,
// so the stage's barrier syncs four waves and the LDS read traffic is 1 KB per
// 64 K of a 32 x 32 block (two waves per SIMD at 128 x 64 read 1.5 KB).
// ---------------------------------------------------------------------------
namespace w4 {
constexpr int kWaves = 4, kThreads = 256;
constexpr int kRowsPerWave = 256 / kWaves;     // DMA rows per operand per wave
// K pairs: the DMA moves 128 bytes of K per row (a whole cache line: half the
// L2 requests of 64-byte rows) into a ring of two pair slots; each pair is two
// 64-byte sub-stages of MFMAs, and one barrier per pair publishes the next.
constexpr int kPairTile = 256 * 128;            // one operand of one pair: 32 KB
constexpr int kPairSlotBytes = 2 * kPairTile;   // activations + weights: 64 KB
constexpr int kPairSlots = 2;
constexpr int kPairLoads = kRowsPerWave / 8;    // 1 KB loads (8 rows) per operand per wave per pair
constexpr int kLoadsPerPair = 2 * kPairLoads;   // 16 per thread
// One parameter set: [sa f32 x 256][sw f32 x 256][bias as stored: <= 1 KB].
// A full 1 KB DMA load per row, so a 2-byte bias row's second half takes the
// next bytes (or zeros) without leaving its row.
constexpr int kParamBytes = 3 * 1024;
constexpr int kParamBase = kPairSlots * kPairSlotBytes;
// A tile's epilogue runs during the next tile's first sub-stage, and tile
// t+3's parameters are issued with its first pair, at the earliest (2-pair
// tiles) during tile t+2's first pair: three sets rotate.
constexpr int kParamSets = 3;
constexpr int kWaveRows = 128;                 // rows of a wave's block, both dimensions
// A wave's epilogue transpose area, its own (no barrier): 32 rows of 128
// bytes (half of its block's 128 features at a time), rows 136 bytes apart:
// row r starts at bank 34 r mod 64, so the 32 rows' 8-byte writes of one
// chunk cover all 64 banks once.
constexpr int kXposeRow = 136;
constexpr int kXpose = 32 * kXposeRow;
constexpr int kXposeBase = kParamBase + kParamSets * kParamBytes;
constexpr int kLdsBytes = kXposeBase + kWaves * kXpose;  // 154 KB
}  // namespace w4

// Loads [first(s), first(s + 1)) of n loads spread over `slots` MFMA slots.
__host__ __device__ constexpr int spread_first(int s, int n, int slots) { return (s * n + slots - 1) / slots; }

// The MFMAs of the one-wave-per-SIMD kernel, with their accumulators pinned
// to AGPRs ("+a"): left to the register allocator, 256 accumulators plus the
// double-buffered fragments are shuffled between the register files and
// spilled.  The compiler sees these as opaque, so the kernel itself keeps the
// MFMA result hazards: a tile's first MFMA per accumulator adds an
// inline-constant zero (no VALU writes to accumulators at all), and the
// epilogue reads accumulators only after mfma_drain's wait states behind the
// tile's last MFMA.  Operand registers are written only by LDS loads, which
// the compiler's wait counts order before the MFMA that reads them; a buffer
// is reloaded only after the barrier that follows its last MFMA.
template <int KIND>
struct MfmaA;
template <>
struct MfmaA<kFp8> {
  static __device__ __forceinline__ void mma(f32x16 &c, const i32x8 &w, const i32x8 &x) {
    asm volatile("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, %0" : "+a"(c) : "v"(w), "v"(x));
  }
  // c = w x (the accumulator's first product: an inline-constant zero addend)
  static __device__ __forceinline__ void mma0(f32x16 &c, const i32x8 &w, const i32x8 &x) {
    asm volatile("v_mfma_f32_32x32x64_f8f6f4 %0, %1, %2, 0" : "=a"(c) : "v"(w), "v"(x));
  }
};
template <>
struct MfmaA<kInt8> {
  static __device__ __forceinline__ void mma(i32x16 &c, const i32x4 &w, const i32x4 &x) {
    asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+a"(c) : "v"(w), "v"(x));
  }
  static __device__ __forceinline__ void mma0(i32x16 &c, const i32x4 &w, const i32x4 &x) {
    asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, 0" : "=a"(c) : "v"(w), "v"(x));
  }
};
// The exact kind: e4m3fn fragments in the FP8 kind's layout, widened to bf16
// (exact for every code) and multiplied by four 32x32x16 bf16 MFMAs, step s on
// bytes 8s..8s+7 of each lane's 32 from both operands, so every product pairs
// the same K index.  The activation fragment is widened once per block row
// (widen_x) and reused by its blocks; the weight fragment per call.
template <>
struct MfmaA<kFp8Exact> {
  struct xw_t {
    bf16x8 s[4];
  };
  static __device__ __forceinline__ xw_t widen_x(const i32x8 &x) {
    xw_t r;
#pragma unroll
    for (int k = 0; k < 4; ++k) r.s[k] = Mfma<kFp8Exact>::widen(x[2 * k], x[2 * k + 1]);
    return r;
  }
  template <bool ZERO>
  static __device__ __forceinline__ void run(f32x16 &c, const i32x8 &w, const xw_t &xb) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bf16x8 wb = Mfma<kFp8Exact>::widen(w[2 * k], w[2 * k + 1]);
      // the operands were just written by VALU conversions: 2 wait states before
      // an MFMA reads them (the compiler cannot see the MFMA inside the assembly)
      if (ZERO && k == 0)
        asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=a"(c) : "v"(wb), "v"(xb.s[k]));
      else
        asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(wb), "v"(xb.s[k]));
    }
  }
  static __device__ __forceinline__ void mma(f32x16 &c, const i32x8 &w, const xw_t &xb) { run<false>(c, w, xb); }
  static __device__ __forceinline__ void mma0(f32x16 &c, const i32x8 &w, const xw_t &xb) { run<true>(c, w, xb); }
  static __device__ __forceinline__ void mma(f32x16 &c, const i32x8 &w, const i32x8 &x) { run<false>(c, w, widen_x(x)); }
  static __device__ __forceinline__ void mma0(f32x16 &c, const i32x8 &w, const i32x8 &x) { run<true>(c, w, widen_x(x)); }
};
// 24 wait states after the last MFMAs before any accumulator is read by VALU
// (16-pass MFMAs need 18 on gfx950).  Every accumulator is an operand, so no
// read of one is scheduled above it.
template <class A>
__device__ __forceinline__ void mfma_drain(A (&acc)[4][4]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
               : "+a"(acc[0][0]), "+a"(acc[1][0]), "+a"(acc[2][0]), "+a"(acc[3][0]), "+a"(acc[0][1]),
                 "+a"(acc[1][1]), "+a"(acc[2][1]), "+a"(acc[3][1]));
  asm volatile("" : "+a"(acc[0][2]), "+a"(acc[1][2]), "+a"(acc[2][2]), "+a"(acc[3][2]), "+a"(acc[0][3]),
                    "+a"(acc[1][3]), "+a"(acc[2][3]), "+a"(acc[3][3]));
}

// 128-byte rows: 16-byte chunk c of row r at c ^ ((r >> 1) & 7); the 16 lanes of
// one 128-bit access (rows r..r+15, one chunk) hit 16 distinct bank groups.
__device__ __forceinline__ int swz128(int row, int chunk) { return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4); }
template <int KIND>
__device__ __forceinline__ typename Mfma<KIND>::frag_t load_pair(const uint8_t *tile, int row, int half, int ks, int lane) {
  if constexpr (KIND == kInt8) {
    const u32x4 v = *reinterpret_cast<const u32x4 *>(tile + swz128(row, half * 4 + ks * 2 + (lane >> 5)));
    return typename Mfma<KIND>::frag_t{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
  } else {
    const int c0 = half * 4 + (lane >> 5) * 2;
    const u32x4 lo = *reinterpret_cast<const u32x4 *>(tile + swz128(row, c0));
    const u32x4 hi = *reinterpret_cast<const u32x4 *>(tile + swz128(row, c0 + 1));
    return typename Mfma<KIND>::frag_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                       (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  }
}

template <int KIND, int ACT, int OUT_DT, bool ACC_OUT, bool GATED>
__global__ __attribute__((amdgpu_flat_work_group_size(w4::kThreads, w4::kThreads), amdgpu_waves_per_eu(1, 1)))
void gemm_w4_kernel(GemmArgs p) {
  using namespace w4;
  typedef Mfma<KIND> T;
  typedef typename T::frag_t frag_t;
  constexpr int FM = 4, FN = 4, KS = T::kSteps;
  constexpr int kMfmas = KS * FM * FN;                 // per stage per wave
  constexpr int kReads = T::kReads * KS * (FM + FN);   // ds_read_b128 per stage per wave
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kLdsBytes];

  // --- this workgroup's tiles: a contiguous range per XCD, strided by workgroup ---
  const int ntiles = p.tiles_m * p.tiles_n;
  const int xcd = blockIdx.x & 7, local = blockIdx.x >> 3, wgs_per_xcd = gridDim.x >> 3;
  const int t_first = xcd * p.per_xcd + local;
  const int t_end = min((xcd + 1) * p.per_xcd, ntiles);
  const int n_my = t_first < t_end ? (t_end - t_first + wgs_per_xcd - 1) / wgs_per_xcd : 0;
  if (n_my == 0) return;
  const int KT = p.kt4;  // 64-byte sub-stages per tile: a multiple of 4; those past K read zeros

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;

  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(p.a), (short)0, (int)p.a_bytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(p.w), (short)0, (int)p.w_bytes, kBufferFlags);
  const int bias_elem = p.bias_dtype == XGEN_DTYPE_F32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(p.sa), (short)0, p.M * 4, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(p.sw), (short)0, p.N * 4, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void *>(p.bias), (short)0, p.bias ? p.N * bias_elem : 0, kBufferFlags);
  const float sa0 = p.sa_stride ? 0.0f : p.sa[0];  // per-tensor scales
  const float sw0 = p.sw_stride ? 0.0f : p.sw[0];
  // the output rows as a buffer: stores at kOutOfRange are dropped
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(p.out, (short)0, (int)p.out_bytes, kBufferFlags);
  // the gated epilogue's residual rows and gate table (reads past them return zeros)
  const __amdgpu_buffer_rsrc_t rres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(p.residual), (short)0, GATED ? (int)p.residual_bytes : 0, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rgate = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(p.gate), (short)0, GATED ? (int)p.gate_bytes : 0, kBufferFlags);
  // the AdaLN indices, read through a buffer (counted by vmcnt only: a flat load
  // would also hold every LDS wait of the epilogue until memory answers); seq < M < 2^28
  const __amdgpu_buffer_rsrc_t rind = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int64_t *>(p.indices), (short)0, GATED ? (int)(p.seq * 8) : 0, kBufferFlags);

  // --- global -> LDS DMA (wave w fills rows [64 w, 64 w + 64) of both tiles) ---
  // lane l fills row (l >> 3) of an 8-row load, physical chunk l & 7: logical
  // chunk (l & 7) ^ ((row >> 1) & 7), i.e. ^ (l >> 4) in even loads, ^ (4 | l >> 4) in odd
  const int ch_e = (lane & 7) ^ (lane >> 4), ch_o = (lane & 7) ^ (4 | (lane >> 4));
  uint32_t offa = 0, offw = 0;  // byte offsets of this lane's first row in the DMA's tile
  int dma_m0 = 0, dma_n0 = 0;
  auto set_dma_tile = [&](int i) {
    tile_origin<256, 256>(t_first + i * wgs_per_xcd, p.tiles_m, p.tiles_n, p.group_m, dma_m0, dma_n0);
    offa = (uint32_t)(dma_m0 + wave * kRowsPerWave + (lane >> 3)) * (uint32_t)p.lda;
    offw = (uint32_t)(dma_n0 + wave * kRowsPerWave + (lane >> 3)) * (uint32_t)p.ldw;
  };
  const int KP = KT / 2;  // pairs per tile
  const int GP = n_my * KP;
  int dma_h = 0, dma_k = 0, dma_i = 0;  // next pair to load: pair dma_k of my tile dma_i
  // this stage's load offsets (load 0 of each operand), or out of range
  struct Issue {
    uint32_t oe, oo, we, wo;  // this pair's offsets for even / odd loads, or out of range
    uint32_t lds;  // offset of this wave's DMA area of slot 0 (the loads' LDS addresses are formed from it per stage)
  };
  auto issue_begin = [&](int slot) {
    if (dma_k == 0 && dma_h < GP) {  // the tile's epilogue parameters ride with its first pair
      uint8_t *prm = smem + kParamBase + (dma_i % kParamSets) * kParamBytes;
      if (wave == 0 && p.sa_stride) dma_load16(rsa, prm, (uint32_t)dma_m0 * 4 + lane * 16);
      if (wave == 1 && p.sw_stride) dma_load16(rsw, prm + 1024, (uint32_t)dma_n0 * 4 + lane * 16);
      // (without a bias the resource is empty: the row reads as zeros)
      if (wave == 2) dma_load16(rb, prm + 2048, (uint32_t)(dma_n0 * bias_elem) + lane * 16);
    }
    const int k0 = dma_k * 128;
    const bool live = dma_h < GP;
    const bool ke = live && k0 + ch_e * 16 < p.K, ko = live && k0 + ch_o * 16 < p.K;
    uint32_t oe = ke ? offa + k0 + ch_e * 16 : kOutOfRange, oo = ko ? offa + k0 + ch_o * 16 : kOutOfRange;
    uint32_t we = ke ? offw + k0 + ch_e * 16 : kOutOfRange, wo = ko ? offw + k0 + ch_o * 16 : kOutOfRange;
    uint32_t lds = (uint32_t)wave * kRowsPerWave * 128;
    asm volatile("" : "+v"(oe), "+v"(oo), "+v"(we), "+v"(wo), "+s"(lds));
    (void)slot;
    return Issue{oe, oo, we, wo, lds};
  };
  // load q of the pair going to pair slot `slot`: A loads are even q, W loads odd q
  // (kOutOfRange + l * 16 * ld stays out of range: the host keeps (M + 512) * lda below 2^32)
  auto issue_load = [&](const Issue &is, int slot, int q) {
    const int l = q >> 1;  // load l of the operand: rows 8 l .. 8 l + 7 of the wave's 64
    uint8_t *dst = smem + is.lds + slot * kPairSlotBytes + l * 8 * 128;
    if (q & 1) dma_load16(rw, dst + kPairTile, ((l & 1) ? is.wo : is.we) + (uint32_t)(l * 8 * p.ldw));
    else dma_load16(ra, dst, ((l & 1) ? is.oo : is.oe) + (uint32_t)(l * 8 * p.lda));
  };
  auto issue_end = [&]() {
    ++dma_h;
    if (++dma_k == KP) {
      dma_k = 0;
      if (++dma_i < n_my) set_dma_tile(dma_i);
    }
  };

  // --- fragments ---------------------------------------------------------------
  const int row_x = wm * kWaveRows + (lane & 31);
  const int row_w = wn * kWaveRows + (lane & 31);
  frag_t xf[2][KS][FM], wf[2][KS][FN];  // [register buffer][k step][fragment]
  // sub-stage slot s = 2 * pair slot + half
  auto read_x = [&](int b, int s, int ks, int j) {
    xf[b][ks][j] = load_pair<KIND>(smem + (s >> 1) * kPairSlotBytes, row_x + j * 32, s & 1, ks, lane);
  };
  auto read_w = [&](int b, int s, int ks, int i) {
    wf[b][ks][i] = load_pair<KIND>(smem + (s >> 1) * kPairSlotBytes + kPairTile, row_w + i * 32, s & 1, ks, lane);
  };

  // defined by each tile's first sub-stage (mma0), read by its epilogue
  typename T::acc_t acc[FN][FM];

  // --- epilogue: dequant + bias (+ GELU), transpose, row stores ---------------
  // acc[i][j] element e: feature n = n0 + wn*128 + i*32 + (e/4)*8 + (lane/32)*4 + e%4,
  //                      token   m = m0 + wm*128 + j*32 + lane%32.
  // on_block(i, j, b) runs once block (i, j)'s accumulators have been read
  // (b = its position 0..15 in the epilogue's order)
  int tile_i = 0;
  auto epilogue = [&](auto on_block) {
    int m0, n0;
    tile_origin<256, 256>(t_first + tile_i * wgs_per_xcd, p.tiles_m, p.tiles_n, p.group_m, m0, n0);
    const uint8_t *prm = smem + kParamBase + (tile_i % kParamSets) * kParamBytes;
    const float *psa = reinterpret_cast<const float *>(prm);
    const float *psw = reinterpret_cast<const float *>(prm + 1024);
    const uint8_t *pb = prm + 2048;
    // the lane index, opaque: the epilogue's addresses are formed here, not
    // hoisted into registers the stage loop needs
    int el = lane;
    asm volatile("" : "+v"(el));
    const int wrow = el & 31, half = el >> 5;
    uint8_t *xb = smem + kXposeBase + wave * kXpose;
    // this lane's write position (row wrow, 8-byte chunk half + constant), and
    // read position (16 bytes: row (el >> 3) + 8 q, chunk el & 7)
    uint8_t *xw = xb + wrow * kXposeRow + half * 8;
    const uint8_t *xr = xb + (el >> 3) * kXposeRow + (el & 7) * 16;
    const int rr = el >> 3;  // this lane's read row (+ 8 q)
    // the per-token scales of this lane's rows, one per j (the same in both halves)
    float sam4[FM];
#pragma unroll
    for (int j = 0; j < FM; ++j) sam4[j] = p.sa_stride ? psa[wm * kWaveRows + j * 32 + wrow] : sa0;
    // The read-back of step (h, j) is stored during step (h, j) + 1, after that
    // step's writes to the same transpose rows: the reads were issued first, and
    // a wave's LDS operations complete in order, so they return step (h, j)'s
    // rows while the next step's values are computed.
    u32x4 prow[4];
    uint32_t pbase = 0;  // output byte offset of the pending rows (row rr, this lane's 8 columns)
    bool pcol = false;   // the pending columns lie below N
    int pm = 0;          // the pending rows' first token (GATED)
    // GATED: each step reads the AdaLN indices of its 4 token rows (mrow + 8 q) before
    // its values are computed, and after its read-back issues the loads of its
    // residual pieces, which its stores use during the next step.  The FP8 instance
    // loads its gate pieces there too; the INT8 one reads them at the store (loading
    // them ahead is 3% faster for FP8, and slower for INT8, whose registers then spill)
    constexpr bool kGateAhead = KIND == kFp8;
    u32x2 gidx[4];
    uint32_t pbad = 0;  // bit q: the pending row q's index lies outside the table
    uint32_t pgrow[4];  // (gate read at the store) the pending rows' gate-table rows
    u32x4 pres[4], pgate[4];
    [[maybe_unused]] int pn = 0;  // this lane's first pending column (gate read at the store)
    // rows past M need no check: their offsets lie past the output's last byte, where the
    // buffer drops stores (the host keeps (M + 256) * ldo * 2 below 2^32)
    auto store_pending = [&]() {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        u32x4 v = prow[q];
        if constexpr (GATED) {
          if constexpr (!kGateAhead)  // (the gate rows are small and cache-resident)
            pgate[q] = __builtin_amdgcn_raw_buffer_load_b128(
                rgate, pcol && !((pbad >> q) & 1u) ? (pgrow[q] * (uint32_t)p.gate_stride + (uint32_t)pn) * 2
                                                   : kOutOfRange, 0, 0);
          if (pcol && pm + q * 8 < p.M)
            v = (pbad >> q) & 1u ? u32x4{0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u}  // index outside the table: NaN
                                 : gate_residual8(pres[q], v, pgate[q]);
        }
        // non-temporal: the output streams past the caches the operands are re-read from
        // (measured: FFN down 4.7%, FFN up 2% faster; QKV unchanged)
        __builtin_amdgcn_raw_buffer_store_b128(v, ro, pcol ? pbase + (uint32_t)(q * 8 * p.ldo * 2) : kOutOfRange, 0,
                                               kCachePolicyNT);
      }
    };
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // features [64 h, 64 h + 64) of the wave's block
      // this lane's 32 features' scales and bias of this half, as f32:
      // [ii][gq] = features wn*128 + (2h + ii)*32 + gq*8 + half*4 .. +3
      // (one uniform branch per parameter kind around all of a half's reads,
      // so they issue together and are waited for once)
      f32x4 swr[2][4], bir[2][4];
      const int nl0 = wn * kWaveRows + 2 * h * 32 + half * 4;  // + ii*32 + gq*8
      if (p.sw_stride) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) swr[ii][gq] = *reinterpret_cast<const f32x4 *>(psw + nl0 + ii * 32 + gq * 8);
      } else {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) swr[ii][gq] = f32x4{sw0, sw0, sw0, sw0};
      }
      if (p.bias_dtype == XGEN_DTYPE_F32) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) bir[ii][gq] = *reinterpret_cast<const f32x4 *>(pb + (nl0 + ii * 32 + gq * 8) * 4);
      } else {
        // 2-byte bias (or none: the set's bias row then holds zeros, which
        // decode to 0.0 either way)
        u32x2 raw[2][4];
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) raw[ii][gq] = *reinterpret_cast<const u32x2 *>(pb + (nl0 + ii * 32 + gq * 8) * 2);
        if (p.bias_dtype == XGEN_DTYPE_F16) {
#pragma unroll
          for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              const u32x2 w2 = raw[ii][gq];
              bir[ii][gq] = f32x4{Half2<XGEN_DTYPE_F16>::lo(w2.x), Half2<XGEN_DTYPE_F16>::hi(w2.x),
                                  Half2<XGEN_DTYPE_F16>::lo(w2.y), Half2<XGEN_DTYPE_F16>::hi(w2.y)};
            }
        } else {
#pragma unroll
          for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              const u32x2 w2 = raw[ii][gq];
              bir[ii][gq] = f32x4{Half2<XGEN_DTYPE_BF16>::lo(w2.x), Half2<XGEN_DTYPE_BF16>::hi(w2.x),
                                  Half2<XGEN_DTYPE_BF16>::lo(w2.y), Half2<XGEN_DTYPE_BF16>::hi(w2.y)};
            }
        }
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int ml = wm * kWaveRows + j * 32 + wrow;
        const float sam = sam4[j];
        if constexpr (GATED) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t m = (uint32_t)(m0 + wm * kWaveRows + j * 32 + rr + 8 * q);
            const uint32_t mq = (__umulhi(m, p.seq_magic) + m) >> p.seq_shift;
            gidx[q] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rind, (m - mq * p.seq) * 8, 0, 0));
          }
        }
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            const int i = 2 * h + ii;
            // pin block (i, j)'s accumulator reads here (not hoisted, which
            // would hold them all in VGPRs at once)
            if (gq == 0) asm volatile("" : "+a"(acc[i][j]));
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float a = T::to_f32(acc[i][j][gq * 4 + e]);
              y[e] = __builtin_fmaf(a, sam * swr[ii][gq][e], bir[ii][gq][e]);
              if constexpr (ACT == XGEN_ACT_GELU_TANH) y[e] = gelu_tanh(round_out<OUT_DT>(y[e]));
            }
            // row wrow, 8-byte chunk ii*8 + gq*2 + half
            *reinterpret_cast<u32x2 *>(xw + (ii * 8 + gq * 2) * 8) =
                u32x2{pack_out<OUT_DT>(y[0], y[1]), pack_out<OUT_DT>(y[2], y[3])};
            if constexpr (ACC_OUT) {
              const int m = m0 + ml, n = n0 + wn * kWaveRows + i * 32 + gq * 8 + half * 4;
              if (m < p.M && n < p.N) {
                if constexpr (KIND != kInt8) {
                  const f32x4 v = {acc[i][j][gq * 4 + 0], acc[i][j][gq * 4 + 1], acc[i][j][gq * 4 + 2],
                                   acc[i][j][gq * 4 + 3]};
                  *reinterpret_cast<f32x4 *>(static_cast<float *>(p.acc_out) + (int64_t)m * p.N + n) = v;
                } else {
                  const i32x4 v = {acc[i][j][gq * 4 + 0], acc[i][j][gq * 4 + 1], acc[i][j][gq * 4 + 2],
                                   acc[i][j][gq * 4 + 3]};
                  *reinterpret_cast<i32x4 *>(static_cast<int32_t *>(p.acc_out) + (int64_t)m * p.N + n) = v;
                }
              }
            }
            if (gq == 3) on_block(2 * h + ii, j, h * 8 + j * 2 + ii);
          }
        if (h > 0 || j > 0) store_pending();
        // read back 8 whole rows per instruction (8 lanes x 16 bytes per row, as
        // two 8-byte reads: rows are 8-byte aligned); stored as 128-byte row
        // segments during the next step
        const int mrow = m0 + wm * kWaveRows + j * 32 + rr;               // + 8 q
        const int ncol = n0 + wn * kWaveRows + h * 64 + (el & 7) * 8;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const u32x2 lo = *reinterpret_cast<const u32x2 *>(xr + q * 8 * kXposeRow);
          const u32x2 hi = *reinterpret_cast<const u32x2 *>(xr + q * 8 * kXposeRow + 8);
          prow[q] = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
        pbase = ((uint32_t)mrow * (uint32_t)p.ldo + (uint32_t)ncol) * 2;
        pcol = ncol < p.N;
        pm = mrow;
        pn = ncol;
        if constexpr (GATED) {
          // (out-of-range rows and columns read zeros, and their stores are dropped)
          pbad = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t m = (uint32_t)(mrow + 8 * q);
            // an int64 index in [0, gate_rows): high word 0, low word below gate_rows (< 2^31)
            const bool ok = gidx[q].y == 0 && gidx[q].x < (uint32_t)p.gate_rows;
            pbad |= ok ? 0u : 1u << q;
            pres[q] = __builtin_amdgcn_raw_buffer_load_b128(
                rres, pcol ? (m * (uint32_t)p.ld_residual + (uint32_t)ncol) * 2 : kOutOfRange, 0, 0);
            if constexpr (kGateAhead)
              pgate[q] = __builtin_amdgcn_raw_buffer_load_b128(
                  rgate, pcol && ok ? (gidx[q].x * (uint32_t)p.gate_stride + (uint32_t)ncol) * 2 : kOutOfRange, 0, 0);
            else
              pgrow[q] = gidx[q].x;
          }
        }
      }
    }
    store_pending();
    ++tile_i;
  };

  // --- one 64-byte sub-stage g, U = g % 4: pair slot U >> 1, half U & 1 -------
  // Its MFMAs use register buffer U & 1 (read during sub-stage g-1); during
  // it the next sub-stage's fragments are read into the other buffer.  The
  // second sub-stage of a pair (U odd) starts by waiting for this thread's
  // DMA of the next pair (the only one outstanding), retiring its own reads;
  // the barrier then publishes every wave's DMA of the next pair and retires
  // every wave's reads of this pair's slot, which takes the DMA of the pair
  // after next, spread over this sub-stage's MFMAs (all at once is measured
  // slower: the loads queue in the address unit ahead of the MFMAs).
  // vector-memory operations of one epilogue after the pending DMA: its 32 row
  // stores (2 halves x 4 token blocks x 4 row groups, all issued, out-of-range
  // ones included); the gated and accumulator-output forms issue a varying
  // number and wait for all
  constexpr int kEpiStores = (GATED || ACC_OUT) ? 0 : 2 * FM * 4;
  bool epi_stores = false;
  auto stage = [&](auto U, auto FRESH, auto READ) {
    constexpr int u = decltype(U)::value;
    constexpr bool fresh = decltype(FRESH)::value;  // the tile's first sub-stage
    constexpr bool read = decltype(READ)::value;    // not the tile's last stage
    constexpr int cb = u & 1, nb = cb ^ 1, ns = (u + 1) & 3;
    constexpr bool odd = u & 1;  // the second sub-stage of a pair: barrier, and the DMA of pair + 2
    Issue is{};
    if constexpr (odd) {
      // the DMA of the next pair; after an epilogue its row stores were issued
      // later and need not have completed (the counter retires in issue order)
      if (epi_stores) wait_vmcnt<kEpiStores>();
      else wait_vmcnt<0>();
      epi_stores = false;
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      lds_barrier();
      is = issue_begin(u >> 1);
    }
    // The MFMAs are volatile asm statements, so the loads written between them
    // stay in this order: per MFMA, its share of the next stage's fragment
    // reads (weights first) and of the DMA loads.
    [[maybe_unused]] typename std::conditional<KIND == kFp8Exact, MfmaA<kFp8Exact>::xw_t, int>::type xw{};
#pragma unroll
    for (int s = 0; s < kMfmas; ++s) {
      const int ks = s / (FM * FN), j = (s / FN) % FM, i = s % FN;
      if constexpr (KIND == kFp8Exact) {
        if (i == 0) xw = MfmaA<KIND>::widen_x(xf[cb][ks][j]);
        if (fresh && ks == 0) MfmaA<KIND>::mma0(acc[i][j], wf[cb][ks][i], xw);
        else MfmaA<KIND>::mma(acc[i][j], wf[cb][ks][i], xw);
      } else {
        if (fresh && ks == 0) MfmaA<KIND>::mma0(acc[i][j], wf[cb][ks][i], xf[cb][ks][j]);
        else MfmaA<KIND>::mma(acc[i][j], wf[cb][ks][i], xf[cb][ks][j]);
      }
      if constexpr (read) {
#pragma unroll
        for (int r = spread_first(s, kReads / T::kReads, kMfmas); r < spread_first(s + 1, kReads / T::kReads, kMfmas); ++r) {
          const int rks = r / (FM + FN), f = r % (FM + FN);
          if (f < FN) read_w(nb, ns, rks, f);
          else read_x(nb, ns, rks, f - FN);
        }
      }
      if constexpr (odd) {
#pragma unroll
        for (int q = spread_first(s, kLoadsPerPair, kMfmas); q < spread_first(s + 1, kLoadsPerPair, kMfmas); ++q)
          if (s < kMfmas) issue_load(is, u >> 1, q);
      }
    }
    if constexpr (odd) issue_end();
  };
  // stage 0's fragments (slot 0, register buffer 0)
  auto read_first = [&]() {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int i = 0; i < FN; ++i) read_w(0, 0, ks, i);
#pragma unroll
      for (int j = 0; j < FM; ++j) read_x(0, 0, ks, j);
    }
  };
  // The next tile's first sub-stage (pair slot 0 half 0, register buffer 0)
  // with this tile's epilogue: each block's first MFMA(s) of the next tile are
  // issued as soon as the epilogue has read that block's accumulators, so the
  // matrix core works through the epilogue.  The second sub-stage's fragments
  // are read at the end, keeping their registers free through the epilogue.
  auto stage0_with_epilogue = [&]() {
    epilogue([&](int i, int j, int b) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks == 0) MfmaA<KIND>::mma0(acc[i][j], wf[0][ks][i], xf[0][ks][j]);
        else MfmaA<KIND>::mma(acc[i][j], wf[0][ks][i], xf[0][ks][j]);
      }
      (void)b;
    });
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int i = 0; i < FN; ++i) read_w(1, 1, ks, i);
#pragma unroll
      for (int j = 0; j < FM; ++j) read_x(1, 1, ks, j);
    }
  };
  typedef std::integral_constant<int, 0> S0;
  typedef std::integral_constant<int, 1> S1;
  typedef std::integral_constant<int, 2> S2;
  typedef std::integral_constant<int, 3> S3;
  typedef std::integral_constant<bool, true> Fresh;
  typedef std::integral_constant<bool, false> Acc;
  typedef std::integral_constant<bool, true> Rd;
  typedef std::integral_constant<bool, false> NoRd;

  // --- prologue: pairs 0 and 1 in flight, sub-stage 0's fragments in registers -
  set_dma_tile(0);
  {
    Issue is = issue_begin(0);
#pragma unroll
    for (int q = 0; q < kLoadsPerPair; ++q) issue_load(is, 0, q);
    issue_end();
    is = issue_begin(1);
#pragma unroll
    for (int q = 0; q < kLoadsPerPair; ++q) issue_load(is, 1, q);
    issue_end();
    wait_vmcnt<kLoadsPerPair>();
    lds_barrier();
    read_first();
  }
  // --- main loop: per tile, its sub-stages four at a time (static slots and
  // register buffers), then its epilogue.  The tile's last sub-stage does not
  // read the next tile's first fragments: they are read after it, so no
  // fragment registers are held through the epilogue. ------------------------
  stage(S0(), Fresh(), Rd());  // the first tile's first sub-stage; the others' run with the epilogues
  for (int t = 0; t < n_my; ++t) {
    if (KT > 4) {
      stage(S1(), Acc(), Rd());
      stage(S2(), Acc(), Rd());
      stage(S3(), Acc(), Rd());
      for (int c = 8; c < KT; c += 4) {
        stage(S0(), Acc(), Rd());
        stage(S1(), Acc(), Rd());
        stage(S2(), Acc(), Rd());
        stage(S3(), Acc(), Rd());
      }
      stage(S0(), Acc(), Rd());
    }
    stage(S1(), Acc(), Rd());
    stage(S2(), Acc(), Rd());
    stage(S3(), Acc(), NoRd());
    mfma_drain(acc);
    // after the last tile too (one epilogue instance: a second one costs the
    // register allocator its fit): the "next tile" is then stages past the
    // stream's end, whose loads read zeros, and its MFMAs' results are unused
    read_first();
    stage0_with_epilogue();
    epi_stores = kEpiStores > 0;
  }
  // the loads of the stages past my last may still be writing LDS
  wait_vmcnt<0>();
}

template <int KIND, int ACT, int OUT_DT>
void launch_gemm_w4(const GemmArgs &a, bool acc_out, hipStream_t stream) {
  const dim3 grid = gemm_grid(a), block(w4::kThreads);
  if (acc_out) gemm_w4_kernel<KIND, ACT, OUT_DT, true, false><<<grid, block, 0, stream>>>(a);
  else gemm_w4_kernel<KIND, ACT, OUT_DT, false, false><<<grid, block, 0, stream>>>(a);
}

template <int KIND>
void launch_gemm_w4_gated(const GemmArgs &a, hipStream_t stream) {
  gemm_w4_kernel<KIND, XGEN_ACT_NONE, XGEN_DTYPE_BF16, false, true>
      <<<gemm_grid(a), dim3(w4::kThreads), 0, stream>>>(a);
}

struct GateParams {  // the gated residual epilogue's inputs (null residual: plain GEMM)
  const void *residual = nullptr;
  int64_t ld_residual = 0;
  const void *gate = nullptr;
  int64_t gate_stride = 0, gate_rows = 0;
  const int64_t *indices = nullptr;
  int64_t seq = 0;
};

template <int KIND>
int gemm_entry(const char *fn, const void *a, int64_t lda, const void *w, int64_t ldw, int64_t M,
               int64_t N, int64_t K, const float *sa, int64_t sa_stride, const float *sw,
               int64_t sw_stride, const void *bias, int bias_dtype, int activation, void *out,
               int out_dtype, int64_t ldo, void *acc_out, hipStream_t stream,
               const GateParams &gp = GateParams()) {
  const bool gated = gp.residual != nullptr;
  if (M < 0 || N <= 0 || K <= 0)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad shape M=%lld N=%lld K=%lld", fn, (long long)M,
                (long long)N, (long long)K);
  if (lda < K || ldw < K || ldo < N)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: leading dimensions must cover the rows", fn);
  if (sa_stride != 0 && sa_stride != 1) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: activation scale stride must be 0 or 1", fn);
  if (sw_stride != 0 && sw_stride != 1) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: weight scale stride must be 0 or 1", fn);
  if (bias && bias_dtype != XGEN_DTYPE_BF16 && bias_dtype != XGEN_DTYPE_F16 && bias_dtype != XGEN_DTYPE_F32)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bias dtype must be BF16, F16 or F32", fn);
  if (activation != XGEN_ACT_NONE && activation != XGEN_ACT_GELU_TANH)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: unknown activation %d", fn, activation);
  if (out_dtype != XGEN_DTYPE_BF16 && out_dtype != XGEN_DTYPE_F16)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: output dtype must be BF16 or F16", fn);
  if (M == 0) return ok();
  if (!a || !w || !sa || !sw || !out) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (K % 16 || N % 16) return fail(XGEN_ERR_UNSUPPORTED, "%s: K and N must be multiples of 16", fn);
  if (lda % 16 || ldw % 16 || !aligned16(a) || !aligned16(w))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: operand rows must be 16-byte aligned", fn);
  if (ldo % 8 || !aligned16(out))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: output rows must be 16-byte aligned", fn);
  if ((bias && !aligned16(bias)) || (sw_stride && !aligned16(sw)) || (sa_stride && !aligned16(sa)) ||
      (acc_out && !aligned16(acc_out)))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: scale, bias and accumulator buffers must be 16-byte aligned", fn);
  if (gated) {
    if (!gp.gate || !gp.indices) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
    if (gp.seq <= 0 || M % gp.seq || gp.gate_rows <= 0 || gp.ld_residual < N || gp.gate_stride < N)
      return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: bad gated residual shape (M %% seq, gate rows, strides)", fn);
    if (gp.ld_residual % 8 || gp.gate_stride % 8 || !aligned16(gp.residual) || !aligned16(gp.gate))
      return fail(XGEN_ERR_UNSUPPORTED, "%s: residual and gate rows must be 16-byte aligned", fn);
    if (M >= 0x7fffffffLL) return fail(XGEN_ERR_UNSUPPORTED, "%s: too many rows", fn);
    // 32-bit offsets of the gate rows
    if ((uint64_t)gp.gate_rows * (uint64_t)gp.gate_stride * 2 >= (1ull << 31))
      return fail(XGEN_ERR_UNSUPPORTED, "%s: gate table above 2 GiB", fn);
  }
  // The kernels address the activation rows, the output rows and the residual rows through 32-bit
  // buffer offsets (rows past M of the last tile-row included).  A call whose rows pass those
  // limits runs as consecutive launches over row chunks: each output row is computed by the same
  // tiles in the same K order whichever launch it falls in, so the results are those of one launch.
  int64_t rows = M;
  auto cap = [&](int64_t limit) { rows = limit < rows ? limit : rows; };
  cap((0x7fffffffLL - K) / lda + 1);                   // activation bytes below 2^31
  cap(0xffffffffLL / lda - 512);                       // DMA offsets of the rows past M below 2^32
  cap((0x7fffffffLL - 2 * N) / (2 * ldo) + 1);         // output bytes below 2^31
  cap(0xffffffffLL / (2 * ldo) - 256);                 // store offsets of the rows past M below 2^32
  if (gated) cap(0x7fffffffLL / (2 * gp.ld_residual) - 256);  // residual rows past M below 2^31
  if (rows < M) {
    rows = rows / 256 * 256;                           // whole tile-rows
    if (gated) rows = rows / gp.seq * gp.seq;          // chunks start at token position 0
    if (rows <= 0) return fail(XGEN_ERR_UNSUPPORTED, "%s: operand rows too long for 32-bit offsets", fn);
    for (int64_t m0 = 0; m0 < M; m0 += rows) {
      const int64_t mi = M - m0 < rows ? M - m0 : rows;
      GateParams gc = gp;
      if (gated) gc.residual = static_cast<const uint8_t *>(gp.residual) + m0 * gp.ld_residual * 2;
      const int st = gemm_entry<KIND>(
          fn, static_cast<const uint8_t *>(a) + m0 * lda, lda, w, ldw, mi, N, K, sa_stride ? sa + m0 : sa, sa_stride,
          sw, sw_stride, bias, bias_dtype, activation, static_cast<uint8_t *>(out) + m0 * ldo * 2, out_dtype, ldo,
          acc_out ? static_cast<uint8_t *>(acc_out) + m0 * N * 4 : nullptr, stream, gc);
      if (st != XGEN_OK) return st;
    }
    return ok();
  }
  const int64_t a_bytes = (M - 1) * lda + K, w_bytes = (N - 1) * ldw + K;
  if (a_bytes >= (int64_t)kOutOfRange || w_bytes >= (int64_t)kOutOfRange)
    return fail(XGEN_ERR_UNSUPPORTED, "%s: operands above 2 GiB", fn);
  // the DMA offsets of the rows past M / N of the last tiles stay below 2^32
  if ((uint64_t)(M + 512) * (uint64_t)lda >= (1ull << 32) || (uint64_t)(N + 512) * (uint64_t)ldw >= (1ull << 32))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: operand rows too long for 32-bit offsets", fn);

  GemmArgs g;
  g.a = static_cast<const uint8_t *>(a);
  g.w = static_cast<const uint8_t *>(w);
  g.lda = (int)lda;
  g.ldw = (int)ldw;
  g.M = (int)M;
  g.N = (int)N;
  g.K = (int)K;
  g.sa = sa;
  g.sa_stride = (int)sa_stride;
  g.sw = sw;
  g.sw_stride = (int)sw_stride;
  g.bias = bias;
  g.bias_dtype = bias_dtype;
  g.out = out;
  g.ldo = ldo;
  g.acc_out = acc_out;
  g.tiles_m = (int)((M + kTileM - 1) / kTileM);
  g.tiles_n = (int)((N + kTileN - 1) / kTileN);
  g.per_xcd = (g.tiles_m * g.tiles_n + 7) / 8;
  // The 32 tiles one XCD runs at once span group_m tile-rows; measured at
  // M=15,624: 8 rows beat 4 for QKV and FFN up by ~1% and tie for FFN down; 2
  // are 4-7% slower, 16 no better.  An activation operand larger than the
  // last-level cache (C5's FFN down: 31,248 x 12,288 bytes) takes 4: the eight
  // XCDs' groups then hold 100 instead of 200 MB of it at once (FFN down at
  // M=31,248: 923 against 962-967 us; the H3 FFN down and the M=31,248 QKV and
  // FFN up, whose activations fit, stay fastest with 8).
  g.group_m = (int64_t)M * K > kLastLevelCacheBytes ? 4 : 8;
  g.a_bytes = (uint32_t)a_bytes;
  g.w_bytes = (uint32_t)w_bytes;
  g.residual = static_cast<const uint8_t *>(gp.residual);
  g.ld_residual = gp.ld_residual;
  g.gate = static_cast<const uint8_t *>(gp.gate);
  g.gate_stride = gp.gate_stride;
  g.gate_rows = gp.gate_rows;
  g.indices = gp.indices;
  g.seq = (uint32_t)gp.seq;
  g.seq_magic = g.seq_shift = 0;  // (read by the gated kernels only)
  if (gated) {
    const FastDiv fd = make_fastdiv((uint32_t)gp.seq);
    g.seq_magic = fd.m;
    g.seq_shift = fd.l;
  }
  g.residual_bytes = gated ? (uint32_t)(((M - 1) * gp.ld_residual + N) * 2) : 0;
  g.gate_bytes = gated ? (uint32_t)(((gp.gate_rows - 1) * gp.gate_stride + N) * 2) : 0;
  g.kt4 = (int)(((K + BK - 1) / BK + 3) / 4 * 4);
  const int64_t out_bytes = ((M - 1) * ldo + N) * 2;
  if (out_bytes >= (int64_t)kOutOfRange)
    return fail(XGEN_ERR_UNSUPPORTED, "%s: output above 2 GiB", fn);
  // the store offsets of the rows past M in the last tile-row stay below 2^32
  if ((uint64_t)(M + 256) * (uint64_t)ldo * 2 >= (1ull << 32))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: output rows too long for 32-bit offsets", fn);
  g.out_bytes = (uint32_t)out_bytes;
  const bool with_acc = acc_out != nullptr;
  if (gated) {
    // (the gated entry takes the FP8 and INT8 kinds only: no exact-kind instance)
    if constexpr (KIND != kFp8Exact) launch_gemm_w4_gated<KIND>(g, stream);
  } else if (activation == XGEN_ACT_NONE) {
    if (out_dtype == XGEN_DTYPE_BF16) launch_gemm_w4<KIND, XGEN_ACT_NONE, XGEN_DTYPE_BF16>(g, with_acc, stream);
    else launch_gemm_w4<KIND, XGEN_ACT_NONE, XGEN_DTYPE_F16>(g, with_acc, stream);
  } else {
    if (out_dtype == XGEN_DTYPE_BF16) launch_gemm_w4<KIND, XGEN_ACT_GELU_TANH, XGEN_DTYPE_BF16>(g, with_acc, stream);
    else launch_gemm_w4<KIND, XGEN_ACT_GELU_TANH, XGEN_DTYPE_F16>(g, with_acc, stream);
  }
  return launch_status(fn);
}

}  // namespace

}  // namespace xgen

using namespace xgen;

extern "C" int xgen_scaled_mm_fp8(const void *a, int64_t lda, const void *w, int64_t ldw, int64_t M,
                                  int64_t N, int64_t K, const float *a_scale, int64_t a_scale_stride,
                                  const float *w_scale, int64_t w_scale_stride, const void *bias,
                                  int bias_dtype, int activation, void *out, int out_dtype,
                                  int64_t ldo, float *acc_out, hipStream_t stream) {
  return gemm_entry<kFp8>("xgen_scaled_mm_fp8", a, lda, w, ldw, M, N, K, a_scale, a_scale_stride,
                          w_scale, w_scale_stride, bias, bias_dtype, activation, out, out_dtype, ldo,
                          acc_out, stream);
}

extern "C" int xgen_scaled_mm_fp8_exact(const void *a, int64_t lda, const void *w, int64_t ldw, int64_t M,
                                        int64_t N, int64_t K, const float *a_scale, int64_t a_scale_stride,
                                        const float *w_scale, int64_t w_scale_stride, const void *bias,
                                        int bias_dtype, int activation, void *out, int out_dtype,
                                        int64_t ldo, float *acc_out, hipStream_t stream) {
  return gemm_entry<kFp8Exact>("xgen_scaled_mm_fp8_exact", a, lda, w, ldw, M, N, K, a_scale, a_scale_stride,
                               w_scale, w_scale_stride, bias, bias_dtype, activation, out, out_dtype, ldo,
                               acc_out, stream);
}

extern "C" int xgen_quant_matmul_int8(const void *a, int64_t lda, const void *w, int64_t ldw,
                                      int64_t M, int64_t N, int64_t K, const float *pertoken_scale,
                                      int64_t pertoken_scale_stride, const float *w_scale,
                                      int64_t w_scale_stride, const void *bias, int bias_dtype,
                                      int activation, void *out, int out_dtype, int64_t ldo,
                                      int32_t *acc_out, hipStream_t stream) {
  return gemm_entry<kInt8>("xgen_quant_matmul_int8", a, lda, w, ldw, M, N, K, pertoken_scale,
                           pertoken_scale_stride, w_scale, w_scale_stride, bias, bias_dtype,
                           activation, out, out_dtype, ldo, acc_out, stream);
}

extern "C" int xgen_w8a8_gate_residual(int in_dtype, const void *a, int64_t lda, const void *w, int64_t ldw,
                                       int64_t M, int64_t N, int64_t K, const float *a_scale,
                                       int64_t a_scale_stride, const float *w_scale, int64_t w_scale_stride,
                                       const void *bias, int bias_dtype, const void *residual,
                                       int64_t ld_residual, const void *gate_table, int64_t gate_row_stride,
                                       int64_t gate_rows, const int64_t *indices, int64_t seq, void *out,
                                       int64_t ldo, hipStream_t stream) {
  const char *fn = "xgen_w8a8_gate_residual";
  if (in_dtype != XGEN_DTYPE_E4M3 && in_dtype != XGEN_DTYPE_I8)
    return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: operand dtype must be E4M3 or I8", fn);
  if (M > 0 && !residual) return fail(XGEN_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  GateParams gp;
  gp.residual = residual;
  gp.ld_residual = ld_residual;
  gp.gate = gate_table;
  gp.gate_stride = gate_row_stride;
  gp.gate_rows = gate_rows;
  gp.indices = indices;
  gp.seq = seq;
  if (in_dtype == XGEN_DTYPE_E4M3)
    return gemm_entry<kFp8>(fn, a, lda, w, ldw, M, N, K, a_scale, a_scale_stride, w_scale, w_scale_stride, bias,
                            bias_dtype, XGEN_ACT_NONE, out, XGEN_DTYPE_BF16, ldo, nullptr, stream, gp);
  return gemm_entry<kInt8>(fn, a, lda, w, ldw, M, N, K, a_scale, a_scale_stride, w_scale, w_scale_stride, bias,
                           bias_dtype, XGEN_ACT_NONE, out, XGEN_DTYPE_BF16, ldo, nullptr, stream, gp);
}
