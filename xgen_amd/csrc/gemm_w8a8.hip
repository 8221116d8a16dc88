// W8A8 GEMM with fused per-token x per-channel dequant, bias and optional
// GELU-tanh epilogue, on gfx950 matrix cores.
//
//   FP8      : v_mfma_f32_32x32x64_f8f6f4 (e4m3fn x e4m3fn -> fp32)
//              replaces torch._scaled_mm at x_base/x_base/operator/h3_fp8.py:63-66
//   FP8 exact: the same e4m3fn operands, converted to bf16 (exactly) after the
//              LDS reads and multiplied by v_mfma_f32_32x32x16_bf16: exact
//              products summed in fp32, the accumulation _scaled_mm's
//              use_fast_accum=False asks for (h3_fp8.py:63-66), at twice the
//              matrix-core time of the FP8 instructions
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
// Tiling: a 256x256 output tile per workgroup of WM x WN waves; each wave owns
// a (256/WM) x (256/WN) block of 32x32 MFMA tiles with accumulators in AGPRs.
// With 8 waves (2 per SIMD) one wave issues MFMAs while the other waits on
// LDS or the barrier.  K advances in stages of 64 bytes through a ring of 4
// LDS slots (4 x (16 KB activations + 16 KB weights)); operands go global ->
// LDS by bounds-checked buffer loads on the LDS-DMA path (no VGPR staging;
// rows past M/N and the K tail read as zero), issued 3 stages ahead of the
// MFMAs that consume them, one barrier per stage.
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
#include "xgen_common.h"

namespace xgen {

namespace {

constexpr int BM = 256, BN = 256;
constexpr int BK = 64;                        // K bytes per pipeline stage
constexpr int kStages = 4;                    // LDS ring depth
constexpr int kTileBytes = 256 * BK;          // one operand tile of one stage: 16 KB
constexpr int kStageBytes = 2 * kTileBytes;   // activations + weights: 32 KB
// instruction classes of __builtin_amdgcn_sched_group_barrier
constexpr int kMfma = 0x008, kVmemRead = 0x020, kDsRead = 0x100;

// Waves per workgroup (along M and N) of the production configuration.
constexpr int kWavesM = 2, kWavesN = 4;

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
  uint32_t a_bytes, w_bytes;
  // gated residual epilogue (GATED kernels only)
  const uint8_t *residual;
  int64_t ld_residual;  // elements
  const uint8_t *gate;
  int64_t gate_stride;  // elements
  int64_t gate_rows;
  const int64_t *indices;
  uint32_t seq;
};

// LDS layout of one operand tile of one stage: 256 rows x 64 bytes (4 chunks
// of 16 bytes).  Chunk c of row r is stored at chunk position c ^ ((r >> 2) & 3).
// gfx950's LDS has 64 banks (256 bytes per cycle): the 16 lanes one 128-bit
// access serves (rows r..r+15, one logical chunk) then hit 16 distinct 16-byte
// bank groups.
__device__ __forceinline__ int swz(int row, int chunk) {
  return row * BK + ((chunk ^ ((row >> 2) & 3)) << 4);
}

// Operand kinds of the kernel template.
enum Kind { kInt8 = 0, kFp8 = 1, kFp8Exact = 2 };

template <int KIND>
struct Mfma;

template <>
struct Mfma<kFp8> {
  typedef f32x16 acc_t;
  typedef i32x8 frag_t;
  static constexpr int kSteps = BK / 64;  // 32x32x64: one step per stage
  static constexpr int kReads = 2;        // ds_read_b128 per fragment
  static __device__ __forceinline__ frag_t load(const uint8_t *tile, int row, int ks, int lane) {
    const int c0 = ks * 4 + (lane >> 5) * 2;
    const u32x4 lo = *reinterpret_cast<const u32x4 *>(tile + swz(row, c0));
    const u32x4 hi = *reinterpret_cast<const u32x4 *>(tile + swz(row, c0 + 1));
    return frag_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  }
  static __device__ __forceinline__ acc_t mma(const frag_t &w, const frag_t &x, const acc_t &c) {
    // cbsz = blgp = 0: both operands e4m3; zero scale operands: unscaled MFMA.
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, x, c, 0, 0, 0, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f32(float v) { return v; }
  static constexpr int kMfmaPerMma = 1;
};

// e4m3fn bytes of one fragment (32 per lane, the FP8 kind's LDS reads) as four
// 32x32x16 bf16 MFMAs: step s takes bytes 8s..8s+7 of each lane's 32, from both
// operands alike, so every product pairs the same K index of the two.  The
// conversion is exact (bf16 holds every e4m3fn value, subnormals included).
template <>
struct Mfma<kFp8Exact> {
  typedef f32x16 acc_t;
  typedef i32x8 frag_t;
  static constexpr int kSteps = 1;
  static constexpr int kReads = 2;
  static __device__ __forceinline__ frag_t load(const uint8_t *tile, int row, int ks, int lane) {
    return Mfma<kFp8>::load(tile, row, ks, lane);
  }
  static __device__ __forceinline__ bf16x8 widen(int lo, int hi) {
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    return bf16x8{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
  }
  // Each call converts its own copies: shared across the calls of a stage the
  // converted weight fragments would stay live (32 more registers) and spill.
  static __device__ __forceinline__ acc_t mma(const frag_t &w, const frag_t &x, const acc_t &c) {
    acc_t r = c;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      int w0 = w[2 * s], w1 = w[2 * s + 1];
      asm volatile("" : "+v"(w0), "+v"(w1));
      r = __builtin_amdgcn_mfma_f32_32x32x16_bf16(widen(w0, w1), widen(x[2 * s], x[2 * s + 1]), r, 0, 0, 0);
    }
    return r;
  }
  static __device__ __forceinline__ float to_f32(float v) { return v; }
  static constexpr int kMfmaPerMma = 4;
};

template <>
struct Mfma<kInt8> {
  typedef i32x16 acc_t;
  typedef i32x4 frag_t;
  static constexpr int kSteps = BK / 32;  // 32x32x32: two steps per stage
  static constexpr int kReads = 1;        // ds_read_b128 per fragment
  static __device__ __forceinline__ frag_t load(const uint8_t *tile, int row, int ks, int lane) {
    const int c = ks * 2 + (lane >> 5);
    const u32x4 v = *reinterpret_cast<const u32x4 *>(tile + swz(row, c));
    return frag_t{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
  }
  static __device__ __forceinline__ acc_t mma(const frag_t &w, const frag_t &x, const acc_t &c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(w, x, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f32(int v) { return (float)v; }
  static constexpr int kMfmaPerMma = 1;
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

// GELU with the tanh approximation, via tanh(z) = 2*sigmoid(2z) - 1:
// 0.5*x*(1 + tanh(z)) = x / (1 + exp(-2z)),  z = sqrt(2/pi) * (x + 0.044715 x^3).
__device__ __forceinline__ float gelu_tanh(float x) {
  constexpr float kBeta = 0.7978845608028654f;  // sqrt(2/pi)
  constexpr float kKappa = 0.044715f;
  constexpr float kNeg2Log2e = -2.0f * 1.4426950408889634f;
  const float z = x * __builtin_fmaf(kBeta * kKappa, x * x, kBeta);
  const float t = __builtin_amdgcn_exp2f(z * kNeg2Log2e);
  return x * __builtin_amdgcn_rcpf(1.0f + t);
}

template <int OUT_DT>
__device__ __forceinline__ float round_out(float v) {
  if constexpr (OUT_DT == XGEN_DTYPE_BF16) return round_bf16(v);
  else return (float)(_Float16)v;
}
template <int OUT_DT>
__device__ __forceinline__ uint32_t pack_out(float a, float b) {
  if constexpr (OUT_DT == XGEN_DTYPE_BF16) return pack_bf16x2(a, b);
  else return pack_f16x2(a, b);
}

// Bias element n of a bf16 / f16 / f32 row, as float.
__device__ __forceinline__ float bias_at(const uint8_t *bias, int dtype, int n) {
  if (dtype == XGEN_DTYPE_F32) return reinterpret_cast<const float *>(bias)[n];
  const uint16_t h = reinterpret_cast<const uint16_t *>(bias)[n];
  return dtype == XGEN_DTYPE_BF16 ? Half2<XGEN_DTYPE_BF16>::lo(h) : Half2<XGEN_DTYPE_F16>::lo(h);
}

// Output tile -> (m0, n0): tiles are walked in groups of group_m tile-rows.
__device__ __forceinline__ void tile_origin(int pid, int tiles_m, int tiles_n, int group_m, int &m0, int &n0) {
  const int group_size = group_m * tiles_n;
  const int group = pid / group_size;
  const int first_m = group * group_m;
  const int gm = min(tiles_m - first_m, group_m);
  const int in_group = pid - group * group_size;
  m0 = (first_m + in_group % gm) * BM;
  n0 = (in_group / gm) * BN;
}

// Persistent kernel: one workgroup per CU.  The tiles of XCD x (workgroups
// x, x+8, ... run there) are the contiguous range [x*per_xcd, (x+1)*per_xcd),
// dealt round-robin to that XCD's workgroups, so the tiles running at once on
// one XCD are neighbours in its L2.  The stage sequence of all of a
// workgroup's tiles is one stream: the DMA ring runs across tile boundaries,
// so a tile's epilogue overlaps the loads of the next tile's first stages.
//
// Epilogue.  gfx9 has a single in-order vector-memory counter, so a global
// load in the epilogue would also wait for the DMA still in flight.  The
// per-token scales, per-channel scales and bias of a tile therefore arrive in
// LDS by the same DMA path, with the tile's first stage (kParamSets buffers,
// indexed by tile), and are read with LDS loads.  Outputs are transposed
// through the ring slot just consumed (free until the next barrier) so every
// store writes full 128-byte row segments.
// One parameter set: [sa f32 x 256][sw f32 x 256][bias as loaded, <= 1 KB][bias f32 x 256].
constexpr int kParamBytes = 1024;  // 256 x 4 bytes: one parameter row of a tile
constexpr int kParamSetBytes = 4 * kParamBytes;
// A tile's parameters are loaded with its first stage, issued kStages stages
// ahead, and read in its epilogue; the set is reloaded kParamSets tiles later.
// With KT stages per tile that reload is issued after the epilogue when
// (kParamSets - 1) * KT >= kStages, for every KT >= 1.
constexpr int kParamSets = kStages + 1;
constexpr int kLdsBytes = kStages * kStageBytes + kParamSets * kParamSetBytes;

// GATED: the bf16 output y feeds out = bf16(residual + bf16(y * gate[indices[m % seq]])).
template <int KIND, int ACT, int OUT_DT, bool ACC_OUT, int WM, int WN, bool GATED = false>
__global__ __launch_bounds__(64 * WM * WN, 1) void gemm_w8a8_kernel(GemmArgs p) {
  typedef Mfma<KIND> T;
  constexpr int kWaves = WM * WN;
  constexpr int FM = BM / WM / 32;               // activation (token) fragments per wave
  constexpr int FN = BN / WN / 32;               // weight (feature) fragments per wave
  constexpr int kRowsPerWave = 256 / kWaves;     // DMA rows per operand per wave
  constexpr int kWaveLoads = kRowsPerWave / 16;  // 1 KB DMA loads per operand per wave
  constexpr int kLoadsPerStage = 2 * kWaveLoads; // per thread
  static_assert(kRowsPerWave % 16 == 0, "DMA rows");
  // epilogue transpose: one 32-row block of the wave's outputs, kRowBytes per row
  constexpr int kRowBytes = FN * 32 * 2;
  constexpr int kRowsPerLine = 256 / kRowBytes;      // rows sharing one 256-byte line of banks
  constexpr int kChunks8 = kRowBytes / 8;            // 8-byte chunks per row
  constexpr int kLanesPerRow = kRowBytes / 16;       // 16-byte chunks per row
  constexpr int kRowsPerRead = 64 / kLanesPerRow;    // rows per 16-byte-per-lane read
  static_assert((kRowBytes == 128 || kRowBytes == 256) && kWaves * 32 * kRowBytes <= kStageBytes,
                "epilogue transpose layout");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kLdsBytes];

  // --- this workgroup's tiles ------------------------------------------------
  const int ntiles = p.tiles_m * p.tiles_n;
  const int xcd = blockIdx.x & 7, local = blockIdx.x >> 3, wgs_per_xcd = gridDim.x >> 3;
  const int t_first = xcd * p.per_xcd + local;
  const int t_end = min((xcd + 1) * p.per_xcd, ntiles);
  const int n_my = t_first < t_end ? (t_end - t_first + wgs_per_xcd - 1) / wgs_per_xcd : 0;
  const int KT = (p.K + BK - 1) / BK;
  const int G = n_my * KT;  // stages of all my tiles
  if (G == 0) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;

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
  // per-tensor scales (stride 0): one uniform value each
  const float sa0 = p.sa_stride ? 0.0f : p.sa[0];
  const float sw0 = p.sw_stride ? 0.0f : p.sw[0];

  // --- global -> LDS DMA ------------------------------------------------------
  // A 16-byte DMA load writes LDS at (wave base + lane * 16), so one wave-load
  // fills 1 KB = 16 rows x 64 bytes.  Wave w fills rows
  // [w * kRowsPerWave, (w + 1) * kRowsPerWave) of both operand tiles; lane l
  // lands on row base + (l >> 2), physical chunk l & 3, i.e. logical chunk
  // (l & 3) ^ ((row >> 2) & 3) = (l & 3) ^ ((l >> 4) & 3), fetched from global.
  const int dma_chunk = (lane & 3) ^ ((lane >> 4) & 3);
  uint32_t offa[kWaveLoads], offw[kWaveLoads];
  int dma_m0 = 0, dma_n0 = 0;
  auto set_dma_tile = [&](int i) {  // row offsets of my i-th tile
    tile_origin(t_first + i * wgs_per_xcd, p.tiles_m, p.tiles_n, p.group_m, dma_m0, dma_n0);
#pragma unroll
    for (int l = 0; l < kWaveLoads; ++l) {
      const int r = wave * kRowsPerWave + l * 16 + (lane >> 2);
      const int ma = dma_m0 + r, nw = dma_n0 + r;
      offa[l] = ma < p.M ? (uint32_t)ma * (uint32_t)p.lda + dma_chunk * 16 : kOutOfRange;
      offw[l] = nw < p.N ? (uint32_t)nw * (uint32_t)p.ldw + dma_chunk * 16 : kOutOfRange;
    }
  };
  // The load stream: the next stage to load is issue_g (slot issue_g %
  // kStages), stage issue_kt of my tile issue_i.  Past my last stage the
  // stream goes on with stages whose loads are all out of range: they write
  // zeros into slots nothing reads, which keeps the stream free of branches.
  int issue_g = 0, issue_kt = 0, issue_i = 0;
  auto issue_params = [&]() {  // a tile's epilogue parameters ride with its first stage
    if (issue_kt != 0 || issue_g >= G) return;
    uint8_t *prm = smem + kStages * kStageBytes + (issue_i % kParamSets) * kParamSetBytes;
    if (wave == 0 && p.sa_stride) dma_load16(rsa, prm, (uint32_t)dma_m0 * 4 + lane * 16);
    if (wave == 1 && p.sw_stride) dma_load16(rsw, prm + kParamBytes, (uint32_t)dma_n0 * 4 + lane * 16);
    if (wave == 2 && p.bias) dma_load16(rb, prm + 2 * kParamBytes, (uint32_t)(dma_n0 * bias_elem) + lane * 16);
  };
  // operand load q (0 .. kLoadsPerStage-1) of stage issue_g
  struct Issue {
    uint8_t *base;
    int k0;
    bool kin;
  };
  auto issue_setup = [&]() {
    const int k0 = issue_kt * BK;
    // K tail and the stages past my last: out of range -> zeros
    return Issue{smem + (issue_g % kStages) * kStageBytes + wave * kRowsPerWave * BK, k0,
                 issue_g < G && k0 + dma_chunk * 16 < p.K};
  };
  auto issue_load = [&](const Issue &is, int q) {
    const int l = q >> 1;
    if (q & 1)
      dma_load16(rw, is.base + kTileBytes + l * 16 * BK, is.kin ? offw[l] + is.k0 : kOutOfRange);
    else
      dma_load16(ra, is.base + l * 16 * BK, is.kin ? offa[l] + is.k0 : kOutOfRange);
  };
  auto issue_advance = [&]() {
    ++issue_g;
    if (++issue_kt == KT) {
      issue_kt = 0;
      if (++issue_i < n_my) set_dma_tile(issue_i);
    }
  };
  auto issue_next = [&]() {  // a whole stage at once (prologue)
    issue_params();
    const Issue is = issue_setup();
#pragma unroll
    for (int q = 0; q < kLoadsPerStage; ++q) issue_load(is, q);
    issue_advance();
  };

  typedef typename T::frag_t frag_t;
  const int row_x = wm * (BM / WM) + (lane & 31);
  const int row_w = wn * (BN / WN) + (lane & 31);
  auto slot_of = [&](int stage) { return smem + (stage % kStages) * kStageBytes; };
  // this thread's loads of stage h (and of the parameter row issued with it)
  // are done once at most the loads of the stages issued after it remain
  // outstanding (the parameter loads only make the count conservative)
  auto wait_stage = [&](int h) {
    const int later = issue_g - 1 - h;
    if (later >= 2) wait_vmcnt<2 * kLoadsPerStage>();
    else if (later == 1) wait_vmcnt<kLoadsPerStage>();
    else wait_vmcnt<0>();
  };

  typename T::acc_t acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = typename T::acc_t{};

  int tile_i = 0, kt = 0;
  // Operand fragments in registers: xf = activation fragments of the stage
  // being multiplied; wf[c] = weight fragments of it, wf[c ^ 1] = those of the
  // next stage.  Each activation fragment is refilled with the next stage's
  // as soon as its last MFMA has been issued, so the LDS reads of stage g+1
  // overlap the MFMAs of stage g within 64 fragment registers.
  frag_t xf[T::kSteps][FM], wf[2][T::kSteps][FN];

  // One stage.  The barrier at the top publishes every wave's DMA of stage
  // g+1 and retires every wave's reads of slot g % kStages, which then takes
  // the DMA of stage g + kStages.  (Past the last stage the reads of "stage
  // g+1" fetch stale LDS that nothing uses.)
  auto stage = [&](int g, int c) {
    wait_stage(g + 1);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): my reads of slot g are done
    lds_barrier();
    issue_params();
    const Issue is = issue_setup();
    const uint8_t *nx = slot_of(g + 1), *nw = nx + kTileBytes;
#pragma unroll
    for (int ks = 0; ks < T::kSteps; ++ks)
#pragma unroll
      for (int f = 0; f < FN; ++f) wf[c ^ 1][ks][f] = T::load(nw, row_w + f * 32, ks, lane);
    // The operand loads of stage g + kStages are spread over the MFMAs: issued
    // together, the workgroup's loads queue up in the address unit, and a wave
    // whose load waits there cannot issue its MFMAs either.
    constexpr int kSlots = T::kSteps * FM;
    constexpr int kEvery = kSlots >= kLoadsPerStage ? kSlots / kLoadsPerStage : 1;
    constexpr int kPerSlot = kSlots >= kLoadsPerStage ? 1 : kLoadsPerStage / kSlots;
    static_assert(kSlots % kLoadsPerStage == 0 || kLoadsPerStage % kSlots == 0, "load spacing");
#pragma unroll
    for (int ks = 0; ks < T::kSteps; ++ks)
#pragma unroll
      for (int j = 0; j < FM; ++j) {
#pragma unroll
        for (int i = 0; i < FN; ++i) acc[i][j] = T::mma(wf[c][ks][i], xf[ks][j], acc[i][j]);
        xf[ks][j] = T::load(nx, row_x + j * 32, ks, lane);
        const int slot = ks * FM + j;
        if (slot % kEvery == 0)
#pragma unroll
          for (int u = 0; u < kPerSlot; ++u) issue_load(is, slot / kEvery * kPerSlot + u);
      }
    // Keep that order in the schedule: the weight reads, then per activation
    // fragment its MFMAs, its refill and (every kEvery fragments) one load.
    // (Left alone the scheduler issues most MFMAs first and the reads of the
    // next stage too late.)
    __builtin_amdgcn_sched_group_barrier(kDsRead, T::kReads * T::kSteps * FN, 0);
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
      __builtin_amdgcn_sched_group_barrier(kMfma, FN * T::kMfmaPerMma, 0);
      __builtin_amdgcn_sched_group_barrier(kDsRead, T::kReads, 0);
      if (k % kEvery == 0) __builtin_amdgcn_sched_group_barrier(kVmemRead, kPerSlot, 0);
    }
    issue_advance();
    if (++kt < KT) return;

    // --- epilogue of my tile tile_i -------------------------------------------
    // acc[i][j] element e: feature n = n0 + wn*(BN/WN) + i*32 + (e/4)*8 + (lane/32)*4 + e%4,
    //                      token   m = m0 + wm*(BM/WM) + j*32 + lane%32.
    int m0, n0;
    tile_origin(t_first + tile_i * wgs_per_xcd, p.tiles_m, p.tiles_n, p.group_m, m0, n0);
    uint8_t *prm = smem + kStages * kStageBytes + (tile_i % kParamSets) * kParamSetBytes;
    float *psa = reinterpret_cast<float *>(prm);
    float *psw = reinterpret_cast<float *>(prm + kParamBytes);
    float *pbf = reinterpret_cast<float *>(prm + 3 * kParamBytes);
    // The transpose area: this wave's 4 KB of slot (g+1) % kStages, whose
    // fragments every wave must have read first.  Its next DMA is issued after
    // the barrier of stage g+1.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    lds_barrier();
    // Parameters as float rows: per-tensor scales broadcast, bias converted
    // (zeros without one), so the loops below read them without branches.
    if (tid < 256) {
      if (!p.sa_stride) psa[tid] = sa0;
    } else {
      const int t = tid - 256;
      if (!p.sw_stride) psw[t] = sw0;
      pbf[t] = p.bias ? bias_at(prm + 2 * kParamBytes, p.bias_dtype, t) : 0.0f;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    lds_barrier();
    uint8_t *xb = smem + ((g + 1) % kStages) * kStageBytes + wave * 32 * kRowBytes;
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int ml = wm * (BM / WM) + j * 32 + (lane & 31);
      const float sam = psa[ml];
      const int wrow = lane & 31;
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int nl = wn * (BN / WN) + i * 32 + gq * 8 + (lane >> 5) * 4;
          const f32x4 sw4 = *reinterpret_cast<const f32x4 *>(psw + nl);
          const f32x4 b4 = *reinterpret_cast<const f32x4 *>(pbf + nl);
          const float swv[4] = {sw4.x, sw4.y, sw4.z, sw4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
          float y[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a = T::to_f32(acc[i][j][gq * 4 + e]);
            y[e] = __builtin_fmaf(a, sam * swv[e], bv[e]);
            if constexpr (ACT == XGEN_ACT_GELU_TANH) y[e] = gelu_tanh(round_out<OUT_DT>(y[e]));
          }
          // row wrow, 8-byte chunk c8 (4 outputs) of the wave's row, XOR-swizzled
          // by the row's index among the rows of its bank line: conflict-free
          // 64-bit writes
          const int c8 = i * 8 + gq * 2 + (lane >> 5);
          *reinterpret_cast<u32x2 *>(xb + wrow * kRowBytes + ((c8 ^ ((wrow / kRowsPerLine) & (kChunks8 - 1))) << 3)) =
              u32x2{pack_out<OUT_DT>(y[0], y[1]), pack_out<OUT_DT>(y[2], y[3])};
          if constexpr (ACC_OUT) {
            const int m = m0 + ml, n = n0 + nl;
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
        }
      // read back kRowsPerRead whole rows per instruction, 16 bytes per lane, and
      // store them as full row segments (LDS operations of a wave complete in order)
#pragma unroll
      for (int q = 0; q < 32 / kRowsPerRead; ++q) {
        const int row = q * kRowsPerRead + lane / kLanesPerRow, c16 = lane % kLanesPerRow;
        const int sw4 = (row / kRowsPerLine) & (kChunks8 - 1);
        u32x4 v = *reinterpret_cast<const u32x4 *>(xb + row * kRowBytes + ((c16 ^ (sw4 >> 1)) << 4));
        if (sw4 & 1) v = u32x4{v.z, v.w, v.x, v.y};
        const int m = m0 + wm * (BM / WM) + j * 32 + row;
        const int n = n0 + wn * (BN / WN) + c16 * 8;
        if (m < p.M && n < p.N) {
          if constexpr (GATED) {
            const int64_t gi = p.indices[(uint32_t)m % p.seq];
            if (gi >= 0 && gi < p.gate_rows) {
              const u32x4 r = *reinterpret_cast<const u32x4 *>(p.residual + ((int64_t)m * p.ld_residual + n) * 2);
              const u32x4 t = *reinterpret_cast<const u32x4 *>(p.gate + (gi * p.gate_stride + n) * 2);
              v = gate_residual8(r, v, t);
            } else {
              v = u32x4{0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};  // index outside the table: NaN
            }
          }
          *reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(p.out) + (int64_t)m * p.ldo + n) = v;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = typename T::acc_t{};
    kt = 0;
    ++tile_i;
  };

  set_dma_tile(0);
#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) issue_next();
  wait_stage(0);
  lds_barrier();
  issue_next();
  {
    const uint8_t *sx = slot_of(0), *sw = sx + kTileBytes;
#pragma unroll
    for (int ks = 0; ks < T::kSteps; ++ks) {
#pragma unroll
      for (int f = 0; f < FN; ++f) wf[0][ks][f] = T::load(sw, row_w + f * 32, ks, lane);
#pragma unroll
      for (int f = 0; f < FM; ++f) xf[ks][f] = T::load(sx, row_x + f * 32, ks, lane);
    }
  }
  // two stages per trip so the weight-fragment buffers alternate without copies
  for (int g = 0; g < G; g += 2) {
    stage(g, 0);
    if (g + 1 < G) stage(g + 1, 1);
  }
  // the loads of the stages past my last may still be writing LDS
  wait_vmcnt<0>();
}

// one persistent workgroup per CU (a multiple of the 8 XCDs), never more than the tiles need
dim3 gemm_grid(const GemmArgs &a) {
  const int ntiles = a.tiles_m * a.tiles_n;
  int wgs = device_cu_count() / 8 * 8;
  const int need = ((ntiles + 7) / 8) * 8;
  if (wgs > need) wgs = need;
  if (wgs < 8) wgs = 8;
  return dim3((unsigned)wgs);
}

template <int KIND, int ACT, int OUT_DT>
void launch_gemm(const GemmArgs &a, bool acc_out, hipStream_t stream) {
  const dim3 grid = gemm_grid(a), block(64 * kWavesM * kWavesN);
  if (acc_out) gemm_w8a8_kernel<KIND, ACT, OUT_DT, true, kWavesM, kWavesN><<<grid, block, 0, stream>>>(a);
  else gemm_w8a8_kernel<KIND, ACT, OUT_DT, false, kWavesM, kWavesN><<<grid, block, 0, stream>>>(a);
}

template <int KIND>
void launch_gemm_gated(const GemmArgs &a, hipStream_t stream) {
  gemm_w8a8_kernel<KIND, XGEN_ACT_NONE, XGEN_DTYPE_BF16, false, kWavesM, kWavesN, true>
      <<<gemm_grid(a), dim3(64 * kWavesM * kWavesN), 0, stream>>>(a);
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
  }
  const int64_t a_bytes = (M - 1) * lda + K, w_bytes = (N - 1) * ldw + K;
  if (a_bytes >= (int64_t)kOutOfRange || w_bytes >= (int64_t)kOutOfRange)
    return fail(XGEN_ERR_UNSUPPORTED, "%s: operands above 2 GiB", fn);

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
  g.tiles_m = (int)((M + BM - 1) / BM);
  g.tiles_n = (int)((N + BN - 1) / BN);
  g.per_xcd = (g.tiles_m * g.tiles_n + 7) / 8;
  // The 32 tiles one XCD runs at once span group_m tile-rows.  Measured at
  // M=15,624: 4 rows beat 8 for outputs of 24-63 tile-columns (QKV N=9,216
  // 0.9%, FFN up N=12,288 2.8% faster); 8 beat 4 for FFN down's 12 (1.7%), and
  // for H3's FFN up (N=28,672: 112 tile-columns, 2.5%); 2, 3, 6, 12 and 16
  // were no better.
  g.group_m = g.tiles_n >= 24 && g.tiles_n < 64 ? 4 : 8;
  g.a_bytes = (uint32_t)a_bytes;
  g.w_bytes = (uint32_t)w_bytes;
  g.residual = static_cast<const uint8_t *>(gp.residual);
  g.ld_residual = gp.ld_residual;
  g.gate = static_cast<const uint8_t *>(gp.gate);
  g.gate_stride = gp.gate_stride;
  g.gate_rows = gp.gate_rows;
  g.indices = gp.indices;
  g.seq = (uint32_t)gp.seq;
  const bool with_acc = acc_out != nullptr;
  if (gated) {
    launch_gemm_gated<KIND>(g, stream);
  } else if (activation == XGEN_ACT_NONE) {
    if (out_dtype == XGEN_DTYPE_BF16) launch_gemm<KIND, XGEN_ACT_NONE, XGEN_DTYPE_BF16>(g, with_acc, stream);
    else launch_gemm<KIND, XGEN_ACT_NONE, XGEN_DTYPE_F16>(g, with_acc, stream);
  } else {
    if (out_dtype == XGEN_DTYPE_BF16) launch_gemm<KIND, XGEN_ACT_GELU_TANH, XGEN_DTYPE_BF16>(g, with_acc, stream);
    else launch_gemm<KIND, XGEN_ACT_GELU_TANH, XGEN_DTYPE_F16>(g, with_acc, stream);
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
