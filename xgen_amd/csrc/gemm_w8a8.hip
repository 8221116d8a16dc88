// W8A8 GEMM with fused per-token x per-channel dequant, bias and optional
// GELU-tanh epilogue, on gfx950 matrix cores.
//
//   FP8 : v_mfma_f32_32x32x64_f8f6f4 (e4m3fn x e4m3fn -> fp32)
//         replaces torch._scaled_mm at x_base/x_base/operator/h3_fp8.py:63-66
//   INT8: v_mfma_i32_32x32x32_i8      (int8 x int8 -> exact int32)
//         replaces torch_npu.npu_quant_matmul at x_base/x_base/operator/matmul.py:63-64
//
// out[m, n] = act(cvt(acc[m, n] * (sa[m] * sw[n]) + bias[n])),  acc = sum_k a[m,k] w[n,k]
//
// Tiling: a 256x256 output tile per workgroup of 4 waves (2x2, 128x128 per
// wave = 4x4 MFMA 32x32 blocks, accumulators in AGPRs), K in steps of 128
// bytes, double-buffered in LDS (2 stages x (32 KB activations + 32 KB
// weights)).  Global loads are bounds-checked buffer loads (rows past M/N read
// as zero), staged through registers and written to LDS with the 16-byte chunk
// index XOR-swizzled by (row & 7), so both the 128-bit LDS writes and the
// 128-bit MFMA-operand reads are bank-conflict free.
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

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int kThreads = 256;
constexpr int kTileBytes = 256 * BK;  // one operand tile per stage
constexpr int kGroupM = 8;
constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit dword format (gfx9)
constexpr uint32_t kOutOfRange = 0x80000000u;

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
  uint32_t a_bytes, w_bytes;
};

template <bool FP8>
struct Mfma;

template <>
struct Mfma<true> {
  typedef f32x16 acc_t;
  typedef i32x8 frag_t;
  static constexpr int kSteps = BK / 64;  // 32x32x64
  static __device__ __forceinline__ frag_t load(const uint8_t *tile, int row, int ks, int lane) {
    const int c0 = ks * 4 + (lane >> 5) * 2;
    const int sw = lane & 7;
    const u32x4 lo = *reinterpret_cast<const u32x4 *>(tile + row * BK + ((c0 ^ sw) << 4));
    const u32x4 hi = *reinterpret_cast<const u32x4 *>(tile + row * BK + (((c0 + 1) ^ sw) << 4));
    return frag_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  }
  static __device__ __forceinline__ acc_t mma(const frag_t &w, const frag_t &x, const acc_t &c) {
    // cbsz = blgp = 0: both operands e4m3; zero scale operands: unscaled MFMA.
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, x, c, 0, 0, 0, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f32(float v) { return v; }
};

template <>
struct Mfma<false> {
  typedef i32x16 acc_t;
  typedef i32x4 frag_t;
  static constexpr int kSteps = BK / 32;  // 32x32x32
  static __device__ __forceinline__ frag_t load(const uint8_t *tile, int row, int ks, int lane) {
    const int c = ks * 2 + (lane >> 5);
    const u32x4 v = *reinterpret_cast<const u32x4 *>(tile + row * BK + ((c ^ (lane & 7)) << 4));
    return frag_t{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
  }
  static __device__ __forceinline__ acc_t mma(const frag_t &w, const frag_t &x, const acc_t &c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(w, x, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f32(int v) { return (float)v; }
};

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

__device__ __forceinline__ void load_bias4(const void *bias, int dtype, int n, float (&b)[4]) {
  if (dtype == XGEN_DTYPE_F32) {
    const f32x4 v = *reinterpret_cast<const f32x4 *>(static_cast<const float *>(bias) + n);
    b[0] = v.x; b[1] = v.y; b[2] = v.z; b[3] = v.w;
  } else {
    const u32x2 v = *reinterpret_cast<const u32x2 *>(static_cast<const uint16_t *>(bias) + n);
    if (dtype == XGEN_DTYPE_BF16) {
      b[0] = Half2<XGEN_DTYPE_BF16>::lo(v.x); b[1] = Half2<XGEN_DTYPE_BF16>::hi(v.x);
      b[2] = Half2<XGEN_DTYPE_BF16>::lo(v.y); b[3] = Half2<XGEN_DTYPE_BF16>::hi(v.y);
    } else {
      b[0] = Half2<XGEN_DTYPE_F16>::lo(v.x); b[1] = Half2<XGEN_DTYPE_F16>::hi(v.x);
      b[2] = Half2<XGEN_DTYPE_F16>::lo(v.y); b[3] = Half2<XGEN_DTYPE_F16>::hi(v.y);
    }
  }
}

template <bool FP8, int ACT, int OUT_DT, bool ACC_OUT>
__global__ __launch_bounds__(kThreads, 1) void gemm_w8a8_kernel(GemmArgs p) {
  typedef Mfma<FP8> T;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * 2 * kTileBytes];

  // --- tile selection (XCD-contiguous ranges, grouped rows) ----------------
  const int bid = blockIdx.x;
  const int pid = (bid & 7) * p.per_xcd + (bid >> 3);
  if (pid >= p.tiles_m * p.tiles_n) return;
  const int group_size = kGroupM * p.tiles_n;
  const int group = pid / group_size;
  const int first_m = group * kGroupM;
  const int gm = min(p.tiles_m - first_m, kGroupM);
  const int in_group = pid - group * group_size;
  const int m0 = (first_m + in_group % gm) * BM;
  const int n0 = (in_group / gm) * BN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(p.a), (short)0, (int)p.a_bytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(p.w), (short)0, (int)p.w_bytes, kBufferFlags);

  // --- global -> LDS assignment: 8 rows x one 16-byte chunk per operand ---
  const int lc = tid & 7, lr = tid >> 3;
  uint32_t offa[8], offw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int ma = m0 + lr + 32 * i, nw = n0 + lr + 32 * i;
    offa[i] = ma < p.M ? (uint32_t)ma * (uint32_t)p.lda + lc * 16 : kOutOfRange;
    offw[i] = nw < p.N ? (uint32_t)nw * (uint32_t)p.ldw + lc * 16 : kOutOfRange;
  }
  const int lds_w = lr * BK + ((lc ^ (lr & 7)) << 4);  // + i * 32 * BK

  u32x4 ga[8], gw[8];
  auto load_global = [&](int k0) {
    const bool kin = k0 + lc * 16 < p.K;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ga[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, kin ? offa[i] + k0 : kOutOfRange, 0, 0);
      gw[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, kin ? offw[i] + k0 : kOutOfRange, 0, 0);
    }
  };
  auto store_lds = [&](int stage) {
    uint8_t *sa = smem + stage * 2 * kTileBytes;
    uint8_t *sb = sa + kTileBytes;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      *reinterpret_cast<u32x4 *>(sa + lds_w + i * 32 * BK) = ga[i];
      *reinterpret_cast<u32x4 *>(sb + lds_w + i * 32 * BK) = gw[i];
    }
  };

  typename T::acc_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = typename T::acc_t{};

  const int row_x = wm * 128 + (lane & 31);
  const int row_w = wn * 128 + (lane & 31);
  const int KT = (p.K + BK - 1) / BK;

  load_global(0);
  store_lds(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_global((kt + 1) * BK);
    const uint8_t *sx = smem + cur * 2 * kTileBytes;
    const uint8_t *sw = sx + kTileBytes;
#pragma unroll
    for (int ks = 0; ks < T::kSteps; ++ks) {
      typename T::frag_t fw[4], fx[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        fw[f] = T::load(sw, row_w + f * 32, ks, lane);
        fx[f] = T::load(sx, row_x + f * 32, ks, lane);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = T::mma(fw[i], fx[j], acc[i][j]);
    }
    if (kt + 1 < KT) store_lds(cur ^ 1);
    __syncthreads();
  }

  // --- epilogue -------------------------------------------------------------
  // acc[i][j] element e: feature n = n0 + wn*128 + i*32 + (e/4)*8 + (lane/32)*4 + e%4,
  //                      token   m = m0 + wm*128 + j*32 + lane%32.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = m0 + wm * 128 + j * 32 + (lane & 31);
    if (m >= p.M) continue;
    const float sam = p.sa[(int64_t)m * p.sa_stride];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int n = n0 + wn * 128 + i * 32 + gq * 8 + (lane >> 5) * 4;
        if (n >= p.N) continue;
        float swv[4], bv[4] = {0.f, 0.f, 0.f, 0.f}, y[4];
        if (p.sw_stride) {
          const f32x4 s4 = *reinterpret_cast<const f32x4 *>(p.sw + n);
          swv[0] = s4.x; swv[1] = s4.y; swv[2] = s4.z; swv[3] = s4.w;
        } else {
          swv[0] = swv[1] = swv[2] = swv[3] = p.sw[0];
        }
        if (p.bias) load_bias4(p.bias, p.bias_dtype, n, bv);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = T::to_f32(acc[i][j][gq * 4 + e]);
          y[e] = __builtin_fmaf(a, sam * swv[e], bv[e]);
          if constexpr (ACT == XGEN_ACT_GELU_TANH) y[e] = gelu_tanh(round_out<OUT_DT>(y[e]));
        }
        const u32x2 o = {pack_out<OUT_DT>(y[0], y[1]), pack_out<OUT_DT>(y[2], y[3])};
        *reinterpret_cast<u32x2 *>(static_cast<uint16_t *>(p.out) + (int64_t)m * p.ldo + n) = o;
        if constexpr (ACC_OUT) {
          if constexpr (FP8) {
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
  }
}

template <bool FP8, int ACT, int OUT_DT>
void launch_gemm(const GemmArgs &a, bool acc_out, hipStream_t stream) {
  const int tiles = a.tiles_m * a.tiles_n;
  const dim3 grid((unsigned)(a.per_xcd * 8)), block(kThreads);
  (void)tiles;
  if (acc_out) gemm_w8a8_kernel<FP8, ACT, OUT_DT, true><<<grid, block, 0, stream>>>(a);
  else gemm_w8a8_kernel<FP8, ACT, OUT_DT, false><<<grid, block, 0, stream>>>(a);
}

template <bool FP8>
int gemm_entry(const char *fn, const void *a, int64_t lda, const void *w, int64_t ldw, int64_t M,
               int64_t N, int64_t K, const float *sa, int64_t sa_stride, const float *sw,
               int64_t sw_stride, const void *bias, int bias_dtype, int activation, void *out,
               int out_dtype, int64_t ldo, void *acc_out, hipStream_t stream) {
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
  if (ldo % 4 || (reinterpret_cast<uintptr_t>(out) & 7u))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: output rows must be 8-byte aligned", fn);
  if ((bias && (reinterpret_cast<uintptr_t>(bias) & 15u)) || (sw_stride && !aligned16(sw)) ||
      (acc_out && !aligned16(acc_out)))
    return fail(XGEN_ERR_UNSUPPORTED, "%s: bias, weight scale and accumulator buffers must be 16-byte aligned", fn);
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
  g.a_bytes = (uint32_t)a_bytes;
  g.w_bytes = (uint32_t)w_bytes;
  const bool with_acc = acc_out != nullptr;
  if (activation == XGEN_ACT_NONE) {
    if (out_dtype == XGEN_DTYPE_BF16) launch_gemm<FP8, XGEN_ACT_NONE, XGEN_DTYPE_BF16>(g, with_acc, stream);
    else launch_gemm<FP8, XGEN_ACT_NONE, XGEN_DTYPE_F16>(g, with_acc, stream);
  } else {
    if (out_dtype == XGEN_DTYPE_BF16) launch_gemm<FP8, XGEN_ACT_GELU_TANH, XGEN_DTYPE_BF16>(g, with_acc, stream);
    else launch_gemm<FP8, XGEN_ACT_GELU_TANH, XGEN_DTYPE_F16>(g, with_acc, stream);
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
  return gemm_entry<true>("xgen_scaled_mm_fp8", a, lda, w, ldw, M, N, K, a_scale, a_scale_stride,
                          w_scale, w_scale_stride, bias, bias_dtype, activation, out, out_dtype, ldo,
                          acc_out, stream);
}

extern "C" int xgen_quant_matmul_int8(const void *a, int64_t lda, const void *w, int64_t ldw,
                                      int64_t M, int64_t N, int64_t K, const float *pertoken_scale,
                                      int64_t pertoken_scale_stride, const float *w_scale,
                                      int64_t w_scale_stride, const void *bias, int bias_dtype,
                                      int activation, void *out, int out_dtype, int64_t ldo,
                                      int32_t *acc_out, hipStream_t stream) {
  return gemm_entry<false>("xgen_quant_matmul_int8", a, lda, w, ldw, M, N, K, pertoken_scale,
                           pertoken_scale_stride, w_scale, w_scale_stride, bias, bias_dtype,
                           activation, out, out_dtype, ldo, acc_out, stream);
}
