// Single-instruction probes of gfx950's FP8 matrix arithmetic, run by
// tests/golden/make_mfma_probes.py to write the fixture that pins
// oracle/mfma_model.c.  Test tooling: nothing in xgen_amd uses it.
//
// One wave per 32x32x64 problem: A, B [n][32][64] e4m3fn bytes, C, D
// [n][32][32] float, D = C + A.B^T by the chosen instruction form.  Lane l
// holds row l % 32 and K bytes 32*(l/32) .. +31 (the GEMM kernel's layout);
// output element e of lane l is D[8*(e/4) + 4*(l/32) + e%4][l % 32].
#include <hip/hip_runtime.h>
#include <stdint.h>
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ float dec_e4m3(uint32_t b) {
  uint32_t e = (b >> 3) & 15, m = b & 7;
  float v = e == 0 ? (float)m * 0.001953125f : __builtin_ldexpf(1.0f + m * 0.125f, (int)e - 7);
  return (b & 0x80) ? -v : v;
}

template <int V>
__global__ __launch_bounds__(64) void probe_kernel(const uint8_t *A, const uint8_t *B, const float *C, float *D) {
  const int p = blockIdx.x, lane = threadIdx.x, row = lane & 31, h = lane >> 5;
  const uint8_t *a = A + (size_t)p * 2048 + row * 64;
  const uint8_t *b = B + (size_t)p * 2048 + row * 64;
  const float *c = C + (size_t)p * 1024;
  float *d = D + (size_t)p * 1024;
  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = c[(8 * (e / 4) + 4 * h + (e % 4)) * 32 + row];
  if constexpr (V == 0 || V == 1) {
    i32x8 fa, fb;
    for (int i = 0; i < 8; ++i) {
      fa[i] = *reinterpret_cast<const int32_t *>(a + 32 * h + 4 * i);
      fb[i] = *reinterpret_cast<const int32_t *>(b + 32 * h + 4 * i);
    }
    if constexpr (V == 0) acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa, fb, acc, 0, 0, 0, 0, 0, 0);
    else acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa, fb, acc, 0, 0, 0, 127, 0, 127);
  } else if constexpr (V == 2) {  // gfx942-style 32x32x16 fp8, four instructions (k = 16s + 8h + 0..7)
    for (int s = 0; s < 4; ++s) {
      long fa = *reinterpret_cast<const long *>(a + 16 * s + 8 * h);
      long fb = *reinterpret_cast<const long *>(b + 16 * s + 8 * h);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_fp8_fp8(fa, fb, acc, 0, 0, 0);
    }
  } else if constexpr (V == 3) {  // bf16 32x32x16 on decoded operands, four instructions
    for (int s = 0; s < 4; ++s) {
      bf16x8 fa, fb;
      for (int i = 0; i < 8; ++i) {
        fa[i] = (__bf16)dec_e4m3(a[16 * s + 8 * h + i]);
        fb[i] = (__bf16)dec_e4m3(b[16 * s + 8 * h + i]);
      }
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa, fb, acc, 0, 0, 0);
    }
  } else if constexpr (V == 5) {  // 16x16x128 f8f6f4: k 0..63 real, 64..127 zero
    // lane l: row l%16, k bytes 32*(l/16) .. +31 (both operands)
    const int r16 = lane & 15, q = lane >> 4;
    f32x16 res = {};
    for (int bi = 0; bi < 2; ++bi)
      for (int bj = 0; bj < 2; ++bj) {
        i32x8 fa = {}, fb = {};
        if (q < 2)
          for (int i = 0; i < 8; ++i) {
            fa[i] = *reinterpret_cast<const int32_t *>(A + (size_t)p * 2048 + (16 * bi + r16) * 64 + 32 * q + 4 * i);
            fb[i] = *reinterpret_cast<const int32_t *>(B + (size_t)p * 2048 + (16 * bj + r16) * 64 + 32 * q + 4 * i);
          }
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        f32x4 cc;
        for (int e = 0; e < 4; ++e) cc[e] = C[(size_t)p * 1024 + (16 * bi + 4 * q + e) * 32 + 16 * bj + r16];
        cc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fa, fb, cc, 0, 0, 0, 0, 0, 0);
        for (int e = 0; e < 4; ++e) D[(size_t)p * 1024 + (16 * bi + 4 * q + e) * 32 + 16 * bj + r16] = cc[e];
      }
    return;
  } else if constexpr (V == 4) {  // 32x32x64 with C = 0, then v_add into C (split accumulation)
    i32x8 fa, fb;
    for (int i = 0; i < 8; ++i) {
      fa[i] = *reinterpret_cast<const int32_t *>(a + 32 * h + 4 * i);
      fb[i] = *reinterpret_cast<const int32_t *>(b + 32 * h + 4 * i);
    }
    f32x16 z = {};
    z = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa, fb, z, 0, 0, 0, 0, 0, 0);
    for (int e = 0; e < 16; ++e) acc[e] = acc[e] + z[e];
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) d[(8 * (e / 4) + 4 * h + (e % 4)) * 32 + row] = acc[e];
}

// bf16 bits of every e4m3fn code through v_cvt_scalef32_pk_bf16_fp8 (scale 1),
// the conversion of the GEMM's exact-accumulation kind.  Each packed result is
// stored as the whole 32-bit register, as the GEMM hands it to the MFMA.
__global__ void decode_kernel(uint32_t *out) {
  const int t = threadIdx.x;  // 128 threads: codes 2t, 2t+1
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  const int word = (2 * t) | ((2 * t + 1) << 8) | ((2 * t) << 16) | ((2 * t + 1) << 24);
  out[t] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, 1.0f, false));
  out[128 + t] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, 1.0f, true));
}

extern "C" int decode_all(void *out, hipStream_t s) {
  decode_kernel<<<1, 128, 0, s>>>((uint32_t *)out);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" int probe(int variant, const void *A, const void *B, const void *C, void *D, int n, hipStream_t s) {
  const auto a = (const uint8_t *)A, b = (const uint8_t *)B;
  const auto c = (const float *)C;
  auto d = (float *)D;
  switch (variant) {
    case 0: probe_kernel<0><<<n, 64, 0, s>>>(a, b, c, d); break;
    case 1: probe_kernel<1><<<n, 64, 0, s>>>(a, b, c, d); break;
    case 2: probe_kernel<2><<<n, 64, 0, s>>>(a, b, c, d); break;
    case 3: probe_kernel<3><<<n, 64, 0, s>>>(a, b, c, d); break;
    case 4: probe_kernel<4><<<n, 64, 0, s>>>(a, b, c, d); break;
    case 5: probe_kernel<5><<<n, 64, 0, s>>>(a, b, c, d); break;
    default: return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
