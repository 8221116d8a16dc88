/*
 * xgen_amd — C ABI of the MI355X (gfx950) quantized DiT linear path.
 *
 * Every entry point takes plain device pointers, element counts and strides
 * (in elements), and the HIP stream to launch on.  Nothing here allocates,
 * frees or synchronizes; outputs are caller-owned.  Each call validates its
 * arguments on the host before any HIP call and returns XGEN_OK or an error
 * code; xgen_last_error() returns a per-thread message for the last failure.
 *
 * Dtype codes (XGEN_DTYPE_*) name element types of the buffers:
 *   BF16, F16, F32 (IEEE), E4M3 (OCP float8 e4m3fn), I8, I32.
 *
 * Row convention: a matrix [rows, cols] with leading dimension ld (elements
 * between the starts of consecutive rows); the last dimension is contiguous.
 *
 * Each declaration cites the reference interface it replaces
 * (paths relative to the reference repository root).
 */
#ifndef XGEN_AMD_H
#define XGEN_AMD_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XGEN_ABI_VERSION 1

/* status codes */
#define XGEN_OK 0
#define XGEN_ERR_INVALID_ARGUMENT 1 /* null pointer, negative size, unknown code */
#define XGEN_ERR_UNSUPPORTED 2      /* valid request outside the kernels' limits */
#define XGEN_ERR_HIP 3              /* the HIP runtime reported a launch error */

/* dtype codes */
#define XGEN_DTYPE_BF16 0
#define XGEN_DTYPE_F16 1
#define XGEN_DTYPE_F32 2
#define XGEN_DTYPE_E4M3 3
#define XGEN_DTYPE_I8 4
#define XGEN_DTYPE_I32 5
#define XGEN_DTYPE_NONE (-1)

/* widest SwiGLU half (F) of xgen_swiglu_quant: H3's F = 14,336 fits */
#define XGEN_SWIGLU_MAX_HALF 16384

/* widest row (head_dim) of the FP8 wire codec (the reference takes any multiple of 4) */
#define XGEN_WIRE_MAX_WIDTH 1024

/* normalisation kinds for xgen_norm_affine_quant */
#define XGEN_NORM_LAYER 0 /* (x - mean) * rsqrt(var + eps), biased variance */
#define XGEN_NORM_RMS 1   /* x * rsqrt(mean(x^2) + eps) */
/* OR-ed into norm_kind: scale_table holds bf16(1 + scale) (xgen_adaln_one_plus) */
#define XGEN_NORM_SCALE_ONE_PLUS 0x100

/* GEMM epilogue activations */
#define XGEN_ACT_NONE 0
#define XGEN_ACT_GELU_TANH 1 /* out = bf16(gelu_tanh(bf16(linear))) */

/* Largest row width of the fused norm kernel (the reference limit,
 * x_base/x_base/operator/npu_fusion/capabilities.py:7, is 6144). */
#define XGEN_NORM_MAX_WIDTH 8192

int xgen_abi_version(void);
const char *xgen_status_string(int status);
/* Message of the last failing call on the calling host thread ("" if none). */
const char *xgen_last_error(void);

/*
 * Per-row FP8 (e4m3fn) or INT8 dynamic quantization of a BF16/F16 matrix.
 *
 * out_dtype == XGEN_DTYPE_E4M3 — the per-tensor arithmetic of
 *   quantize_per_tensor, x_base/x_base/operator/h3_fp8.py:9-12, applied to
 *   each row r:  s[r] = max(amax_r / 448, FLT_MIN);
 *   q[r,c] = e4m3fn_rne(clamp(x[r,c] / s[r], -448, 448)).
 * out_dtype == XGEN_DTYPE_I8 — torch_npu.npu_dynamic_quant as called at
 *   x_base/x_base/operator/matmul.py:60, with the arithmetic the reference
 *   restates in npu_fusion/f2bc/op_kernel/f2bc_kernel.asc:89-107:
 *   s[r] = amax_r * fl(1/127); alpha = fl(127 / amax_r);
 *   q[r,c] = rint_half_even(fl(x[r,c] * alpha)); a zero row gives q = 0 and
 *   s = 0 (npu_fusion/f1b/op_kernel/swiglu_quant_kernel.asc:72-75).
 * amax propagates NaN. q is [rows, cols] with leading dimension ldq; scale is
 * float32 [rows].
 */
int xgen_quantize_rows(int in_dtype, const void *x, int64_t rows, int64_t cols, int64_t ldx,
                       int out_dtype, void *q, int64_t ldq, float *scale, hipStream_t stream);

/*
 * xgen_quantize_rows of dtype(gelu_tanh(x)) (dtype = in_dtype) in the same single
 * pass: the FFN's GELU-tanh and the down-projection's per-token input quantization
 * (diffusers FeedForward "gelu-approximate" between the two linears,
 * x_diffusers/x_diffusers/framework/transformer/hunyuan.py:358; the reference
 * materializes the GELU output and its next linear quantizes it).  The GELU is the
 * one the GEMM epilogue applies with XGEN_ACT_GELU_TANH, so an up-projection
 * without it followed by this gives the bytes and scales of the up-projection
 * with it followed by xgen_quantize_rows.  Arguments as xgen_quantize_rows.
 */
int xgen_quantize_rows_gelu(int in_dtype, const void *x, int64_t rows, int64_t cols, int64_t ldx,
                            int out_dtype, void *q, int64_t ldq, float *scale, hipStream_t stream);

/*
 * NaN-propagating max |x| over a contiguous BF16/F16 tensor of numel elements
 * (activation_abs_peak, x_base/x_base/operator/h3_abs_peak.py:21-25).
 * peak: one float32 on the device.  workspace: device memory of at least
 * xgen_abs_peak_workspace_bytes(numel) bytes (partial peaks).
 */
size_t xgen_abs_peak_workspace_bytes(int64_t numel);
int xgen_abs_peak(int in_dtype, const void *x, int64_t numel, float *peak, void *workspace,
                  size_t workspace_bytes, hipStream_t stream);

/*
 * Per-tensor FP8 activation scale: scale = max(abs_peak(x) / 448, FLT_MIN)
 * (quantize_activation, x_base/x_base/operator/h3_fp8_quant.py:19).
 * Same workspace as xgen_abs_peak.
 */
int xgen_fp8_tensor_scale(int in_dtype, const void *x, int64_t numel, float *scale,
                          void *workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * xgen_fp8_tensor_scale without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid hipMalloc).  No counterpart in the reference: an MI355X-side variant
 * of the entry point above.  Its partial maxima live in a file-scope device
 * array of the library (4 KB per GPU, kept for the life of the process), whose
 * address is resolved on the first call on each device (the current device,
 * which must be the stream's).  It calls no hipMalloc / hipFree.  Every call
 * on one GPU shares that array: calls that overlap on one GPU (concurrent
 * streams, threads) race and must be serialised by the caller.  Arguments and
 * results as xgen_fp8_tensor_scale; any numel > 0 fits the scratch.
 */
int xgen_fp8_tensor_scale_noalloc(int in_dtype, const void *x, int64_t numel, float *scale, hipStream_t stream);

/*
 * FP8 pack with a device-resident per-tensor scale
 * (_pack, x_base/x_base/operator/h3_fp8_quant.py:9-15):
 * q[i] = e4m3fn_rne(clamp(x[i] / scale[0], -448, 448)) over numel contiguous elements.
 */
int xgen_fp8_pack(int in_dtype, const void *x, int64_t numel, const float *scale, void *q,
                  hipStream_t stream);

/*
 * Fused normalisation + AdaLN-table modulation + per-row quantization
 * (torch.ops.h3_phaa_nq2.fused, npu_fusion/f2_nq2/op_extension/nq2_queued.asc:53-61,
 *  kernel npu_fusion/f2bc/op_kernel/f2bc_kernel.asc:57-107; LayerNorm form of
 *  x_diffusers/x_diffusers/framework/transformer/hunyuan.py:390-393).
 *
 * x: BF16 [batch, seq, width], element (b, s, c) at x[b*x_stride_batch + s*x_stride_seq + c].
 * Row r = b*seq + s uses table row g = indices[s] (int64, 0 <= g < table_rows):
 *   n    = bf16(norm(x_r) [* weight])          norm_kind LAYER or RMS, fp32 math
 *   f    = bf16(1 + scale_table[g])   (scale_table[g] itself with XGEN_NORM_SCALE_ONE_PLUS in norm_kind)
 *   m    = bf16(bf16(n * f) + shift_table[g])
 *   q[r] = per-row quantization of m (out_dtype E4M3 or I8, as xgen_quantize_rows)
 * norm_weight: NULL (no affine) or [width] of dtype BF16/F32.
 * scale_table/shift_table: BF16 [table_rows, width], rows scale_row_stride /
 * shift_row_stride elements apart.  q: [batch*seq, width] contiguous;
 * token_scale: float32 [batch*seq].  normed_out: NULL or BF16 [batch*seq, width]
 * receiving m (the pre-quantization row; the reference's debug output,
 * f2bc_kernel.asc:86).  An out-of-range index yields q = NaN bytes (E4M3) or 0
 * (I8) and a NaN scale for that row; nothing out of bounds is read.
 */
int xgen_norm_affine_quant(const void *x, int64_t batch, int64_t seq, int64_t width,
                           int64_t x_stride_batch, int64_t x_stride_seq, int norm_kind,
                           const void *norm_weight, int norm_weight_dtype, float eps,
                           const void *scale_table, int64_t scale_row_stride,
                           const void *shift_table, int64_t shift_row_stride, int64_t table_rows,
                           const int64_t *indices, int out_dtype, void *q, float *token_scale,
                           void *normed_out, hipStream_t stream);

/*
 * FP8 W8A8 GEMM with fused dequant epilogue
 * (torch._scaled_mm as called at x_base/x_base/operator/h3_fp8.py:63-66):
 *   acc[m,n] = sum_k a[m,k] * w[n,k]            (e4m3fn operands, fp32 accumulation)
 *   y[m,n]   = acc * (a_scale[m*a_scale_stride] * w_scale[n*w_scale_stride]) + bias[n]
 *   out[m,n] = out_dtype(y), or with XGEN_ACT_GELU_TANH out_dtype(gelu_tanh(out_dtype(y)))
 * a: [M, K] (lda), w: [N, K] (ldw) — the weight as stored by H3FP8Linear, so
 * the product is a @ w.T.  Scale strides 0 (per-tensor) or 1 (per-token /
 * per-channel).  bias: NULL or [N] of bias_dtype (BF16/F16/F32).
 * out_dtype BF16 or F16, out [M, N] with leading dimension ldo.
 * acc_out: NULL or float32 [M, N] (leading dimension N) receiving acc.
 * Requires K % 16 == 0 and N % 16 == 0 (the reference's alignment,
 * h3_fp8.py:20-21), 16-byte aligned a/w rows, and w below 2 GiB.  M is not
 * bounded by the kernels' 32-bit offsets: rows beyond them run as consecutive
 * launches over row chunks, with the results of one launch.
 */
int xgen_scaled_mm_fp8(const void *a, int64_t lda, const void *w, int64_t ldw, int64_t M,
                       int64_t N, int64_t K, const float *a_scale, int64_t a_scale_stride,
                       const float *w_scale, int64_t w_scale_stride, const void *bias,
                       int bias_dtype, int activation, void *out, int out_dtype, int64_t ldo,
                       float *acc_out, hipStream_t stream);

/*
 * The same GEMM with exact products summed in fp32: what torch._scaled_mm's
 * use_fast_accum=False asks for at x_base/x_base/operator/h3_fp8.py:63-66.
 * gfx950's FP8 MFMA instructions truncate each product of a group of 8
 * consecutive K to a multiple of 2^(E - 13), E the group's largest exponent sum,
 * before summing (measured; xgen_scaled_mm_fp8 and torch._scaled_mm on this
 * GPU compute that); here the e4m3fn operands are converted to bf16 (exactly)
 * and multiplied on the bf16 MFMA, at twice the matrix-core time.  Arguments
 * and contract as xgen_scaled_mm_fp8.
 */
int xgen_scaled_mm_fp8_exact(const void *a, int64_t lda, const void *w, int64_t ldw, int64_t M,
                             int64_t N, int64_t K, const float *a_scale, int64_t a_scale_stride,
                             const float *w_scale, int64_t w_scale_stride, const void *bias,
                             int bias_dtype, int activation, void *out, int out_dtype, int64_t ldo,
                             float *acc_out, hipStream_t stream);

/*
 * INT8 W8A8 GEMM with fused dequant epilogue
 * (torch_npu.npu_quant_matmul as called at x_base/x_base/operator/matmul.py:63-64 and
 *  npu_fusion/runtime.py:87-91):
 *   acc[m,n] = sum_k a[m,k] * w[n,k]            (int8 operands, exact int32 accumulation)
 *   y[m,n]   = float(acc) * (pertoken_scale[m] * w_scale[n]) + bias[n]
 *   out = out_dtype(y) or, with XGEN_ACT_GELU_TANH, out_dtype(gelu_tanh(out_dtype(y))).
 * Scale strides as in xgen_scaled_mm_fp8.  acc_out: NULL or int32 [M, N]
 * (leading dimension N) receiving the exact accumulators.  Requires K % 16 == 0.
 */
int xgen_quant_matmul_int8(const void *a, int64_t lda, const void *w, int64_t ldw, int64_t M,
                           int64_t N, int64_t K, const float *pertoken_scale,
                           int64_t pertoken_scale_stride, const float *w_scale,
                           int64_t w_scale_stride, const void *bias, int bias_dtype,
                           int activation, void *out, int out_dtype, int64_t ldo,
                           int32_t *acc_out, hipStream_t stream);

/*
 * Gated residual with an indexed gate table
 * (torch.ops.h3_phaa_gate_residual.gate_residual,
 *  x_base/x_base/operator/npu_fusion/f2a/op_extension/gate_residual_queued.asc:33-35, kernel
 *  f2a/op_kernel/gate_residual_kernel.asc:57-67; eager form x_base/x_base/operator/h3_indexed_affine.py:49):
 *   out[b,s,c] = bf16(residual[b,s,c] + bf16(branch[b,s,c] * gate_table[indices[s], c]))
 * multiply, round, add, round (no fused multiply-add).  residual / branch: BF16
 * [batch, seq, width] with the given batch / seq strides (elements, last stride
 * 1); gate_table BF16 [gate_rows, width], rows gate_row_stride apart; indices
 * int64 [seq]; out BF16 [batch, seq, width] contiguous.  An index outside
 * [0, gate_rows) writes a NaN row.  width and strides multiples of 8 elements.
 */
int xgen_gate_residual(const void *residual, int64_t res_stride_batch, int64_t res_stride_seq,
                       const void *branch, int64_t br_stride_batch, int64_t br_stride_seq,
                       const void *gate_table, int64_t gate_row_stride, int64_t gate_rows,
                       const int64_t *indices, int64_t batch, int64_t seq, int64_t width, void *out,
                       hipStream_t stream);

/*
 * BF16 layouts of the head-parallel attention's exchange: torch.ops.h3_phaa_layout.{pack, back,
 * merge} (x_base/x_base/operator/npu_fusion/f4/op_extension/layout_queued.asc:27-55, kernels
 * f4/op_kernel/layout_kernel.asc:33-59, wrapper npu_fusion/phaa_layout.py:13-28; caller
 * x_base/x_base/phaa/fused_layout.py:27-52).  Byte moves only; buffers 16-byte aligned, strides
 * in elements and multiples of 8, each tensor below 2^31 16-byte units.
 *
 * xgen_phaa_pack_qkv: q/k/v [1, seq, heads, head_dim] (heads contiguous, row strides given),
 *   heads = owners * chunks * heads_per_chunk, into q/k/v_send [chunks, owners, seq, 1,
 *   heads_per_chunk, head_dim] contiguous: send[c, d, s, 0, i] = x[0, s, d * chunks *
 *   heads_per_chunk + c * heads_per_chunk + i].  The reference's geometry: owners 4, chunks 7,
 *   heads_per_chunk 2, head_dim 128.
 * xgen_phaa_pack_back: attn [1, heads, length, head_dim] (head / position strides given) into
 *   back_send [rows, heads * head_dim] contiguous: row s < length holds attn[0, :, s, :], rows
 *   from length on are zero (padding tokens); the reference's rows = 4 * S, length 4S or 4S - 1.
 * xgen_phaa_merge_back: back_recv [chunks, owners, seq, batch, chunk] contiguous into merged
 *   [batch, seq, owners * chunks * chunk] contiguous: merged[b, s, (o * chunks + c) * chunk + j] =
 *   back_recv[c, o, s, b, j] (the layout xgen_merge_quant quantizes).
 */
int xgen_phaa_pack_qkv(const void *q, const void *k, const void *v, int64_t seq, int64_t owners, int64_t chunks,
                       int64_t heads_per_chunk, int64_t head_dim, int64_t q_row_stride, int64_t k_row_stride,
                       int64_t v_row_stride, void *q_send, void *k_send, void *v_send, hipStream_t stream);
int xgen_phaa_pack_back(const void *attn, int64_t heads, int64_t length, int64_t head_dim, int64_t head_stride,
                        int64_t position_stride, int64_t rows, void *back_send, hipStream_t stream);
int xgen_phaa_merge_back(const void *back_recv, int64_t chunks, int64_t owners, int64_t seq, int64_t batch,
                         int64_t chunk, void *merged, hipStream_t stream);

/*
 * Merge of the head-parallel attention's returned chunks + per-row quantization
 * of the out-projection's input: torch.ops.h3_phaa_merge_quant.fused
 * (x_base/x_base/operator/npu_fusion/f4_merge_quant/op_extension/merge_quant_queued.asc:9-28,
 * kernel op_kernel/merge_quant_kernel.asc:20-87; wrapper npu_fusion/merge_quant.py:9-14;
 * caller x_base/x_base/phaa/fused_layout.py:44-48).
 * back_recv: BF16 [splits, owners, seq, batch, chunk], contiguous, 16-byte aligned.
 * Row b * seq + s of the output holds back_recv[c, o, s, b, :] at columns
 * (o * splits + c) * chunk: q [batch * seq, splits * owners * chunk] (contiguous,
 * 8-byte aligned) of out_dtype (XGEN_DTYPE_I8: scale mode 1 of the INT8 row
 * quantizer, as the reference's kernel; XGEN_DTYPE_E4M3: the FP8 row quantizer),
 * scale f32 [batch * seq].  The reference's geometry is splits 7, owners 4,
 * batch 1, chunk 256 (H3's 56 heads x 128).  chunk a multiple of 8,
 * splits * owners * chunk <= 16384, batch * seq < 2^31.
 */
int xgen_merge_quant(int out_dtype, const void *back_recv, int64_t splits, int64_t owners, int64_t seq,
                     int64_t batch, int64_t chunk, void *q, float *scale, hipStream_t stream);

/*
 * Indexed AdaLN modulation of normalised rows: the modulation half of the
 * reference's indexed affine (x_base/x_base/operator/h3_indexed_affine.py:9-29 and
 * :32-48, `_apply(x, scale, shift, indices, modulation=True)`, and the eager bf16
 * expression of its fallback, :46-48; the output AdaLN of
 * x_diffusers/x_diffusers/framework/transformer/minimax_h3.py:690-694):
 *   out[b,s,c] = bf16(bf16(x[b,s,c] * f) + shift_table[g, c]),  g = indices[s],
 *   f = bf16(1 + scale_table[g, c]), or scale_table[g, c] itself when
 *   scale_is_one_plus (a table prepared by xgen_adaln_one_plus).
 * x: BF16 [batch, seq, width] with the given batch / seq strides (elements, last
 * stride 1); tables BF16 [table_rows, width], rows scale_row_stride /
 * shift_row_stride apart; indices int64 [seq]; out BF16 [batch, seq, width]
 * contiguous.  An index outside [0, table_rows) writes a NaN row.  width and
 * strides multiples of 8 elements, buffers 16-byte aligned.
 */
int xgen_indexed_modulate(const void *x, int64_t x_stride_batch, int64_t x_stride_seq, const void *scale_table,
                          int64_t scale_row_stride, const void *shift_table, int64_t shift_row_stride,
                          int64_t table_rows, const int64_t *indices, int64_t batch, int64_t seq, int64_t width,
                          int scale_is_one_plus, void *out, hipStream_t stream);

/*
 * W8A8 GEMM whose bf16 output feeds the gated residual in the same epilogue:
 * the out-projection / FFN-down of a DiT block followed by
 * `residual + gate[idx] * y` (x_base/x_base/operator/h3_indexed_affine.py:58-61;
 * x_diffusers/x_diffusers/framework/transformer/hunyuan.py:387,400):
 *   y[m,n]   = bf16(acc * (a_scale[m*a_scale_stride] * w_scale[n*w_scale_stride]) + bias[n])
 *              (xgen_scaled_mm_fp8 for in_dtype E4M3, xgen_quant_matmul_int8 for I8)
 *   out[m,n] = bf16(residual[m,n] + bf16(y[m,n] * gate_table[indices[m % seq], n]))
 * residual BF16 [M, N] (leading dimension ld_residual); gate_table BF16
 * [gate_rows, N] rows gate_row_stride apart; indices int64 [seq] with M a
 * multiple of seq; out BF16 [M, N] (ldo).  Equal bit for bit to
 * xgen_scaled_mm_fp8 / xgen_quant_matmul_int8 (BF16 out) followed by
 * xgen_gate_residual.  Operand requirements as those entry points.
 */
int xgen_w8a8_gate_residual(int in_dtype, const void *a, int64_t lda, const void *w, int64_t ldw,
                            int64_t M, int64_t N, int64_t K, const float *a_scale, int64_t a_scale_stride,
                            const float *w_scale, int64_t w_scale_stride, const void *bias, int bias_dtype,
                            const void *residual, int64_t ld_residual, const void *gate_table,
                            int64_t gate_row_stride, int64_t gate_rows, const int64_t *indices, int64_t seq,
                            void *out, int64_t ldo, hipStream_t stream);

/*
 * SwiGLU + per-row quantization (the H3 FFN's activation and the requant before
 * its down-projection; torch.ops.h3_phaa_fusion_quant_reuse.swiglu_quantize,
 * x_base/x_base/operator/npu_fusion/f1b/op_extension/swiglu_quant_reuse_queued.asc:33-35,
 * kernel f1b/op_kernel/swiglu_quant_reuse_kernel.asc:36-105; gate-first layout of
 * x_base/x_base/operator/h3_swiglu.py:15-29):
 *   u: BF16 [batch, seq, 2F], row (b, s) at u + b*u_stride_batch + s*u_stride_seq (elements);
 *      gate_first 0: [hidden | gate] (the NPU kernel), 1: [gate | hidden] (h3_swiglu.py)
 *   a = bf16(silu(gate)) with silu(g) = g / (1 + exp(-g)); v = bf16(hidden * a)
 *   q, scale = per-row quantization of v: E4M3 as xgen_quantize_rows, or I8 with
 *   scale_mode 1: scale = amax * fl(1/127), 0: scale = 1 / fl(127/amax).
 * q: [batch*seq, F] contiguous; scale float32 [batch*seq]; act_out NULL or BF16
 * [batch*seq, F] receiving v.  F <= XGEN_SWIGLU_MAX_HALF, F and strides multiples of 8.
 */
int xgen_swiglu_quant(const void *u, int64_t batch, int64_t seq, int64_t half_width, int64_t u_stride_batch,
                      int64_t u_stride_seq, int gate_first, int out_dtype, int scale_mode, void *q, float *scale,
                      void *act_out, hipStream_t stream);

/*
 * table[i] = bf16(silu(bf16 with bits i)) for all 65,536 bit patterns (128 KB, 16-byte aligned),
 * with xgen_swiglu_quant's silu (IEEE division, the device expf): the same values by construction.
 * No reference counterpart (the reference evaluates silu per element); prepared once per device.
 */
int xgen_silu_bf16_table(void *table, hipStream_t stream);

/*
 * xgen_swiglu_quant with a = silu_table[gate bits] (from xgen_silu_bf16_table): the same outputs;
 * the table is read into LDS and the exponential and division leave the per-element work.
 */
int xgen_swiglu_quant_lut(const void *u, int64_t batch, int64_t seq, int64_t half_width, int64_t u_stride_batch,
                          int64_t u_stride_seq, int gate_first, int out_dtype, int scale_mode, void *q, float *scale,
                          void *act_out, const void *silu_table, hipStream_t stream);

/*
 * out = bf16(1 + scale_table) over [rows, width] BF16 rows (strides in elements): the
 * `1.0 + scale` of the eager AdaLN modulation (x_base/x_base/operator/h3_indexed_affine.py:22-28,
 * x_diffusers/x_diffusers/framework/transformer/hunyuan.py:393), computed once per table so that
 * xgen_norm_affine_quant with XGEN_NORM_SCALE_ONE_PLUS reads it per token instead of recomputing
 * it (the reference recomputes it in every call).  width and strides multiples of 8.
 */
int xgen_adaln_one_plus(const void *scale_table, int64_t rows, int64_t width, int64_t scale_row_stride,
                        void *out, int64_t out_row_stride, hipStream_t stream);

/*
 * Per-row FP8 wire codec of the head-parallel attention exchange: the encode
 * and decode kernels around the byte all-to-all of
 * x_base/x_base/phaa/fp8_transport.py:26-78 (_encode / _decode, launched at
 * :137-144 by fp8_all_to_all_many, :85).  Each row of `width` values travels as
 * `width` e4m3fn bytes then its float32 scale (width + 4 bytes):
 *   scale = max(max|v| / 448, 1e-12);  byte = e4m3fn(clamp(v / scale, +-448));
 *   decoded = out_dtype(fl32(e4m3(byte) * scale)).
 * Rows of `streams` (1, or 3 for Q/K/V) inputs of `peers * peer_rows` rows each
 * are ordered [peer][stream][peer row]; each peer block is followed by
 * peer_padding zero bytes.  width: multiple of 4, <= XGEN_WIRE_MAX_WIDTH;
 * streams * peers * peer_rows < 2^31.
 */

/* Zero bytes after each peer block for the 16-byte peer alignment option
 * (fp8_transport.py:103-105, XGEN_PHAA_FP8_ALIGN16): (-peer_bytes) mod 16 with
 * peer_bytes = streams * peer_rows * (width + 4) when align16, else 0. */
int64_t xgen_fp8_wire_peer_padding(int streams, int64_t peer_rows, int64_t width, int align16);

/*
 * Encode (fp8_transport.py:26-63).  in_dtype BF16, F16 or F32.  Stream s (q,
 * then k, v when streams == 3) is a [peers, seq, batch, heads, width] view:
 * row (p, t, b, h) starts at element p*strides[4s] + t*strides[4s+1] +
 * b*strides[4s+2] + h*strides[4s+3] (host array of 4*streams non-negative
 * element strides; unit last stride).  peer_rows = seq*batch*heads.  wire:
 * peers * (streams*peer_rows*(width+4) + peer_padding) bytes, 4-byte aligned.
 */
int xgen_fp8_wire_encode(int in_dtype, int streams, const void *q, const void *k, const void *v,
                         const int64_t *strides, int64_t peers, int64_t seq, int64_t batch, int64_t heads,
                         int64_t width, int64_t peer_padding, void *wire, hipStream_t stream);

/*
 * Decode (fp8_transport.py:66-78) into contiguous [peers*peer_rows, width]
 * outputs q (and k, v when streams == 3) of out_dtype BF16, F16 or F32.
 */
int xgen_fp8_wire_decode(int out_dtype, int streams, const void *wire, int64_t peers, int64_t peer_rows,
                         int64_t width, int64_t peer_padding, void *q, void *k, void *v, hipStream_t stream);

/*
 * The asynchronous transport's layouts (x_base/x_base/phaa/fp8_async_transport.py:13-80,
 * _encode / _decode launched by _pack_exchange :126-180 and _unpack_exchange :183-193).
 * Its wire has no peer padding.
 *
 * Encode with a valid sequence length (the fused return pack, RETURN_SEQ,
 * :22-27,41-44): as xgen_fp8_wire_encode with peer_padding 0, except that a row
 * (p, t, b, h) with p*seq + t >= valid_seq is not read and travels as a zero
 * row (scale 1e-12, zero bytes).  valid_seq >= peers*seq encodes every row.
 */
int xgen_fp8_wire_encode_masked(int in_dtype, int streams, const void *q, const void *k, const void *v,
                                const int64_t *strides, int64_t peers, int64_t seq, int64_t batch, int64_t heads,
                                int64_t width, int64_t valid_seq, void *wire, hipStream_t stream);

/*
 * Decode into strided outputs (the direct gather GATHER_SEQ, :67-73, and the
 * return layout CHUNK_HEADS / HEAD_START, :74-78): wire row (p, t, b, h) of
 * stream s (peer_rows = seq*batch*heads, rows ordered as the encoder's) is
 * written as `width` contiguous values at element p*dst_strides[0] +
 * t*dst_strides[1] + b*dst_strides[2] + h*dst_strides[3] of output s (host
 * array of 4 non-negative element strides, shared by the streams); rows with
 * p*seq + t >= valid_seq are not written.
 */
int xgen_fp8_wire_decode_strided(int out_dtype, int streams, const void *wire, int64_t peers, int64_t seq,
                                 int64_t batch, int64_t heads, int64_t width, const int64_t *dst_strides,
                                 int64_t valid_seq, void *q, void *k, void *v, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* XGEN_AMD_H */
