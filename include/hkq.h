/*
 * hkq.h -- C ABI of the MI355X (gfx950) quantized-GEMM library (libhkq.so).
 *
 * Plain pointers and sizes only: every tensor is a caller-owned device buffer,
 * every call is asynchronous on `stream` (0 = the null stream, which is where
 * the reference launches everything), and every call returns 0 on success or a
 * hipError_t code. Argument errors return hipErrorInvalidValue (1) before any
 * launch; the message is available from hkq_last_error().
 *
 * Data formats
 *   bf16     : raw 16-bit patterns;
 *   FP8      : OCP E4M3FN codes (torch.float8_e4m3fn), one byte each;
 *   FP4      : OCP E2M1 codes, two per byte, even K index in the low nibble;
 *   e8m0     : one byte, value 2^(code - 127);
 *   strides  : in elements of the tensor they describe (bytes for u8 tensors).
 *
 * Each entry point names the reference interface it replaces (paths relative
 * to the m8than/amd-kernels repository).
 */
#ifndef HKQ_H
#define HKQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hkq_stream_t; /* the same type as hipStream_t */

#define HKQ_KIND_FP8 0  /* E4M3FN codes, QMAX 448 */
#define HKQ_KIND_INT8 1 /* int8, QMAX 127, round-half-even (the reference quant_tk rule) */

/* Message of the last argument or launch error raised on this thread. */
const char* hkq_last_error(void);

/* Library version, (major << 16) | minor. */
int hkq_version(void);

/* ---- quantizers ------------------------------------------------------------ */

/* Per-token dynamic quantization: s[m] = max(amax(x[m,:]) / QMAX, 1e-10),
 * q[m,k] = encode(clamp(x[m,k] * (1/s[m]), +-QMAX)).
 * x bf16 [M, ldx]; q u8/i8 [M, ldq]; s fp32 [M]. K % 8 == 0, K <= 32768.
 * Replaces quant_tk.per_token_quant_fwd (kernels/quantization/quant/kernel.cpp:140-166),
 * which is the HKQ_KIND_INT8 rule; HKQ_KIND_FP8 is the same rule with QMAX 448
 * and an E4M3FN encoder. */
int hkq_per_token_quant(const void* x, void* q, float* s, int64_t M, int64_t K, int64_t ldx, int64_t ldq, int kind,
                        hkq_stream_t stream);

/* 1 x group dynamic quantization (group in {32,64,128,256,512}):
 * s[m, g] over columns [g*group, (g+1)*group), same rule as above.
 * s fp32 [M, lds]. Replaces the quantization step of
 * fused_fp8_quant_tk.fused_rmsnorm_fp8_quant_fwd
 * (kernels/quantization/fused_fp8_quant/kernel.cpp:190-206, 240-268) without the
 * RMSNorm and with a real E4M3FN encoder in place of the affine byte at :206. */
int hkq_group_quant(const void* x, void* q, float* s, int64_t M, int64_t K, int64_t ldx, int64_t ldq, int64_t lds,
                    int64_t group, int kind, hkq_stream_t stream);

/* y = E4M3FN(clamp(x / scale[0], +-448)), n elements (n % 8 == 0).
 * Replaces quant_moe_tk.downcast_to_static_fp8 (kernels/moe-misc/quant_moe/kernel.cpp:392-410),
 * with round-to-nearest-even in place of its truncating encoder (:50-73). */
int hkq_static_quant_fp8(const void* x, void* y, const float* scale, int64_t n, hkq_stream_t stream);

/* MX quantization along the contiguous dim in blocks of 32, x bf16 [M, ldx].
 * is_fp4: q [M, K/2] E2M1 pairs, s [M, K/32] e8m0 by the MXFP4 rule of
 *   fused_mxfp4_quant (kernels/quantization/fused_mxfp4_quant/kernel.cpp:97-162);
 * else  : q [M, K] E4M3FN, s [M, K/32] by the MX-FP8 rule of
 *   quant_moe (kernels/moe-misc/quant_moe/kernel.cpp:143-217).
 * Replaces quant_moe_tk.downcast_to_mxfp (quant_moe/kernel.cpp:412-431), whose
 * FP4 branch writes zeros (:211-214). */
int hkq_mx_quant(const void* x, void* q, void* s, int64_t M, int64_t K, int64_t ldx, int is_fp4, hkq_stream_t stream);

/* out bf16 [M, K] = decode(q) * 2^(s - 127), s = 0xFF -> NaN.
 * Replaces quant_moe_tk.upcast_from_mxfp (kernels/moe-misc/quant_moe/kernel.cpp:433-450). */
int hkq_mx_dequant(const void* q, const void* s, void* out, int64_t M, int64_t K, int is_fp4, hkq_stream_t stream);

/* ---- dense GEMMs (A [M, K], B [N, K], both K-contiguous; C bf16 [M, ldc]) ---- */

/* C = bf16((A . B^T) * sa[m] * sb[n]); A, B E4M3FN; sa fp32 [M], sb fp32 [N].
 * K % 64 == 0 (as the reference requires), N % 4 == 0, ldc % 4 == 0.
 * Replaces gemm_a8w8_tk.dispatch(A, B, a_scale, b_scale, C)
 * (kernels/gemm-basic/gemm_a8w8/kernel.cpp:162-175) and
 * gemm_a8w8_per_token_scale_tk.dispatch(A, B, C, a_scale, b_scale)
 * (kernels/gemm-basic/gemm_a8w8_per_token_scale/kernel.cpp:158-171). */
int hkq_gemm_a8w8(const void* A, const void* B, const float* sa, const float* sb, void* C, int64_t M, int64_t N,
                  int64_t K, int64_t lda, int64_t ldb, int64_t ldc, hkq_stream_t stream);

/* hkq_gemm_a8w8 with a caller-provided device workspace (16-byte aligned).
 * Shapes whose tiles would fill at most half of the CUs (256 x 256 tiles
 * become 128 x 128, or (32 or 64) x 256 for M <= 64, first) split K over
 * several workgroups and add the fp32 partials in a second kernel; that needs
 * hkq_gemm_a8w8_workspace(M, N, K) bytes (0: no split for this shape). With a smaller workspace (or NULL) the
 * call runs unsplit. Same results either way up to fp32 summation order. The
 * workspace is in use until the work queued on `stream` completes. No
 * counterpart in the reference, whose kernels have no split path; the drop-in
 * modules (gemm_a8w8_tk, gemm_a8w8_per_token_scale_tk) call it with a
 * workspace from torch's allocator. */
size_t hkq_gemm_a8w8_workspace(int64_t M, int64_t N, int64_t K);
int hkq_gemm_a8w8_ws(const void* A, const void* B, const float* sa, const float* sb, void* C, int64_t M, int64_t N,
                     int64_t K, int64_t lda, int64_t ldb, int64_t ldc, void* workspace, size_t workspace_bytes,
                     hkq_stream_t stream);

/* MXFP4 A4W4: C = bf16(sum_k e2m1(A) 2^(As-127) e2m1(B) 2^(Bs-127)).
 * A u8 [M, lda >= K/2], As u8 [M, ldsa >= K/32], B u8 [N, ldb], Bs u8 [N, ldsb].
 * K % 128 == 0, N % 4 == 0, ldc % 4 == 0. Replaces gemm_afp4wfp4_tk.dispatch (kernels/gemm-basic/gemm_afp4wfp4/kernel.cpp:147-159),
 * taking the packed format its header documents (:3-6) instead of
 * pre-dequantized bf16. */
int hkq_gemm_mxfp4(const void* A, const void* As, const void* B, const void* Bs, void* C, int64_t M, int64_t N,
                   int64_t K, int64_t lda, int64_t ldb, int64_t ldsa, int64_t ldsb, int64_t ldc, hkq_stream_t stream);

/* hkq_gemm_mxfp4 with a caller-provided workspace: the split-K plan of
 * hkq_gemm_a8w8_ws for the MXFP4 GEMM (no counterpart in the reference;
 * gemm_afp4wfp4_tk calls it with a workspace from torch's allocator). */
size_t hkq_gemm_mxfp4_workspace(int64_t M, int64_t N, int64_t K);
int hkq_gemm_mxfp4_ws(const void* A, const void* As, const void* B, const void* Bs, void* C, int64_t M, int64_t N,
                      int64_t K, int64_t lda, int64_t ldb, int64_t ldsa, int64_t ldsb, int64_t ldc, void* workspace,
                      size_t workspace_bytes, hkq_stream_t stream);

/* Block-scale FP8 GEMM (DeepSeek-V3 style):
 * C = bf16(sum_g (A_g . B_g^T) * sa[m, g] * sb[g, n / group_n]), g = 128-wide K group.
 * A, B E4M3FN [M, K] / [N, K]; sa fp32 [M, lsa >= K/128]; sb fp32 [K/128, lsb] with
 * lsb >= N (group_n 1, per column) or >= ceil(N/128) (group_n 128, 128x128 blocks).
 * K % 128 == 0, N % 4 == 0, ldc % 4 == 0. Replaces
 * gemm_a8w8_blockscale_tk.dispatch(A, B, C, a_scale, b_scale)
 * (kernels/gemm-basic/gemm_a8w8_blockscale/kernel.cpp:167-180; formula
 * kernels/gemm-basic/gemm_a8w8_blockscale/test_parity.py:57-76). */
int hkq_gemm_blockscale(const void* A, const void* B, const float* sa, const float* sb, void* C, int64_t M, int64_t N,
                        int64_t K, int64_t lda, int64_t ldb, int64_t lsa, int64_t lsb, int64_t ldc, int64_t group_n,
                        hkq_stream_t stream);

/* ---- MoE grouped GEMM over OGS routing metadata -------------------------- */

/* For every routing tile ExptData[pm] = e | (b << 16) (-1: skipped), pm < grid_m,
 * rows gm = b*128 + r < hist[e], sorted index s = offs[e] + gm,
 * token = gather[s] / topk (gather == NULL: token = s):
 *   Y[s, n] = bf16((sum_k X[token, k] * W[e, n, k]) * xs(token) * ws(e, n) + bias[e, n]).
 * X E4M3FN [T, stride_xm], K contiguous; W E4M3FN with expert stride stride_we and
 * row (n) stride stride_wn, K contiguous (the reference's [E, K, N] layout has to
 * be passed transposed to [E, N, K]); Y bf16 rows of stride_ym, y_rows of them.
 * xs: NULL (1), x_scale[0] (xs_stride_tok 0) or x_scale[token * xs_stride_tok].
 * ws: NULL (1) or w_scale[e * ws_stride_e + (n / ws_group_n) * ws_stride_n]
 *   (per expert: ws_stride_n 0; per channel: ws_stride_e N, ws_stride_n 1, ws_group_n 1).
 * bias: NULL or fp32 bias[e * bias_stride_e + n]. K % 64 == 0, N % 4 == 0.
 * Routing entries that name an expert >= E, rows past gather_len and tokens past
 * T read zero or are skipped. Replaces moe_op_gemm_a8w8_tk.moe_a8w8
 * (kernels/moe-gemm/moe_op_gemm_a8w8/kernel.cpp:194-271) and, for group_k == K,
 * moe_op_gemm_a8w8_blockscale_tk.moe_a8w8_blockscale
 * (kernels/moe-gemm/moe_op_gemm_a8w8_blockscale/kernel.cpp:192-280). */
int hkq_moe_a8w8(const void* X, const void* W, void* Y, const float* x_scale, int64_t xs_stride_tok,
                 const float* w_scale, int64_t ws_stride_e, int64_t ws_stride_n, int64_t ws_group_n, const float* bias,
                 int64_t bias_stride_e, const int32_t* gather, const int32_t* hist, const int32_t* offs,
                 const int32_t* expt_data, int64_t T, int64_t E, int64_t N, int64_t K, int64_t grid_m, int64_t topk,
                 int64_t stride_xm, int64_t stride_we, int64_t stride_wn, int64_t stride_ym, int64_t y_rows,
                 int64_t gather_len, hkq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HKQ_H */
