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

/* ---- quantizers fused with their producer -------------------------------- */

/* RMSNorm + quantization of x bf16 [M, ldx] with weight w bf16 [D] (D <= 8192):
 * r = 1 / sqrt(sum(x^2) / D + eps), y = (x * r) * w, with sum(x^2) reduced in a
 * fixed order (per lane of a wave: fma chain over the 16-byte chunks
 * c = lane + 64 i, then an xor butterfly over the 64 lanes), then
 * kind 0: 1x128 FP8, s[m, g] = max(amax/448, 1e-10) fp32 [M, lds],
 *         q = E4M3FN(clamp(y / s)) [M, ldq] (D % 128 == 0);
 * kind 1: MXFP4, s = e8m0 of the MX shared exponent [M, lds] bytes, q = two
 *         E2M1 codes per byte [M, ldq] (D % 32 == 0), elements rounded to
 *         nearest even (the OCP MX rule, as hkq_mx_quant);
 * kind 2: as kind 1 with elements floored by the threshold ladder of
 *         fused_mxfp4_quant/kernel.cpp:128-150 (largest E2M1 magnitude at or
 *         below |y| * 2^-e, sign kept), the reference module's codes.
 * Replaces fused_rmsnorm_fp8_quant_fwd (kernels/quantization/fused_fp8_quant/
 * kernel.cpp:251-268) and fused_rmsnorm_mxfp4_quant_fwd (fused_mxfp4_quant/
 * kernel.cpp:291-308), which accept only D in {4096, 8192} and write an affine
 * byte instead of E4M3 codes (fused_fp8_quant/kernel.cpp:206). */
int hkq_rmsnorm_quant(const void* x, const void* w, void* q, void* s, int64_t M, int64_t D, int64_t ldx, int64_t ldq,
                      int64_t lds, float eps, int kind, hkq_stream_t stream);

/* SwiGLU + FP8 quantization of a gate/up GEMM output y bf16 [M, ldy] (2F
 * columns used): act = silu(g) * u with silu(g) = g / (1 + 2^(-log2(e) * alpha * g))
 * (the silu of kernels/moe-gemm/moe_op_gemm_a8w8/kernel.cpp:57-59);
 * (g, u) = columns (k, F + k), or (2k, 2k + 1) when interleaved (the column
 * order of kernels/moe-gemm/moe_op_silu_fused/kernel.cpp:9-12). group 0: one
 * scale per row s[m]; group 128: s[m * lds + k / 128]; s = max(amax/448, 1e-10),
 * q = E4M3FN(clamp(act / s)) [M, ldq]. No counterpart in the reference, which
 * leaves the activation to a separate kernel (moe_op_gemm_a8w8/kernel.cpp:162);
 * this feeds the per-token FP8 down projection of hkq_moe_a8w8. */
int hkq_swiglu_quant(const void* y, void* q, float* s, int64_t M, int64_t F, int64_t ldy, int64_t ldq, int64_t lds,
                     float alpha, int interleaved, int group, hkq_stream_t stream);

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
 * become 128 x 128 or 128 x 64, or (32 or 64) x 256 for M <= 64, first) split
 * K over several workgroups in one launch: each writes its fp32 partial sums
 * to the workspace, and the last split of a tile to finish adds all of them in
 * split order and writes C (bit-identical whichever split finishes last).
 * That needs hkq_gemm_a8w8_workspace(M, N, K) bytes (0: no split for this
 * shape; M <= 16 runs a single-launch streaming kernel that needs none). With
 * a smaller workspace (or NULL) the call runs unsplit. Same results either way
 * up to fp32 summation order. The workspace needs no clearing: its first 4 KB
 * hold per-tile arrival counters that each call leaves marked idle (a
 * workspace that held other data is claimed on first use, at the cost of one
 * compare-and-swap per counter). It is in use until the work queued on
 * `stream` completes; calls that may overlap need separate workspaces. No
 * counterpart in the reference, whose kernels have no split path; the drop-in
 * modules (gemm_a8w8_tk, gemm_a8w8_per_token_scale_tk) call it with a
 * workspace from torch's allocator. */
size_t hkq_gemm_a8w8_workspace(int64_t M, int64_t N, int64_t K);
int hkq_gemm_a8w8_ws(const void* A, const void* B, const float* sa, const float* sb, void* C, int64_t M, int64_t N,
                     int64_t K, int64_t lda, int64_t ldb, int64_t ldc, void* workspace, size_t workspace_bytes,
                     hkq_stream_t stream);

/* hkq_gemm_a8w8_ws without a caller workspace and without allocating: the
 * split-K counters and partials go to a library-owned device array of
 * hkq_gemm_a8w8_noalloc_max_workspace() bytes (32 MiB) that each GPU the
 * library runs on holds until the process ends. Shapes whose plan needs more
 * are rejected with hipErrorInvalidValue (none on a 256-CU MI355X). Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (several
 * streams or host threads) race and must be serialized by the caller. No
 * counterpart in the reference; for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). */
size_t hkq_gemm_a8w8_noalloc_max_workspace(void);
int hkq_gemm_a8w8_noalloc(const void* A, const void* B, const float* sa, const float* sb, void* C, int64_t M,
                          int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, hkq_stream_t stream);

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

/* Block-scale FP8 GEMM with a multiply-add epilogue:
 * C = bf16(c_a[m, n] * G[m, n] + c_b[m, n]), G the fp32 block-scale sum of
 * hkq_gemm_blockscale (not rounded before the multiply-add); c_a / c_b bf16
 * rows of ldca / ldcb elements (>= N, multiples of 4). Replaces
 * fused_gemm_a8w8_blockscale_mul_add_tk.dispatch(a, b, c, a_scale, b_scale, c_a, c_b)
 * (kernels/gemm-fused/fused_gemm_a8w8_blockscale_mul_add/kernel.cpp:47-194; formula
 * tests/test_gemm.py:498-533). */
int hkq_gemm_blockscale_mul_add(const void* A, const void* B, const float* sa, const float* sb, void* C,
                                const void* c_a, const void* c_b, int64_t M, int64_t N, int64_t K, int64_t lda,
                                int64_t ldb, int64_t lsa, int64_t lsb, int64_t ldc, int64_t ldca, int64_t ldcb,
                                int64_t group_n, hkq_stream_t stream);

/* ---- batched and bf16 GEMMs ---------------------------------------------- */

/* Batched A8W8 GEMM: for z < batch,
 * C_z = bf16((A_z . B_z^T) * sa_z[m] * sb_z[n] + bias_z[n]),
 * operand z at z * batch_stride_* (bytes for A/B, elements for C, sa, sb and
 * bias); bias bf16 [N] per batch or NULL. Shapes and strides as hkq_gemm_a8w8;
 * batch <= 65535. Replaces batched_gemm_a8w8_tk.dispatch(A, B, a_scale, b_scale, C, bias)
 * (kernels/gemm-batched/batched_gemm_a8w8/kernel.cpp:59-203; formula
 * tests/test_gemm.py:349-390), with E4M3FN codes for A and B. */
int hkq_batched_gemm_a8w8(const void* A, const void* B, const float* sa, const float* sb, const void* bias, void* C,
                          int64_t batch, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                          int64_t batch_stride_a, int64_t batch_stride_b, int64_t batch_stride_c,
                          int64_t batch_stride_sa, int64_t batch_stride_sb, int64_t batch_stride_bias,
                          hkq_stream_t stream);

/* bf16 GEMM C = bf16(A . B^T), A [M, K], B [N, K], C [M, N] bf16 with row
 * strides lda, ldb, ldc in elements (lda, ldb multiples of 8; K % 32 == 0).
 * Replaces gemm_a16w16_tk.dispatch(A, B, C)
 * (kernels/gemm-basic/gemm_a16w16, which holds no kernel source in the reference tree; formula tests/test_gemm.py:21-42)
 * and the bf16 half of fused_gemm_a8w8_blockscale_a16w16_tk.dispatch
 * (kernels/gemm-fused/fused_gemm_a8w8_blockscale_a16w16/kernel.cpp:60-270; tests/test_gemm.py:454-496). */
int hkq_gemm_bf16(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                  int64_t ldc, hkq_stream_t stream);

/* Batched bf16 GEMM with bias: C_z = bf16(A_z . B_z^T + bias_z[n]), strides in
 * elements, bias bf16 [N] per batch or NULL; with batch == 1 and no bias a
 * workspace of hkq_gemm_bf16_workspace bytes lets small grids split K (the
 * plan of hkq_gemm_a8w8_ws). Replaces batched_gemm_bf16_tk.dispatch(A, B, C, bias)
 * (kernels/gemm-batched/batched_gemm_bf16/kernel.cpp:53-187; formula tests/test_gemm.py:316-347). */
size_t hkq_gemm_bf16_workspace(int64_t M, int64_t N, int64_t K);
int hkq_batched_gemm_bf16(const void* A, const void* B, const void* bias, void* C, int64_t batch, int64_t M, int64_t N,
                          int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t batch_stride_a,
                          int64_t batch_stride_b, int64_t batch_stride_c, int64_t batch_stride_bias, void* workspace,
                          size_t workspace_bytes, hkq_stream_t stream);

/* ---- MoE grouped GEMM over OGS routing metadata -------------------------- */

/* For every routing tile ExptData[pm] = e | (b << 16) (-1: skipped), pm < grid_m,
 * rows gm = b*128 + r < hist[e], sorted index s = offs[e] + gm,
 * token = gather[s] / topk (gather == NULL: token = s):
 *   Y[s, n] = bf16((sum_k X[token, k] * W[e, n, k]) * xs(token) * ws(e, n) + bias[e, n]).
 * X E4M3FN [T, stride_xm], K contiguous; W E4M3FN with expert stride stride_we and
 * row (n) stride stride_wn, K contiguous (the reference's N-contiguous [E, K, N]
 * layout: hkq_moe_a8w8_kn); Y bf16 rows of stride_ym, y_rows of them.
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

/* hkq_moe_a8w8 on the reference's N-contiguous weights: W[e, k, n] at
 * W + e * stride_we + k * stride_wk + n (stride_wk >= N, a multiple of 16;
 * K % 128 == 0; K * stride_wk < 2^31). The kernels stage each K-tile of W as
 * it lies (rows of K) and build the MFMA operand with transposed LDS reads, so
 * no K-major copy is made; every output element is the one hkq_moe_a8w8 gives
 * for the same weights in [E, N, K] (bit for bit). Decode-sized launches run the
 * tiled kernel. Replaces moe_op_gemm_a8w8_tk.moe_a8w8 with stride_wn == 1, the
 * reference's own call (kernels/moe-gemm/moe_op_gemm_a8w8/kernel.cpp:120, the
 * weight read W[e*stride_we + k*stride_wk + n*stride_wn]; tests/test_moe.py:703-729). */
int hkq_moe_a8w8_kn(const void* X, const void* W, void* Y, const float* x_scale, int64_t xs_stride_tok,
                    const float* w_scale, int64_t ws_stride_e, int64_t ws_stride_n, int64_t ws_group_n,
                    const float* bias, int64_t bias_stride_e, const int32_t* gather, const int32_t* hist,
                    const int32_t* offs, const int32_t* expt_data, int64_t T, int64_t E, int64_t N, int64_t K,
                    int64_t grid_m, int64_t topk, int64_t stride_xm, int64_t stride_we, int64_t stride_wk,
                    int64_t stride_ym, int64_t y_rows, int64_t gather_len, hkq_stream_t stream);

/* The same grouped GEMM with per-K-group scales: for group g = k / group_k
 * (group_k a multiple of 64),
 *   Y[s, n] = bf16(sum_g (sum_{k in g} X[token, k] W[e, n, k])
 *                  * x_scale[token * xs_stride_m + g * xs_stride_k]
 *                  * w_scale[e * ws_stride_e + g * ws_stride_k + (n / group_n) * ws_stride_n]
 *                  + bias[e * bias_stride_e + n]).
 * Routing, X, W, Y, bias and the argument checks as hkq_moe_a8w8; x_scale and
 * w_scale are required. Replaces moe_op_gemm_a8w8_blockscale_tk.moe_a8w8_blockscale
 * (kernels/moe-gemm/moe_op_gemm_a8w8_blockscale/kernel.cpp:192-280; per-tile
 * promotion :114-145) for any group_k; group_k == K is also served, faster, by
 * hkq_moe_a8w8 with per-token x per-channel-group scales. */
int hkq_moe_a8w8_blockscale(const void* X, const void* W, void* Y, const float* x_scale, int64_t xs_stride_m,
                            int64_t xs_stride_k, const float* w_scale, int64_t ws_stride_e, int64_t ws_stride_k,
                            int64_t ws_stride_n, int64_t group_k, int64_t group_n, const float* bias,
                            int64_t bias_stride_e, const int32_t* gather, const int32_t* hist, const int32_t* offs,
                            const int32_t* expt_data, int64_t T, int64_t E, int64_t N, int64_t K, int64_t grid_m,
                            int64_t topk, int64_t stride_xm, int64_t stride_we, int64_t stride_wn, int64_t stride_ym,
                            int64_t y_rows, int64_t gather_len, hkq_stream_t stream);

/* hkq_moe_a8w8_blockscale on the reference's N-contiguous weights: W[e, k, n]
 * at W + e * stride_we + k * stride_wk + n (stride_wk >= N, a multiple of 16;
 * K * stride_wk < 2^31), read in place by the kernels (K-tiles staged as rows
 * of K, the MFMA operand built with transposed LDS reads); every output
 * element is the one hkq_moe_a8w8_blockscale gives for the same weights in
 * [E, N, K], bit for bit. Replaces moe_op_gemm_a8w8_blockscale_tk.moe_a8w8_blockscale
 * with stride_wn == 1, the reference's own call (kernels/moe-gemm/
 * moe_op_gemm_a8w8_blockscale/kernel.cpp:108, the weight read
 * W[e*stride_we + k*stride_wk + n*stride_wn]; tests/test_moe.py:771-815). */
int hkq_moe_a8w8_blockscale_kn(const void* X, const void* W, void* Y, const float* x_scale, int64_t xs_stride_m,
                               int64_t xs_stride_k, const float* w_scale, int64_t ws_stride_e, int64_t ws_stride_k,
                               int64_t ws_stride_n, int64_t group_k, int64_t group_n, const float* bias,
                               int64_t bias_stride_e, const int32_t* gather, const int32_t* hist, const int32_t* offs,
                               const int32_t* expt_data, int64_t T, int64_t E, int64_t N, int64_t K, int64_t grid_m,
                               int64_t topk, int64_t stride_xm, int64_t stride_we, int64_t stride_wk,
                               int64_t stride_ym, int64_t y_rows, int64_t gather_len, hkq_stream_t stream);

/* Byte-plane transpose dst[e][n][r] = src[e][r][n] (src row r at
 * src + e*src_stride_e + r*src_stride_r, N contiguous bytes; dst row n at
 * dst + e*dst_stride_e + n*dst_stride_n, R contiguous bytes). Turns the
 * reference's N-contiguous MoE weights -- E4M3FN [E, K, N], E2M1 pairs
 * [E, K/2, N] and e8m0 weight scales [E, K/32, N] (tests/test_moe.py:723-729,
 * 808-815, 909-925) -- into the K-contiguous rows the MoE GEMMs above read.
 * The reference's kernels read W through stride_wk / stride_wn instead
 * (kernels/moe-gemm/moe_op_gemm_a8w8/kernel.cpp:120,
 * moe_op_gemm_a8w8_blockscale/kernel.cpp:108, moe_op_mxfp4/kernel.cpp:155);
 * the reference-named modules call this on such weights before the GEMM. */
int hkq_moe_pack_kmajor(const void* src, void* dst, int64_t E, int64_t R, int64_t N, int64_t src_stride_e,
                        int64_t src_stride_r, int64_t dst_stride_e, int64_t dst_stride_n, hkq_stream_t stream);

/* MXFP4 MoE over block-sorted routing (the output of hkq_moe_align_block_size):
 * tile row r of 128-row block pm is gate id = sorted_token_ids[pm*128 + r]
 * (rows with id >= num_valid_tokens are padding), expert e = expert_ids[pm]:
 *   C[id, n] = bf16((sum_k A[id / top_k, k] B[e, n, k]) * A_scale[0] * B_scale[e]
 *                   * (mul_routed_weight ? topk_weights[id] : 1))
 * (A_scale / B_scale NULL: 1); a block with e == -1 writes zeros to its valid
 * rows. A [num_tokens, stride_am] bytes and B[e] [N, stride_bn] bytes hold E2M1
 * pairs, K contiguous (even k in the low nibble); A_mx_scale [num_tokens,
 * stride_amxm] and B_mx_scale[e] [N, stride_bmxn] hold e8m0 bytes per 32 K
 * values; expert e at B + e*stride_be, B_mx_scale + e*stride_bmxe; C bf16 rows
 * of stride_cm. K % 128 == 0, N % 4 == 0. Replaces moe_op_mxfp4_tk.moe_mxfp4
 * (kernels/moe-gemm/moe_op_mxfp4/kernel.cpp:263-330) with K-contiguous
 * weights; the reference's own [E, K/2, N] weights and [E, K/32, N] scales go
 * to hkq_moe_mxfp4_kn. */
int hkq_moe_mxfp4(const void* A, const void* B, void* C, const void* A_mx_scale, const void* B_mx_scale,
                  const float* A_scale, const float* B_scale, const float* topk_weights,
                  const int32_t* sorted_token_ids, const int32_t* expert_ids, int64_t N, int64_t K,
                  int64_t num_valid_tokens, int64_t top_k, int mul_routed_weight, int64_t stride_am,
                  int64_t stride_be, int64_t stride_bn, int64_t stride_cm, int64_t stride_amxm, int64_t stride_bmxe,
                  int64_t stride_bmxn, int64_t num_tokens, int64_t num_experts, int64_t grid_m, hkq_stream_t stream);

/* hkq_moe_mxfp4 on the reference's N-contiguous weights: B[e] [K/2, N] (E2M1
 * pairs of K for each column, row stride stride_bk) and B_mx_scale[e] [K/32, N]
 * (row stride stride_bmxk), read in place by the kernels (K-tiles staged as
 * rows of K, operands and e8m0 scale operands built with transposed LDS
 * reads); every output element is the one hkq_moe_mxfp4 gives for the same
 * values in [E, N, K/2] / [E, N, K/32], bit for bit. K % 256 == 0; stride_bk,
 * stride_bmxk >= N; stride_bk, stride_bmxk, stride_be, stride_bmxe multiples
 * of 16 and B_mx_scale 16-byte aligned. Decode-sized launches run the tiled
 * kernel. Replaces moe_op_mxfp4_tk.moe_mxfp4 with stride_bn == stride_bmxn == 1,
 * the reference's own call (kernels/moe-gemm/moe_op_mxfp4/kernel.cpp:155, the
 * weight read through stride_bk / stride_bn; tests/test_moe.py:909-925). */
int hkq_moe_mxfp4_kn(const void* A, const void* B, void* C, const void* A_mx_scale, const void* B_mx_scale,
                     const float* A_scale, const float* B_scale, const float* topk_weights,
                     const int32_t* sorted_token_ids, const int32_t* expert_ids, int64_t N, int64_t K,
                     int64_t num_valid_tokens, int64_t top_k, int mul_routed_weight, int64_t stride_am,
                     int64_t stride_be, int64_t stride_bk, int64_t stride_cm, int64_t stride_amxm,
                     int64_t stride_bmxe, int64_t stride_bmxk, int64_t num_tokens, int64_t num_experts,
                     int64_t grid_m, hkq_stream_t stream);

/* ---- MoE routing metadata producers --------------------------------------- */
/* All index outputs are deterministic: gates of one expert keep their input
 * order (the order of the reference's test formulas, tests/test_moe.py:97-128,
 * 229-256), and no output needs to be cleared beforehand. */

/* Top-K of each row of bf16 logits X [n_rows, stride_xm] (n_expts_tot <= 1024,
 * 1 <= K <= 16): Yi[r*stride_ym + k] = expert of the k-th largest logit (ties:
 * lower expert first; -0 == +0; NaN and -inf never chosen; -1 when fewer than
 * K are eligible), Yv = its logit (bf16, -inf for -1), or with apply_softmax
 * expf(v_k - v_0) * (1 / sum_k expf(v_k - v_0)). Bits (NULL: skipped) gets
 * ceil(n_expts_tot / 32) words per row at Bits[r*stride_bm + w*stride_bn],
 * bit e%32 of word e/32 set for each chosen expert. Replaces launch_moe_topk
 * (kernels/moe-routing/moe_topk/kernel.cpp:218-270), which always writes 8
 * words and handles only K in {2, 4, 8} over the first 256 experts. */
int hkq_moe_topk(const void* X, int64_t stride_xm, void* Yv, int32_t* Yi, int64_t stride_ym, uint32_t* Bits,
                 int64_t stride_bm, int64_t stride_bn, int64_t n_rows, int64_t n_expts_tot, int K, int apply_softmax,
                 hkq_stream_t stream);

/* Column sums of the bitmatrix B (word w of row r at B[r*stride_bm + w*stride_bn],
 * shape_bn words per row): Ret[e] = rows with bit e set (32*shape_bn entries);
 * Partials[t*stride_pm + e*stride_pn] = the same count over the 128-row tiles
 * before tile t, for t < ceil(shape_bm / 128) and e < shape_pn. Replaces
 * launch_sum_bitmatrix_rows (kernels/moe-routing/moe_bitmatrix/kernel.cpp:208-241). */
int hkq_sum_bitmatrix_rows(const uint32_t* B, int64_t shape_bm, int64_t stride_bm, int64_t stride_bn, uint32_t* Ret,
                           uint32_t* Partials, int64_t stride_pm, int64_t stride_pn, int64_t shape_pn,
                           int64_t shape_bn, hkq_stream_t stream);

/* Ret only, over all shape_bm rows (the reference reads at most 128). Replaces
 * launch_sum_bitmatrix_rows_fused (moe_bitmatrix/kernel.cpp:244-297). */
int hkq_sum_bitmatrix_rows_fused(const uint32_t* B, int64_t shape_bm, int64_t stride_bm, int64_t stride_bn,
                                 uint32_t* Ret, int64_t n_blks_bitmatrix, hkq_stream_t stream);

/* OGS expert data from the per-expert histogram (n_expts_tot <= 4096), tiles of
 * 2^tile_dim_log2 rows: TokenStart[e] / TileStart[e] = exclusive prefix sums of
 * Hist and of ceil(Hist / tile), TokenStart[E] = n_gates, TileStart[E] = total
 * tiles; MDTileInfo[t] = e | (i << 16) for the i-th tile of expert e and
 * 0xFFFFFFFF for total <= t < max_num_tiles (entries past max_num_tiles are
 * never written). Stage 1 writes the starts and the 0xFFFFFFFF tail; stage 2
 * the tiles from the caller's TileStart; the fused stage 2 only each expert's
 * first tile. Replace launch_expt_data_stage1 / _stage2 / _stage2_fused /
 * _compute (kernels/moe-routing/moe_expt_data/kernel.cpp:110-196). */
int hkq_expt_data_stage1(const int32_t* Hist, int32_t* TokenStart, int32_t* TileStart, uint32_t* MDTileInfo,
                         int64_t n_expts_tot, int64_t max_num_tiles, int64_t n_gates, int tile_dim_log2,
                         hkq_stream_t stream);
int hkq_expt_data_stage2(const int32_t* Hist, const int32_t* TileStart, uint32_t* TileInfo, int64_t n_expts_tot,
                         int tile_dim_log2, hkq_stream_t stream);
int hkq_expt_data_stage2_fused(const int32_t* Hist, const int32_t* TileStart, uint32_t* TileInfo, int64_t n_expts_tot,
                               hkq_stream_t stream);
int hkq_expt_data_compute(const int32_t* Hist, int32_t* TokenStart, int32_t* TileStart, uint32_t* MDTileInfo,
                          int64_t n_expts_tot, int64_t max_num_tiles, int64_t n_gates, int tile_dim_log2,
                          int use_fused_stage2, hkq_stream_t stream);

/* Gate placement (1 <= n_expts_act <= 16): gate g of ExptIndx (flattened
 * [tokens, n_expts_act], expert ids < 1024) in 128-token block b = g / (128 *
 * n_expts_act) goes to pos = TokensStart[e] + PartialOffs[b*stride_pm +
 * e*stride_pn] + (gates of e before g in block b); ScatterIndx[g] = pos,
 * GatherIndx[pos] = g, GateScal[pos] = ExptScal[g] (bf16; both NULL: skipped).
 * Gates with an id outside [0, 1024) (e.g. -1) get ScatterIndx = -1. The fused
 * form takes no PartialOffs and counts across blocks itself, for any n_gates
 * (the reference's handles one block). Replace launch_routing_compute_indx /
 * _fused (kernels/moe-routing/moe_routing/kernel.cpp:209-306). */
int hkq_routing_compute_indx(int32_t* GatherIndx, int32_t* ScatterIndx, void* GateScal, const void* ExptScal,
                             const int32_t* ExptIndx, const int32_t* PartialOffs, int64_t stride_pm,
                             int64_t stride_pn, const int32_t* TokensStart, int64_t n_gates, int n_expts_act,
                             hkq_stream_t stream);
int hkq_routing_compute_indx_fused(int32_t* GatherIndx, int32_t* ScatterIndx, void* GateScal, const void* ExptScal,
                                   const int32_t* ExptIndx, const int32_t* TokensStart, int64_t n_gates,
                                   int n_expts_act, hkq_stream_t stream);

/* Block-padded expert order of numel expert ids (num_experts <= 1024):
 * cumsum_buffer[e] = sum_{e' < e} ceil(c[e'] / block_size) * block_size with
 * c = per-expert counts, total_tokens_post_pad[0] = cumsum_buffer[E];
 * sorted_token_ids[cumsum[e] + i] = index of the i-th id equal to e (input
 * order), padded slots = numel; expert_ids[j] = e for the blocks of expert e.
 * Ids outside [0, E) are skipped. tokens_cnts_buffer ((E + 1) * E int32) is
 * scratch. sorted_token_ids needs total entries (at most numel + E *
 * (block_size - 1)). Replaces launch_moe_align_block_size
 * (kernels/moe-routing/moe_align_block_size/kernel.cpp:131-181). */
int hkq_moe_align_block_size(const int32_t* topk_ids, int32_t* sorted_token_ids, int32_t* expert_ids,
                             int32_t* tokens_cnts_buffer, int32_t* cumsum_buffer, int32_t* total_tokens_post_pad,
                             int64_t num_experts, int64_t block_size, int64_t numel, hkq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HKQ_H */
