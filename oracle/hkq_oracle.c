/*
 * hkq_oracle.c -- CPU restatement of the reference's quantized-GEMM arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product path may link or call this
 * file; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * use it, and only as the checker (or the timed CPU baseline).
 *
 * Plain scalar C, written for clarity, not speed. Every routine cites the
 * reference formula it restates (paths relative to the reference repository).
 * How each routine is pinned (library routine / closed form / brute force) is
 * listed in oracle/oracle.py's header and exercised by tests/test_oracle_*.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float bits2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* fmaxf/fminf with IEEE maxNum semantics (a NaN operand is ignored), as the
 * reference's device fmaxf/fminf (quantization/quant/kernel.cpp:51,106). */
static inline float max_num(float a, float b) { return isnan(b) ? a : (isnan(a) ? b : (a > b ? a : b)); }
static inline float min_num(float a, float b) { return isnan(b) ? a : (isnan(a) ? b : (a < b ? a : b)); }

float orc_bf16_to_f32(uint16_t h) { return bits2f((uint32_t)h << 16); }

/* fp32 -> bf16, round to nearest even (the rounding of __float2bfloat16 used by
 * every reference epilogue, e.g. moe-gemm/moe_op_gemm_a8w8/kernel.cpp:167). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f2bits(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* OCP E4M3FN encode, round to nearest even, saturating at +-448; NaN -> 0x7F|sign.
 * Replaces the reference's placeholder encoders (quantization/fused_fp8_quant/
 * kernel.cpp:206 writes an affine byte; moe-misc/quant_moe/kernel.cpp:62-71
 * truncates). Its oracle is the reference test's own encoder,
 * torch.float8_e4m3fn (tests/test_moe.py:997-999). */
uint8_t orc_e4m3fn_encode(float x) {
    uint32_t u = f2bits(x);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint8_t)(sign | 0x7Fu);
    if (a >= 0x43E00000u) return (uint8_t)(sign | 0x7Eu);       /* >= 448 */
    if (a >= 0x3C800000u) {                                      /* >= 2^-6: normal */
        uint32_t v = a >> 20;                                    /* exp8 | top 3 mantissa bits */
        uint32_t rem = a & 0xFFFFFu;
        if (rem > 0x80000u || (rem == 0x80000u && (v & 1u))) v++;
        return (uint8_t)(sign | (uint8_t)(v - (120u << 3)));     /* rebias 127 -> 7 */
    }
    /* subnormal: n * 2^-9, n in [0, 8]; the scaling by 512 is exact */
    float n = rintf(bits2f(a) * 512.0f);
    return (uint8_t)(sign | (uint8_t)n);
}

float orc_e4m3fn_decode(uint8_t c) {
    int e = (c >> 3) & 0xF, m = c & 7;
    float v;
    if (e == 15 && m == 7) v = NAN;
    else if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return (c & 0x80) ? -v : v;
}

/* E2M1 encode, round to nearest even onto {0,.5,1,1.5,2,3,4,6}, saturating at 6;
 * sign taken from the sign bit (as quantization/fused_mxfp4_quant/kernel.cpp:
 * 121-152 does); NaN -> +6 (code 0x7). The reference kernel floors onto the
 * grid (:131-147); the OCP MX rounding is to nearest even (ties listed below). */
uint8_t orc_e2m1_encode(float q) {
    if (isnan(q)) return 0x7;
    uint8_t sign = (uint8_t)((f2bits(q) >> 31) << 3);
    float a = fabsf(q);
    uint8_t m;
    if (a <= 0.25f) m = 0;          /* tie 0.25 -> 0   (even) */
    else if (a < 0.75f) m = 1;      /* tie 0.75 -> 1.0 */
    else if (a <= 1.25f) m = 2;     /* tie 1.25 -> 1.0 */
    else if (a < 1.75f) m = 3;      /* tie 1.75 -> 2.0 */
    else if (a <= 2.5f) m = 4;      /* tie 2.5  -> 2.0 */
    else if (a < 3.5f) m = 5;       /* tie 3.5  -> 4.0 */
    else if (a <= 5.0f) m = 6;      /* tie 5.0  -> 4.0 */
    else m = 7;
    return (uint8_t)(sign | m);
}

/* E2M1 encode by the threshold ladder of the reference's fused MXFP4
 * quantizer (quantization/fused_mxfp4_quant/kernel.cpp:128-150): the largest
 * grid magnitude at or below |q| (6 from 6 up, 0 below 0.5), sign bit of q
 * added (so -0 and a NaN with the sign bit set give 0x8); NaN fails every
 * comparison: magnitude code 0. */
uint8_t orc_e2m1_floor(float q) {
    const uint8_t sign = (uint8_t)((f2bits(q) >> 31) << 3);
    const float a = fabsf(q);
    uint8_t m;
    if (a >= 6.0f) m = 0x7;
    else if (a >= 4.0f) m = 0x6;
    else if (a >= 3.0f) m = 0x5;
    else if (a >= 2.0f) m = 0x4;
    else if (a >= 1.5f) m = 0x3;
    else if (a >= 1.0f) m = 0x2;
    else if (a >= 0.5f) m = 0x1;
    else m = 0x0;
    return (uint8_t)(sign | m);
}

/* E2M1 value table (moe-gemm/moe_op_mxfp4/kernel.cpp:32-35). */
float orc_e2m1_decode(uint8_t nib) {
    static const float lut[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    float v = lut[nib & 7];
    return (nib & 8) ? -v : v;
}

/* E8M0 decode per the OCP MX spec: 2^(s-127), 0xFF = NaN. (The reference's
 * decode_mx_scale maps 0 -> 0 and 255 -> inf, moe-gemm/moe_op_mxfp4/kernel.cpp:
 * 77-88; neither code is produced by the quantizers below for finite input
 * except code 0 for an all-zero block, whose elements are all zero.) */
float orc_e8m0_decode(uint8_t s) {
    if (s == 0xFF) return NAN;
    return ldexpf(1.0f, (int)s - 127);
}

/* MXFP4 shared-exponent rule of quantization/fused_mxfp4_quant/kernel.cpp:
 * 99-105 (and :238-243): P = (bits(amax) + 0x200000) & 0xFF800000,
 * e = clamp(floor(log2 P) - 2, -127, 127). Restated on the exponent field
 * E of P: e = clamp(E - 129, -127, 127); E = 255 (amax rounds to inf) gives
 * 127, as the float rule does; amax = 0 gives -127 (code 0), where the float
 * rule is undefined (log2 0). */
int orc_mx_scale_exp(float amax) {
    uint32_t p = (f2bits(amax) + 0x200000u) & 0xFF800000u;
    int ep = (int)((p >> 23) & 0xFF);
    if (ep == 255) return 127;
    int e = ep - 129;
    return e < -127 ? -127 : e;
}

/* Row-wise dynamic quantization in groups of `group` columns.
 *   amax = max|x| over the group; s = fmaxf(amax / QMAX, 1e-10f);
 *   r = 1.0f / s; q = encode(clamp(x * r, -QMAX, QMAX))
 * per quantization/quant/kernel.cpp:46-107 (group = K, per-token) and
 * quantization/fused_fp8_quant/kernel.cpp:157-204 (group = 128, RMSNorm
 * omitted). kind 0: QMAX = 448, OCP e4m3fn RNE code; kind 1: QMAX = 127,
 * int8 = (int8)rintf(.) clamped (quant/kernel.cpp:105-107).
 * x bf16 bits [M, ldx]; q [M, ldq]; s fp32 [M, lds] with K/group per row. */
void orc_quant_rowwise(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int64_t group,
                       int kind, uint8_t* q, int64_t ldq, float* s, int64_t lds) {
    const float qmax = kind == 0 ? 448.0f : 127.0f;
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t g0 = 0; g0 < K; g0 += group) {
            float amax = 0.0f;
            for (int64_t k = g0; k < g0 + group; ++k)
                amax = max_num(amax, fabsf(orc_bf16_to_f32(x[m * ldx + k])));
            float sc = max_num(amax / qmax, 1e-10f);
            float r = 1.0f / sc;
            s[m * lds + g0 / group] = sc;
            for (int64_t k = g0; k < g0 + group; ++k) {
                float v = orc_bf16_to_f32(x[m * ldx + k]) * r;
                if (kind == 0) {
                    v = max_num(min_num(v, qmax), -qmax);
                    q[m * ldq + k] = orc_e4m3fn_encode(v);
                } else {
                    v = rintf(v);
                    v = max_num(min_num(v, qmax), -qmax);
                    q[m * ldq + k] = (uint8_t)(int8_t)v;
                }
            }
        }
    }
}

/* Static-scale FP8 downcast: y = e4m3(clamp(x / scale, +-448))
 * (moe-misc/quant_moe/kernel.cpp:50-53,93-100), RNE encoder in place of the
 * truncating one. */
void orc_static_fp8(const uint16_t* x, int64_t n, float scale, uint8_t* y) {
    for (int64_t i = 0; i < n; ++i) {
        float v = orc_bf16_to_f32(x[i]) / scale;
        v = max_num(-448.0f, min_num(448.0f, v));
        y[i] = orc_e4m3fn_encode(v);
    }
}

/* MXFP4 quantization of bf16 [M, K] (K % 32 == 0): e8m0 code per 32 columns
 * (orc_mx_scale_exp + 127), elements e2m1(x * 2^-e) RNE, two per byte with
 * the even column in the low nibble (fused_mxfp4_quant/kernel.cpp:155-162).
 * q [M, K/2], s [M, K/32]. */
void orc_mx_quant_fp4(const uint16_t* x, int64_t M, int64_t K, uint8_t* q, uint8_t* s) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t b = 0; b < K / 32; ++b) {
            const uint16_t* xb = x + m * K + b * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) amax = max_num(amax, fabsf(orc_bf16_to_f32(xb[i])));
            int e = orc_mx_scale_exp(amax);
            s[m * (K / 32) + b] = (uint8_t)(e + 127);
            for (int i = 0; i < 32; i += 2) {
                uint8_t lo = orc_e2m1_encode(ldexpf(orc_bf16_to_f32(xb[i]), -e));
                uint8_t hi = orc_e2m1_encode(ldexpf(orc_bf16_to_f32(xb[i + 1]), -e));
                q[m * (K / 2) + b * 16 + i / 2] = (uint8_t)(lo | (hi << 4));
            }
        }
    }
}

/* MX-FP8 quantization (downcast_to_mxfp, is_fp4 = false): scale code =
 * exponent field of amax/448 rounded up to a power of two, 0xFF for amax = 0
 * (moe-misc/quant_moe/kernel.cpp:143-161); element = e4m3(clamp(x * (1/2^(c-127))))
 * with quant scale 0 for code 0 (:199-217). q [M, K], s [M, K/32]. */
void orc_mx_quant_fp8(const uint16_t* x, int64_t M, int64_t K, uint8_t* q, uint8_t* s) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t b = 0; b < K / 32; ++b) {
            const uint16_t* xb = x + m * K + b * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) amax = max_num(amax, fabsf(orc_bf16_to_f32(xb[i])));
            uint8_t code;
            if (amax == 0.0f) code = 0xFF;
            else code = (uint8_t)(((f2bits(amax / 448.0f) + 0x007FFFFFu) & 0x7F800000u) >> 23);
            s[m * (K / 32) + b] = code;
            float deq = bits2f((uint32_t)code << 23);
            float qs = (code == 0xFF) ? 0.0f : (deq == 0.0f ? 0.0f : 1.0f / deq);
            for (int i = 0; i < 32; ++i) {
                float v = orc_bf16_to_f32(xb[i]) * qs;
                v = max_num(-448.0f, min_num(448.0f, v));
                q[m * K + b * 32 + i] = orc_e4m3fn_encode(v);
            }
        }
    }
}

/* MX dequantization to bf16 (upcast_from_mxfp, moe-misc/quant_moe/kernel.cpp:
 * 290-359): out = decode(elem) * 2^(s-127) rounded to bf16; s = 0xFF -> NaN.
 * FP4 elements are decoded with the e2m1 table (the reference stub writes 0,
 * :345-349). q [M, K] (fp8) or [M, K/2] (fp4), s [M, K/32], out bf16 [M, K]. */
void orc_mx_dequant(const uint8_t* q, const uint8_t* s, int64_t M, int64_t K, int is_fp4,
                    uint16_t* out) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t k = 0; k < K; ++k) {
            uint8_t sc = s[m * (K / 32) + k / 32];
            float v;
            if (sc == 0xFF) v = NAN;
            else {
                float e;
                if (is_fp4) {
                    uint8_t byte = q[m * (K / 2) + k / 2];
                    e = orc_e2m1_decode((k & 1) ? (byte >> 4) : (byte & 0xF));
                } else {
                    e = orc_e4m3fn_decode(q[m * K + k]);
                }
                v = e * orc_e8m0_decode(sc);
            }
            out[m * K + k] = orc_f32_to_bf16(v);
        }
    }
}

/* Bulk decoders used by the GEMM references (oracle/oracle.py). */
void orc_e4m3fn_decode_array(const uint8_t* c, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_e4m3fn_decode(c[i]);
}

/* Dequantize MXFP4 [R, K/2] codes with [R, K/32] e8m0 scales to fp32 [R, K]. */
void orc_mx_fp4_dequant_f32(const uint8_t* q, const uint8_t* s, int64_t R, int64_t K, float* out) {
    for (int64_t r = 0; r < R; ++r)
        for (int64_t k = 0; k < K; ++k) {
            uint8_t byte = q[r * (K / 2) + k / 2];
            float e = orc_e2m1_decode((k & 1) ? (byte >> 4) : (byte & 0xF));
            out[r * K + k] = e * orc_e8m0_decode(s[r * (K / 32) + k / 32]);
        }
}

/* Bulk codec entry points for the vectorised pinning tests. */
void orc_e4m3fn_encode_array(const float* x, int64_t n, uint8_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_e4m3fn_encode(x[i]);
}

void orc_e2m1_encode_array(const float* x, int64_t n, uint8_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_e2m1_encode(x[i]);
}

void orc_e2m1_floor_array(const float* x, int64_t n, uint8_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_e2m1_floor(x[i]);
}

void orc_mx_scale_exp_array(const float* amax, int64_t n, int32_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_mx_scale_exp(amax[i]);
}

/* ---- quantizers fused with their producer ---------------------------------- */

/* RMSNorm + quantization (quantization/fused_fp8_quant/kernel.cpp:37-204,
 * fused_mxfp4_quant/kernel.cpp:40-243): y = x * rsqrt(mean(x^2) + eps) * w,
 * then the 1x128 FP8 rule (kind 0) or the MXFP4 rule with elements rounded to
 * nearest even (kind 1) or floored by the reference's ladder (kind 2,
 * fused_mxfp4_quant/kernel.cpp:128-150; orc_e2m1_floor). The reference
 * leaves the summation order and the rsqrt rounding open (a 256-thread tree,
 * an approximate rsqrtf); this restatement fixes both as the product does so
 * the codes can be compared bit for bit: 64 partial sums, partial l an fmaf
 * chain over columns 8c .. 8c+7 of the chunks c = l, l + 64, ..., then an xor
 * butterfly (partial l += partial l^o for o = 1, 2, ..., 32); r = 1 / sqrtf(sum
 * / D + eps) correctly rounded; y = (x * r) * w. x, w bf16 bits; q, s as the
 * product writes them (s fp32 per 128 columns, or e8m0 bytes per 32). */
void orc_rmsnorm_quant(const uint16_t* x, const uint16_t* w, int64_t M, int64_t D, float eps, int kind, uint8_t* q,
                       void* s) {
    const int64_t nch = D / 8;
    float* y = (float*)malloc(sizeof(float) * (size_t)D);
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* xr = x + m * D;
        float part[64];
        for (int l = 0; l < 64; ++l) {
            float acc = 0.0f;
            for (int64_t c = l; c < nch; c += 64)
                for (int j = 0; j < 8; ++j) {
                    const float v = orc_bf16_to_f32(xr[c * 8 + j]);
                    acc = fmaf(v, v, acc);
                }
            part[l] = acc;
        }
        for (int o = 1; o < 64; o <<= 1) {
            float nxt[64];
            for (int l = 0; l < 64; ++l) nxt[l] = part[l] + part[l ^ o];
            memcpy(part, nxt, sizeof(part));
        }
        const float r = 1.0f / sqrtf(part[0] / (float)D + eps);
        for (int64_t k = 0; k < D; ++k) y[k] = (orc_bf16_to_f32(xr[k]) * r) * orc_bf16_to_f32(w[k]);
        if (kind == 0) {
            for (int64_t g0 = 0; g0 < D; g0 += 128) {
                float amax = 0.0f;
                for (int64_t k = g0; k < g0 + 128; ++k) amax = max_num(amax, fabsf(y[k]));
                const float sc = max_num(amax / 448.0f, 1e-10f);
                const float rc = 1.0f / sc;
                ((float*)s)[m * (D / 128) + g0 / 128] = sc;
                for (int64_t k = g0; k < g0 + 128; ++k)
                    q[m * D + k] = orc_e4m3fn_encode(max_num(min_num(y[k] * rc, 448.0f), -448.0f));
            }
        } else {
            for (int64_t g0 = 0; g0 < D; g0 += 32) {
                float amax = 0.0f;
                for (int64_t k = g0; k < g0 + 32; ++k) amax = max_num(amax, fabsf(y[k]));
                const int e = orc_mx_scale_exp(amax);
                const float mul = ldexpf(1.0f, -e);
                ((uint8_t*)s)[m * (D / 32) + g0 / 32] = (uint8_t)(e + 127);
                for (int64_t k = g0; k < g0 + 32; k += 2) {
                    const uint8_t lo = kind == 2 ? orc_e2m1_floor(y[k] * mul) : orc_e2m1_encode(y[k] * mul);
                    const uint8_t hi = kind == 2 ? orc_e2m1_floor(y[k + 1] * mul) : orc_e2m1_encode(y[k + 1] * mul);
                    q[m * (D / 2) + k / 2] = (uint8_t)(lo | (hi << 4));
                }
            }
        }
    }
    free(y);
}

/* SwiGLU + FP8 quantization: act = silu(g) * u, silu(g) = g / (1 + exp2f(-1.44269504089f
 * * alpha * g)) (moe-gemm/moe_op_gemm_a8w8/kernel.cpp:57-59), (g, u) = columns (k, F + k)
 * or (2k, 2k + 1) when interleaved (moe-gemm/moe_op_silu_fused/kernel.cpp:9-12);
 * then per row (group 0) or per 128 columns s = max(amax/448, 1e-10),
 * q = E4M3FN(clamp(act * (1/s), +-448)). y bf16 bits [M, 2F]; act fp32 [M, F]
 * is returned too (NULL: not). */
void orc_swiglu_quant(const uint16_t* y, int64_t M, int64_t F, float alpha, int interleaved, int group, uint8_t* q,
                      float* s, float* act_out) {
    float* act = (float*)malloc(sizeof(float) * (size_t)F);
    const int64_t G = group ? group : F;
    for (int64_t m = 0; m < M; ++m) {
        const uint16_t* yr = y + m * 2 * F;
        for (int64_t k = 0; k < F; ++k) {
            const float g = orc_bf16_to_f32(interleaved ? yr[2 * k] : yr[k]);
            const float u = orc_bf16_to_f32(interleaved ? yr[2 * k + 1] : yr[F + k]);
            act[k] = g / (1.0f + exp2f(-1.44269504089f * alpha * g)) * u;
            if (act_out) act_out[m * F + k] = act[k];
        }
        for (int64_t g0 = 0; g0 < F; g0 += G) {
            float amax = 0.0f;
            for (int64_t k = g0; k < g0 + G; ++k) amax = max_num(amax, fabsf(act[k]));
            const float sc = max_num(amax / 448.0f, 1e-10f);
            const float rc = 1.0f / sc;
            s[group ? m * (F / G) + g0 / G : m] = sc;
            for (int64_t k = g0; k < g0 + G; ++k)
                q[m * F + k] = orc_e4m3fn_encode(max_num(min_num(act[k] * rc, 448.0f), -448.0f));
        }
    }
    free(act);
}
