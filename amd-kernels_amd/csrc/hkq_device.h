// hkq_device.h -- device-side helpers shared by the quantizer, GEMM and MoE
// kernels (gfx950 / CDNA4 only).
//
// Conventions used throughout:
//   * bf16 tensors are handled as raw uint16 bit patterns;
//   * FP8 is OCP E4M3FN (max 448, NaN 0x7F/0xFF, no infinities);
//   * FP4 is OCP E2M1, two codes per byte, the even K index in the low nibble;
//   * E8M0 scales are biased exponents: value 2^(code - 127).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hkq {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

#define HKQ_LDS __attribute__((address_space(3)))

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even; NaN keeps its payload top bits and
// is forced quiet (bit 6 of the bf16 mantissa).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) | 0x40u) & 0xFFFFu;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

// Two fp32 -> two bf16 (round to nearest even) packed as lo | hi << 16: one
// v_cvt_pk_bf16_f32. Finite values round exactly as f32_to_bf16; NaN comes out
// as a quiet NaN (payload bits not guaranteed).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// IEEE maxNum / minNum (a NaN operand is ignored): v_max_f32 / v_min_f32 under
// the default IEEE mode, the semantics of fmaxf/fminf.
__device__ __forceinline__ float max_num(float a, float b) { return __builtin_fmaxf(a, b); }
__device__ __forceinline__ float min_num(float a, float b) { return __builtin_fminf(a, b); }

// Two fp32 -> two OCP E4M3FN codes (round to nearest even) packed in the low
// 16 bits. Callers clamp to [-448, 448] first, so the saturation mode of the
// converter never matters and NaN cannot reach it.
__device__ __forceinline__ uint32_t cvt_pk_e4m3(float a, float b) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}

// Four values -> four E4M3FN codes, value j in byte j: the second pair is
// converted into the high half of the first pair's result (word select), so no
// shift or mask is needed.
__device__ __forceinline__ uint32_t cvt_pk4_e4m3(float a, float b, float c, float d) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false), true);
}

// Eight values (already multiplied by the block's 2^-e) -> eight E2M1 codes,
// value j in nibble j. The rule: round to nearest even on the grid
// {0, .5, 1, 1.5, 2, 3, 4, 6}, saturating at 6, sign from the sign bit, NaN ->
// +6 (code 0x7). v_cvt_scalef32_pk_fp4_f32 with scale 1.0 implements it except
// for NaN, whose sign it keeps (checked on the GPU against a compare-based
// encoder over every tie +-3 ulp and 2^20 random values), so values go through
// min(v, 6) first: NaN becomes +6 (the minimum of a NaN and a number is the
// number), and values above 6 saturate to the same code either way.
__device__ __forceinline__ uint32_t e2m1_encode8(const float* v) {
    uint32_t w = 0;
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = min_num(v[j], 6.0f);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a[0], a[1], 1.0f, 0);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a[2], a[3], 1.0f, 1);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a[4], a[5], 1.0f, 2);
    w = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a[6], a[7], 1.0f, 3);
    return w;
}

// E2M1 codes of 8 values (value j in nibble j) by the threshold ladder of the
// reference's fused MXFP4 quantizer (quantization/fused_mxfp4_quant/
// kernel.cpp:128-150): the largest grid magnitude at or below |v| (6 from 6 up,
// 0 below 0.5; NaN fails every comparison: 0), the sign bit of v kept.
__device__ __forceinline__ uint32_t e2m1_floor8(const float* v) {
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float a = __builtin_fabsf(v[j]);
        const uint32_t m = (uint32_t)(a >= 0.5f) + (uint32_t)(a >= 1.0f) + (uint32_t)(a >= 1.5f) +
                           (uint32_t)(a >= 2.0f) + (uint32_t)(a >= 3.0f) + (uint32_t)(a >= 4.0f) + (uint32_t)(a >= 6.0f);
        w |= (m | ((__float_as_uint(v[j]) >> 28) & 8u)) << (4 * j);
    }
    return w;
}

// Unbiased shared exponent of the MXFP4 scale rule: P = (bits(amax) + 0x200000)
// & 0xFF800000 (amax rounded up at the E2M1 mantissa), e = exponent(P) - 2,
// clamped to [-127, 127]; amax = 0 gives -127 (code 0), amax -> inf gives 127.
__device__ __forceinline__ int mx_scale_exp(float amax) {
    uint32_t p = (__float_as_uint(amax) + 0x200000u) & 0xFF800000u;
    int ep = (int)(p >> 23) & 0xFF;
    int e = ep - 129;
    e = e < -127 ? -127 : e;
    return ep == 255 ? 127 : e;
}

// 2^k for k in [-127, 127] as an exact fp32 (2^-127 is subnormal).
__device__ __forceinline__ float exp2i(int k) {
    return k == -127 ? __uint_as_float(0x00400000u) : __uint_as_float((uint32_t)(k + 127) << 23);
}

// 16-byte streaming load (read once: non-temporal hint).
__device__ __forceinline__ uint4 ld_stream16(const void* p) {
    v4i v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
    return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}

// Buffer resource over [base, base + bytes): loads at offsets >= bytes return
// zero, which is how every kernel masks rows past M/N and columns past K.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Value of v in the partner lane of a butterfly step over aligned groups of
// 2*H lanes (H = 1, 2, 4, 8: DPP quad_perm [1,0,3,2] / [2,3,0,1], half-row
// mirror, row mirror; 16: ds_swizzle xor 16; 32: bpermute xor 32). The mirror
// steps pair lane i with 2H-1-i instead of i^H; once the previous steps have
// made every H-lane subgroup uniform, both pairings combine the same values.
template <int H>
__device__ __forceinline__ float butterfly_partner(float v) {
    const int x = __float_as_int(v);
    if constexpr (H == 1) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
    else if constexpr (H == 2) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
    else if constexpr (H == 4) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false));
    else if constexpr (H == 8) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false));
    else if constexpr (H == 16) return __int_as_float(__builtin_amdgcn_ds_swizzle(x, 0x401F));
    else return __shfl_xor(v, 32, 64);
}

// Maximum over groups of W adjacent lanes (W a power of two <= 64, all lanes
// active, the result in every lane of the group) of values that are +0 or
// positive and never NaN (absolute maxima accumulated from 0 with max_num):
// their bit patterns order as unsigned integers, so each butterfly step is one
// integer max of the DPP-moved value, with no NaN quieting around it.
template <int W>
__device__ __forceinline__ float group_max_abs(float v) {
    uint32_t x = __float_as_uint(v);
    auto step = [&](float o) {
        const uint32_t y = __float_as_uint(o);
        x = x > y ? x : y;
    };
    if constexpr (W >= 2) step(butterfly_partner<1>(__uint_as_float(x)));
    if constexpr (W >= 4) step(butterfly_partner<2>(__uint_as_float(x)));
    if constexpr (W >= 8) step(butterfly_partner<4>(__uint_as_float(x)));
    if constexpr (W >= 16) step(butterfly_partner<8>(__uint_as_float(x)));
    if constexpr (W >= 32) step(butterfly_partner<16>(__uint_as_float(x)));
    if constexpr (W >= 64) step(butterfly_partner<32>(__uint_as_float(x)));
    return __uint_as_float(x);
}

// max_num(m / 448, 1e-10) for m >= 0 (the E4M3 group-scale rule), with the
// division done as q0 = RN(m * RN(1/448)), its remainder m - 448 q0 exact by
// an FMA, then q0 + remainder * RN(1/448): 3 FMA-unit instructions instead of
// the IEEE division sequence's ~11. Equal to the IEEE result for every finite
// m >= 0 (checked exhaustively on the host and on MI355X; quotients that
// differ are subnormal, below the 1e-10 floor); +inf gives +inf.
__device__ __forceinline__ float fp8_group_scale(float m) {
    constexpr float R448 = 1.0f / 448.0f;
    const float q0 = m * R448;
    const float q = __builtin_fmaf(__builtin_fmaf(-q0, 448.0f, m), R448, q0);
    return m == __builtin_inff() ? m : max_num(q, 1e-10f);
}

// 1 / s correctly rounded for s in [1e-10, 2^127) and s = +inf: v_rcp_f32 and
// one FMA correction step (checked against the IEEE division for every s in
// [1e-10, 2^127) on MI355X; from 2^127 up the reciprocal is subnormal and the
// step is not exact).
__device__ __forceinline__ float recip_scale(float s) {
    const float r0 = __builtin_amdgcn_rcpf(s);
    const float r1 = __builtin_fmaf(__builtin_fmaf(-s, r0, 1.0f), r0, r0);
    return s == __builtin_inff() ? 0.0f : r1;
}

// Sum by the same butterfly: every lane of the group ends with the same bits,
// equal to the xor butterfly (v += v[lane ^ o] for o = 1, 2, ..., W/2).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (W >= 2) v = v + butterfly_partner<1>(v);
    if constexpr (W >= 4) v = v + butterfly_partner<2>(v);
    if constexpr (W >= 8) v = v + butterfly_partner<4>(v);
    if constexpr (W >= 16) v = v + butterfly_partner<8>(v);
    if constexpr (W >= 32) v = v + butterfly_partner<16>(v);
    if constexpr (W >= 64) v = v + butterfly_partner<32>(v);
    return v;
}

// n / d with C's truncation toward zero, for |n| < 2^31 and 1 <= d < 2^16,
// from r = 1.0 / d rounded to double (3 VALU instructions instead of an
// integer division's ~20): |n * r - n / d| <= 2^31 * 2^-52 = 2^-21, and a
// quotient that is not an integer lies at least 1/d > 2^-16 from the
// integers, so moving 2^-20 away from zero before truncating gives the exact
// quotient in both cases.
__device__ __forceinline__ int div_recip(int n, double r) {
    const double x = (double)n * r;
    return (int)(n >= 0 ? x + 0x1p-20 : x - 0x1p-20);
}

}  // namespace hkq
