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

// E2M1 code of q (round to nearest even on the grid {0,.5,1,1.5,2,3,4,6},
// saturating at 6; sign from the sign bit; NaN -> +6). Branch-free compares.
__device__ __forceinline__ uint32_t e2m1_encode(float q) {
    float a = __builtin_fabsf(q);
    uint32_t m = (a > 0.25f) + (a >= 0.75f) + (a > 1.25f) + (a >= 1.75f) + (a > 2.5f) + (a >= 3.5f) + (a > 5.0f);
    m = (q != q) ? 7u : m;
    uint32_t s = (q != q) ? 0u : ((__float_as_uint(q) >> 28) & 8u);
    return s | m;
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

// Wave-level reductions over groups of W adjacent lanes (W a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = 1; o < W; o <<= 1) v = max_num(v, __shfl_xor(v, o, 64));
    return v;
}

}  // namespace hkq
