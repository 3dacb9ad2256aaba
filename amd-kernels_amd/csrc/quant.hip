// quant.hip -- activation quantizers (HBM-bound; one read of the input, one
// write of codes + scales, 16-byte vector loads, wave-shuffle amax).
//
// Kernels and the reference arithmetic each restates:
//   rowwise_group_kernel  per-token (group = K) and 1 x G group quantization,
//                         quantization/quant/kernel.cpp:46-107 (per-token, int8
//                         QMAX 127) and quantization/fused_fp8_quant/kernel.cpp:
//                         190-204 (1x128, QMAX 448) with a real E4M3FN encoder;
//   static_fp8_kernel     moe-misc/quant_moe/kernel.cpp:75-104 (x / scale[0]);
//   mx_quant_kernel       MXFP4: quantization/fused_mxfp4_quant/kernel.cpp:97-162
//                         (scale rule, nibble packing), RNE element rounding;
//                         MXFP8: moe-misc/quant_moe/kernel.cpp:143-217;
//   mx_dequant_kernel     moe-misc/quant_moe/kernel.cpp:290-359 with working
//                         E4M3 and E2M1 decoders.
#include "hkq_device.h"
#include "hkq_host.h"

namespace hkq {

// --------------------------------------------------------------------------
// Row-wise dynamic quantization.
//
// Per-token (one group per row): a workgroup of 256 threads owns a row, keeps
// it in registers (CHUNKS x 8 bf16 per thread), reduces amax across the block,
// then encodes from registers -- one HBM read per element.
// --------------------------------------------------------------------------
enum { KIND_FP8 = 0, KIND_INT8 = 1 };

template <int KIND>
__device__ __forceinline__ uint32_t encode4(float a, float b, float c, float d, float r) {
    const float qmax = KIND == KIND_FP8 ? 448.0f : 127.0f;
    float v[4] = {a * r, b * r, c * r, d * r};
    if (KIND == KIND_FP8) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = max_num(min_num(v[i], qmax), -qmax);
        return cvt_pk4_e4m3(v[0], v[1], v[2], v[3]);
    } else {
        uint32_t out = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float q = max_num(min_num(__builtin_rintf(v[i]), qmax), -qmax);
            out |= ((uint32_t)(int32_t)q & 0xFFu) << (8 * i);
        }
        return out;
    }
}

template <int KIND>
__device__ __forceinline__ uint2 encode8(const uint4& x, float r) {
    uint2 o;
    o.x = encode4<KIND>(bf16_to_f32(x.x & 0xFFFF), bf16_to_f32(x.x >> 16), bf16_to_f32(x.y & 0xFFFF),
                        bf16_to_f32(x.y >> 16), r);
    o.y = encode4<KIND>(bf16_to_f32(x.z & 0xFFFF), bf16_to_f32(x.z >> 16), bf16_to_f32(x.w & 0xFFFF),
                        bf16_to_f32(x.w >> 16), r);
    return o;
}

__device__ __forceinline__ float amax8(const uint4& x) {
    float m = 0.0f;
    uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m = max_num(m, __builtin_fabsf(bf16_to_f32(w[i] & 0xFFFF)));
        m = max_num(m, __builtin_fabsf(bf16_to_f32(w[i] >> 16)));
    }
    return m;
}

// Per-token: grid = (M), block = 256; CHUNKS = ceil(K / 8 / 256).
template <int KIND, int CHUNKS>
__global__ __launch_bounds__(256) void per_token_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                        float* __restrict__ s, int64_t K, int64_t ldx, int64_t ldq) {
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t nch = K >> 3;
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
    uint4 v[CHUNKS];
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
        int64_t ch = tid + c * 256;
        v[c] = ch < nch ? ld_stream16(xr + ch) : make_uint4(0, 0, 0, 0);
        m = max_num(m, amax8(v[c]));
    }
    m = group_max_abs<64>(m);
    __shared__ float red[4];
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = max_num(max_num(red[0], red[1]), max_num(red[2], red[3]));
    const float qmax = KIND == KIND_FP8 ? 448.0f : 127.0f;
    const float sc = KIND == KIND_FP8 ? fp8_group_scale(m) : max_num(m / qmax, 1e-10f);
    const float r = KIND == KIND_FP8 ? recip_scale(sc) : 1.0f / sc;
    if (tid == 0) s[row] = sc;
    uint2* qr = reinterpret_cast<uint2*>(q + row * ldq);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
        int64_t ch = tid + c * 256;
        if (ch < nch) qr[ch] = encode8<KIND>(v[c], r);
    }
}

// 1 x G groups (G in {32,...,512}, power of two, G/8 lanes per group): every
// thread owns 8 consecutive elements; the G/8 lanes of a group reduce amax with
// xor-shuffles. Grid-stride over all 8-element chunks of the [M, K] matrix.
// Row and column of flat chunk ch (< total + 256) of a matrix with cpr chunks
// per row. When total + 256 < 2^31 and cpr < 2^16 (a wave-uniform test), the
// quotient comes from div_recip (3 VALU instructions) instead of a 64-bit
// integer division (~40).
struct ChunkIndex {
    int64_t cpr;
    double rcpr;
    bool small;
    __device__ ChunkIndex(int64_t cpr_, int64_t total)
        : cpr(cpr_), rcpr(1.0 / (double)cpr_), small(total < 0x7FFFFF00 && cpr_ < 0x10000) {}
    __device__ __forceinline__ void operator()(int64_t ch, int64_t& row, int64_t& col) const {
        row = small ? (int64_t)div_recip((int)ch, rcpr) : ch / cpr;
        col = ch - row * cpr;
    }
};

template <int KIND, int GL>
__global__ __launch_bounds__(256) void group_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                    float* __restrict__ s, int64_t M, int64_t K, int64_t ldx,
                                                    int64_t ldq, int64_t lds) {
    const int64_t cpr = K >> 3;  // chunks per row
    const int64_t total = M * cpr;
    const ChunkIndex index(cpr, total);
    const float qmax = KIND == KIND_FP8 ? 448.0f : 127.0f;
    for (int64_t base = (int64_t)blockIdx.x * 256; base < total; base += (int64_t)gridDim.x * 256) {
        // total is a multiple of GL (K % G == 0) and base of 256, so a whole
        // group is either in range or out of range together.
        const int64_t ch = base + threadIdx.x;
        const bool ok = ch < total;
        int64_t row, col;
        index(ok ? ch : 0, row, col);
        uint4 v = ok ? ld_stream16(reinterpret_cast<const uint4*>(x + row * ldx) + col)
                     : make_uint4(0, 0, 0, 0);
        float m = group_max_abs<GL>(amax8(v));
        const float sc = KIND == KIND_FP8 ? fp8_group_scale(m) : max_num(m / qmax, 1e-10f);
        const float r = KIND == KIND_FP8 ? recip_scale(sc) : 1.0f / sc;
        if (ok) {
            reinterpret_cast<uint2*>(q + row * ldq)[col] = encode8<KIND>(v, r);
            if ((threadIdx.x & (GL - 1)) == 0) s[row * lds + col / GL] = sc;
        }
    }
}

// --------------------------------------------------------------------------
// Static-scale FP8: y = e4m3(clamp(x / scale[0], +-448)). Flat over n elements
// (n % 8 == 0), 8 per thread.
// --------------------------------------------------------------------------
__global__ __launch_bounds__(256) void static_fp8_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ y,
                                                         const float* __restrict__ scale, int64_t n8) {
    const float sc = scale[0];
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
        uint4 v = ld_stream16(reinterpret_cast<const uint4*>(x) + i);
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
        float f[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f[2 * j] = max_num(-448.0f, min_num(448.0f, bf16_to_f32(w[j] & 0xFFFF) / sc));
            f[2 * j + 1] = max_num(-448.0f, min_num(448.0f, bf16_to_f32(w[j] >> 16) / sc));
        }
        uint2 o;
        o.x = cvt_pk4_e4m3(f[0], f[1], f[2], f[3]);
        o.y = cvt_pk4_e4m3(f[4], f[5], f[6], f[7]);
        reinterpret_cast<uint2*>(y)[i] = o;
    }
}

// --------------------------------------------------------------------------
// MX quantization (32-element blocks along the contiguous dim): 4 lanes x 8
// elements per block. FP4: codes packed two per byte (even index low nibble),
// q [M, K/2]; FP8: q [M, K]. Scales e8m0 [M, K/32].
// --------------------------------------------------------------------------
template <bool FP4>
__global__ __launch_bounds__(256) void mx_quant_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                       uint8_t* __restrict__ s, int64_t M, int64_t K, int64_t ldx) {
    const int64_t cpr = K >> 3;
    const int64_t total = M * cpr;
    const ChunkIndex index(cpr, total);
    for (int64_t base = (int64_t)blockIdx.x * 256; base < total; base += (int64_t)gridDim.x * 256) {
        const int64_t ch = base + threadIdx.x;
        const bool ok = ch < total;
        int64_t row, col;
        index(ok ? ch : 0, row, col);
        uint4 v = ok ? ld_stream16(reinterpret_cast<const uint4*>(x + row * ldx) + col)
                     : make_uint4(0, 0, 0, 0);
        const float m = group_max_abs<4>(amax8(v));
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
        if (FP4) {
            const int e = mx_scale_exp(m);
            const float mul = exp2i(-e);  // exact: ldexp(x, -e)
            float t[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                t[2 * j] = bf16_to_f32(w[j] & 0xFFFF) * mul;
                t[2 * j + 1] = bf16_to_f32(w[j] >> 16) * mul;
            }
            const uint32_t packed = e2m1_encode8(t);
            if (ok) {
                reinterpret_cast<uint32_t*>(q + row * (K >> 1))[col] = packed;
                if ((threadIdx.x & 3) == 0) s[row * (K >> 5) + (col >> 2)] = (uint8_t)(e + 127);
            }
        } else {
            // code = exponent field of amax/448 rounded up to a power of two; 0xFF for amax = 0
            uint32_t code = m == 0.0f ? 0xFFu : (((__float_as_uint(m / 448.0f) + 0x007FFFFFu) & 0x7F800000u) >> 23);
            const float deq = __uint_as_float(code << 23);
            const float qs = (code == 0xFFu || deq == 0.0f) ? 0.0f : 1.0f / deq;
            float f[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f[2 * j] = max_num(-448.0f, min_num(448.0f, bf16_to_f32(w[j] & 0xFFFF) * qs));
                f[2 * j + 1] = max_num(-448.0f, min_num(448.0f, bf16_to_f32(w[j] >> 16) * qs));
            }
            if (ok) {
                uint2 o;
                o.x = cvt_pk4_e4m3(f[0], f[1], f[2], f[3]);
                o.y = cvt_pk4_e4m3(f[4], f[5], f[6], f[7]);
                reinterpret_cast<uint2*>(q + row * K)[col] = o;
                if ((threadIdx.x & 3) == 0) s[row * (K >> 5) + (col >> 2)] = (uint8_t)code;
            }
        }
    }
}

__device__ __forceinline__ float e4m3_decode(uint32_t c) {
    const uint32_t e = (c >> 3) & 0xF, m = c & 7;
    float v = e == 0 ? (float)m * 0.001953125f : __uint_as_float(((e + 120) << 23) | (m << 20));
    v = (e == 15 && m == 7) ? __builtin_nanf("") : v;
    return (c & 0x80) ? -v : v;
}

__device__ __forceinline__ float e2m1_decode(uint32_t n) {
    // grid {0, .5, 1, 1.5, 2, 3, 4, 6}: e = n>>1 & 3, m = n & 1
    const uint32_t e = (n >> 1) & 3, m = n & 1;
    float v = e == 0 ? 0.5f * (float)m : __uint_as_float(((e + 126) << 23) | (m << 22));
    return (n & 8) ? -v : v;
}

// out bf16 [M, K] = decode(q) * 2^(s - 127); s = 0xFF -> NaN. 8 outputs per thread.
template <bool FP4>
__global__ __launch_bounds__(256) void mx_dequant_kernel(const uint8_t* __restrict__ q, const uint8_t* __restrict__ s,
                                                         uint16_t* __restrict__ out, int64_t M, int64_t K) {
    const int64_t cpr = K >> 3;
    const int64_t total = M * cpr;
    const ChunkIndex index(cpr, total);
    for (int64_t ch = (int64_t)blockIdx.x * 256 + threadIdx.x; ch < total; ch += (int64_t)gridDim.x * 256) {
        int64_t row, col;
        index(ch, row, col);
        const uint32_t sc = s[row * (K >> 5) + (col >> 2)];
        const float mul = sc == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(sc << 23);  // 2^-127 is subnormal
        float f[8];
        if (FP4) {
            uint32_t p = reinterpret_cast<const uint32_t*>(q + row * (K >> 1))[col];
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = e2m1_decode((p >> (4 * j)) & 0xF) * mul;
        } else {
            uint2 p = reinterpret_cast<const uint2*>(q + row * K)[col];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f[j] = e4m3_decode((p.x >> (8 * j)) & 0xFF) * mul;
                f[4 + j] = e4m3_decode((p.y >> (8 * j)) & 0xFF) * mul;
            }
        }
        if (sc == 0xFF) {
#pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = __builtin_nanf("");
        }
        uint4 o;
        o.x = f32_to_bf16(f[0]) | (f32_to_bf16(f[1]) << 16);
        o.y = f32_to_bf16(f[2]) | (f32_to_bf16(f[3]) << 16);
        o.z = f32_to_bf16(f[4]) | (f32_to_bf16(f[5]) << 16);
        o.w = f32_to_bf16(f[6]) | (f32_to_bf16(f[7]) << 16);
        reinterpret_cast<uint4*>(out + row * K)[col] = o;
    }
}

static int grid_for(int64_t threads_needed) {
    // enough workgroups to cover the chip several times; grid-stride covers the rest
    int64_t g = (threads_needed + 255) / 256;
    return (int)(g < 8192 ? (g < 1 ? 1 : g) : 8192);
}

}  // namespace hkq

using namespace hkq;

extern "C" {

int hkq_per_token_quant(const void* x, void* q, float* s, int64_t M, int64_t K, int64_t ldx, int64_t ldq, int kind,
                        hipStream_t stream) {
    HKQ_CHECK_ARG(kind == HKQ_KIND_FP8 || kind == HKQ_KIND_INT8, "kind must be HKQ_KIND_FP8 or HKQ_KIND_INT8");
    HKQ_CHECK_ARG(M >= 0 && K > 0 && K % 8 == 0, "K must be a positive multiple of 8");
    HKQ_CHECK_ARG(K <= 8 * 256 * 16, "K must be <= 32768");
    HKQ_CHECK_ARG(ldx >= K && ldq >= K && ldx % 8 == 0 && ldq % 8 == 0, "row strides must be >= K and multiples of 8");
    HKQ_CHECK_ALIGN(x, 16);
    HKQ_CHECK_ALIGN(q, 8);
    if (M == 0) return 0;
    const int chunks = (int)((K / 8 + 255) / 256);
    auto* xp = static_cast<const uint16_t*>(x);
    auto* qp = static_cast<uint8_t*>(q);
#define HKQ_PT(C)                                                                                          \
    if (kind == HKQ_KIND_FP8)                                                                             \
        per_token_kernel<KIND_FP8, C><<<dim3((unsigned)M), 256, 0, stream>>>(xp, qp, s, K, ldx, ldq);    \
    else                                                                                                  \
        per_token_kernel<KIND_INT8, C><<<dim3((unsigned)M), 256, 0, stream>>>(xp, qp, s, K, ldx, ldq);
    if (chunks <= 1) { HKQ_PT(1) }
    else if (chunks <= 2) { HKQ_PT(2) }
    else if (chunks <= 4) { HKQ_PT(4) }
    else if (chunks <= 8) { HKQ_PT(8) }
    else { HKQ_PT(16) }
#undef HKQ_PT
    return hkq_launch_status();
}

int hkq_group_quant(const void* x, void* q, float* s, int64_t M, int64_t K, int64_t ldx, int64_t ldq, int64_t lds,
                    int64_t group, int kind, hipStream_t stream) {
    HKQ_CHECK_ARG(kind == HKQ_KIND_FP8 || kind == HKQ_KIND_INT8, "kind must be HKQ_KIND_FP8 or HKQ_KIND_INT8");
    HKQ_CHECK_ARG(group == 32 || group == 64 || group == 128 || group == 256 || group == 512,
                  "group must be one of 32, 64, 128, 256, 512");
    HKQ_CHECK_ARG(M >= 0 && K > 0 && K % group == 0, "K must be a positive multiple of group");
    HKQ_CHECK_ARG(ldx >= K && ldq >= K && ldx % 8 == 0 && ldq % 8 == 0, "row strides must be >= K and multiples of 8");
    HKQ_CHECK_ARG(lds >= K / group, "scale row stride must be >= K / group");
    HKQ_CHECK_ALIGN(x, 16);
    HKQ_CHECK_ALIGN(q, 8);
    if (M == 0) return 0;
    auto* xp = static_cast<const uint16_t*>(x);
    auto* qp = static_cast<uint8_t*>(q);
    const int grid = grid_for(M * (K / 8));
#define HKQ_G(GL)                                                                                                   \
    if (kind == HKQ_KIND_FP8)                                                                                      \
        group_kernel<KIND_FP8, GL><<<grid, 256, 0, stream>>>(xp, qp, s, M, K, ldx, ldq, lds);                      \
    else                                                                                                           \
        group_kernel<KIND_INT8, GL><<<grid, 256, 0, stream>>>(xp, qp, s, M, K, ldx, ldq, lds);
    switch (group) {
        case 32: HKQ_G(4) break;
        case 64: HKQ_G(8) break;
        case 128: HKQ_G(16) break;
        case 256: HKQ_G(32) break;
        default: HKQ_G(64) break;
    }
#undef HKQ_G
    return hkq_launch_status();
}

int hkq_static_quant_fp8(const void* x, void* y, const float* scale, int64_t n, hipStream_t stream) {
    HKQ_CHECK_ARG(n >= 0 && n % 8 == 0, "element count must be a multiple of 8");
    HKQ_CHECK_ALIGN(x, 16);
    HKQ_CHECK_ALIGN(y, 8);
    if (n == 0) return 0;
    static_fp8_kernel<<<grid_for(n / 8), 256, 0, stream>>>(static_cast<const uint16_t*>(x),
                                                           static_cast<uint8_t*>(y), scale, n / 8);
    return hkq_launch_status();
}

int hkq_mx_quant(const void* x, void* q, void* s, int64_t M, int64_t K, int64_t ldx, int is_fp4, hipStream_t stream) {
    HKQ_CHECK_ARG(M >= 0 && K > 0 && K % 32 == 0, "K must be a positive multiple of 32");
    HKQ_CHECK_ARG(ldx >= K && ldx % 8 == 0, "row stride must be >= K and a multiple of 8");
    HKQ_CHECK_ALIGN(x, 16);
    HKQ_CHECK_ALIGN(q, is_fp4 ? 4 : 8);
    if (M == 0) return 0;
    const int grid = grid_for(M * (K / 8));
    if (is_fp4)
        mx_quant_kernel<true><<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(x), static_cast<uint8_t*>(q),
                                                        static_cast<uint8_t*>(s), M, K, ldx);
    else
        mx_quant_kernel<false><<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(x), static_cast<uint8_t*>(q),
                                                         static_cast<uint8_t*>(s), M, K, ldx);
    return hkq_launch_status();
}

int hkq_mx_dequant(const void* q, const void* s, void* out, int64_t M, int64_t K, int is_fp4, hipStream_t stream) {
    HKQ_CHECK_ARG(M >= 0 && K > 0 && K % 32 == 0, "K must be a positive multiple of 32");
    HKQ_CHECK_ALIGN(q, is_fp4 ? 4 : 8);
    HKQ_CHECK_ALIGN(out, 16);
    if (M == 0) return 0;
    const int grid = grid_for(M * (K / 8));
    if (is_fp4)
        mx_dequant_kernel<true><<<grid, 256, 0, stream>>>(static_cast<const uint8_t*>(q),
                                                          static_cast<const uint8_t*>(s), static_cast<uint16_t*>(out), M, K);
    else
        mx_dequant_kernel<false><<<grid, 256, 0, stream>>>(static_cast<const uint8_t*>(q),
                                                           static_cast<const uint8_t*>(s), static_cast<uint16_t*>(out), M, K);
    return hkq_launch_status();
}

}  // extern "C"
