// norm_quant.hip -- quantizers fused with the op that produces their input:
//
//   rmsnorm_quant_kernel  RMSNorm + 1x128 FP8 (E4M3FN) or MXFP4 quantization,
//                         quantization/fused_fp8_quant/kernel.cpp:37-204 and
//                         quantization/fused_mxfp4_quant/kernel.cpp:40-243
//                         (y = x * rsqrt(mean(x^2) + eps) * w, then the 1x128
//                         per-block rule or the MX shared-exponent rule);
//   swiglu_quant_kernel   SiLU-and-mul of a gate/up GEMM output followed by
//                         per-token or 1x128 FP8 quantization: the activation of
//                         moe-gemm/moe_op_silu_fused/kernel.cpp:1-13 and the
//                         silu of moe-gemm/moe_op_gemm_a8w8/kernel.cpp:57-59,
//                         feeding the down projection.
//
// Both are HBM-bound: each input element is read once into registers, the
// row statistic is reduced, and the codes are encoded from registers.
#include "hkq_device.h"
#include "hkq_host.h"

namespace hkq {

// buffer-instruction cache policies (gfx950): non-temporal loads and stores
constexpr int CPOL_NT_LD = 2, CPOL_NT_ST = 2;

// MXFP4 elements rounded to nearest even (NQ_MXFP4) or floored by the
// reference module's ladder (NQ_MXFP4_FLOOR); the shared exponent is the same
enum { NQ_FP8_G128 = 0, NQ_MXFP4 = 1, NQ_MXFP4_FLOOR = 2 };

__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = bf16_to_f32(w[i] & 0xFFFF);
        f[2 * i + 1] = bf16_to_f32(w[i] >> 16);
    }
}

// --------------------------------------------------------------------------
// RMSNorm + quantization. One wave per row, four rows per workgroup; lane l
// holds the 16-byte chunks c = l + 64 i (8 bf16 each) of x in registers, the
// workgroup's rows share the weight row in LDS.
//   sum  = fma-chain of x^2 over the lane's chunks (i, then element order),
//          then the xor butterfly over lanes;
//   r    = 1 / sqrt(sum / D + eps)   (correctly rounded sqrt and division);
//   y    = (x * r) * w               (two fp32 roundings);
// FP8: per 128 columns (16 chunks = 16 adjacent lanes) s = max(amax/448, 1e-10),
//      q = E4M3FN(clamp(y * (1/s), +-448)); MXFP4: per 32 columns (4 lanes)
//      the MX shared exponent e of amax, q = E2M1(y * 2^-e), scale byte e + 127.
// --------------------------------------------------------------------------
template <int MODE, int NC>
__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ w, uint8_t* __restrict__ q,
                                                            void* __restrict__ s, int M, int D, int64_t ldx,
                                                            int64_t ldq, int64_t lds, float eps) {
    // the weight row, shared by the workgroup's four rows: held in LDS rather
    // than in every lane's registers, so that more rows fit in flight per SIMD
    __shared__ uint4 wl[NC * 64];
    const int lane = threadIdx.x & 63;
    // wave-uniform (made visibly so: the buffer resources below are then built in SGPRs)
    const int row = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    const int nch = D >> 3;
    // Buffer loads and stores over the row: chunks past D read zero and their
    // stores are dropped by the buffer bounds, so no lane branches around them
    // (only whole chunk columns past D are skipped, a wave-uniform test).
    const auto rx = make_rsrc(x + (int64_t)row * ldx, (uint32_t)D * 2u);
    const auto rw = make_rsrc(w, (uint32_t)D * 2u);
    // the weight's loads go out first (every wave, also one past M, takes its
    // share and the barrier), then the row's HBM loads, which stay in flight
    // while the weight is written to LDS
    constexpr int WPT = (NC * 64 + 255) / 256;  // weight chunks per thread
    uint4 wt[WPT];
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
        const int c = (int)threadIdx.x + 256 * i;
        const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rw, c < NC * 64 ? (uint32_t)c * 16u : 0x80000000u, 0, 0);
        wt[i] = make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
    }
    uint4 xv[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        xv[i] = make_uint4(0, 0, 0, 0);
        if (row < M && 64 * i < nch) {
            const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(lane + 64 * i) * 16u, 0, CPOL_NT_LD);
            xv[i] = make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
        }
    }
#pragma unroll
    for (int i = 0; i < WPT; ++i)
        if (threadIdx.x + 256 * i < NC * 64) wl[threadIdx.x + 256 * i] = wt[i];
    __syncthreads();
    if (row >= M) return;  // no barriers below
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        float f[8];
        unpack8(xv[i], f);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(f[j], f[j], ss);
    }
    ss = group_sum<64>(ss);
    const float r = 1.0f / __builtin_sqrtf(ss / (float)D + eps);
    const auto rq = make_rsrc(q + (int64_t)row * ldq, (uint32_t)(MODE == NQ_FP8_G128 ? D : D / 2));
    const auto rs = MODE == NQ_FP8_G128 ? make_rsrc(static_cast<float*>(s) + (int64_t)row * lds, (uint32_t)(D / 128) * 4u)
                                        : make_rsrc(static_cast<uint8_t*>(s) + (int64_t)row * lds, (uint32_t)(D / 32));

#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + 64 * i;
        if (64 * i >= nch) break;  // wave-uniform: no lane has a chunk here
        float xf[8], wf[8], y[8];
        unpack8(xv[i], xf);
        unpack8(wl[c], wf);
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            y[j] = (xf[j] * r) * wf[j];
            m = max_num(m, __builtin_fabsf(y[j]));
        }
        if (MODE == NQ_FP8_G128) {
            m = group_max_abs<16>(m);
            const float sc = fp8_group_scale(m);
            const float rc = recip_scale(sc);
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = max_num(min_num(y[j] * rc, 448.0f), -448.0f);
            const uint32_t lo = cvt_pk4_e4m3(v[0], v[1], v[2], v[3]);
            const uint32_t hi = cvt_pk4_e4m3(v[4], v[5], v[6], v[7]);
            // non-temporal: measured on MI355X, [4096, 4096] 12.1 -> 10.3 us
            // (the same policy made the SwiGLU kernel's codes 8% slower)
            __builtin_amdgcn_raw_buffer_store_b64(v2i{(int)lo, (int)hi}, rq, (uint32_t)c * 8u, 0, CPOL_NT_ST);
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(sc), rs, (lane & 15) == 0 ? (uint32_t)(c >> 4) * 4u : 0x80000000u,
                                                  0, 0);
        } else {
            m = group_max_abs<4>(m);
            const int e = mx_scale_exp(m);
            const float mul = exp2i(-e);
            float t[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) t[j] = y[j] * mul;
            const uint32_t packed = MODE == NQ_MXFP4_FLOOR ? e2m1_floor8(t) : e2m1_encode8(t);
            __builtin_amdgcn_raw_buffer_store_b32((int)packed, rq, (uint32_t)c * 4u, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b8((unsigned char)(e + 127), rs, (lane & 3) == 0 ? (uint32_t)(c >> 2) : 0x80000000u,
                                                 0, 0);
        }
    }
}

// --------------------------------------------------------------------------
// SwiGLU + FP8 quantization. One workgroup (256 threads) per row of the
// gate/up GEMM output y [M, 2F] (bf16); thread t owns the activation chunks
// c = t + 256 i (8 columns each):
//   act = silu(g) * u,  silu(g) = g / (1 + 2^(-log2(e) * alpha * g))
// with (g, u) = (y[:, k], y[:, F + k]) for split halves, or (y[:, 2k], y[:, 2k+1])
// interleaved (moe_op_silu_fused's column order). Per token (GROUP 0):
// s = max(amax(act row)/448, 1e-10); 1x128 (GROUP 128): per 16 chunks.
// q = E4M3FN(clamp(act * (1/s), +-448)).
// --------------------------------------------------------------------------
__device__ __forceinline__ float silu_alpha(float g, float alpha) {
    return g * __builtin_amdgcn_rcpf(1.0f + exp2f(-1.44269504089f * alpha * g));
}

template <int INTERLEAVED, int GROUP, int NC>
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const uint16_t* __restrict__ y, uint8_t* __restrict__ q,
                                                           float* __restrict__ s, int M, int F, int64_t ldy,
                                                           int64_t ldq, int64_t lds, float alpha) {
    __shared__ float wmax[4];
    const int row = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int nch = F >> 3;
    const uint16_t* yr = y + (int64_t)row * ldy;
    float act[NC][8];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = t + 256 * i;
        uint4 g4 = make_uint4(0, 0, 0, 0), u4 = make_uint4(0, 0, 0, 0);
        if (c < nch) {
            if (INTERLEAVED) {
                const uint4 a = ld_stream16(yr + (int64_t)c * 16), b = ld_stream16(yr + (int64_t)c * 16 + 8);
                // a = g0 u0 g1 u1 g2 u2 g3 u3, b = g4 u4 ... g7 u7
                g4 = make_uint4((a.x & 0xFFFF) | (a.y << 16), (a.z & 0xFFFF) | (a.w << 16),
                                (b.x & 0xFFFF) | (b.y << 16), (b.z & 0xFFFF) | (b.w << 16));
                u4 = make_uint4((a.x >> 16) | (a.y & 0xFFFF0000u), (a.z >> 16) | (a.w & 0xFFFF0000u),
                                (b.x >> 16) | (b.y & 0xFFFF0000u), (b.z >> 16) | (b.w & 0xFFFF0000u));
            } else {
                g4 = ld_stream16(yr + (int64_t)c * 8);
                u4 = ld_stream16(yr + F + (int64_t)c * 8);
            }
        }
        float g[8], u[8];
        unpack8(g4, g);
        unpack8(u4, u);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            act[i][j] = silu_alpha(g[j], alpha) * u[j];
            m = max_num(m, __builtin_fabsf(act[i][j]));
        }
    }
    float sc_tok = 0.0f, rc_tok = 0.0f;
    if (GROUP == 0) {
        m = group_max_abs<64>(m);
        if (lane == 0) wmax[wave] = m;
        __syncthreads();
        m = max_num(max_num(wmax[0], wmax[1]), max_num(wmax[2], wmax[3]));
        sc_tok = fp8_group_scale(m);
        rc_tok = recip_scale(sc_tok);
        if (t == 0) s[row] = sc_tok;
    }
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = t + 256 * i;
        if (256 * i >= nch) break;  // block-uniform
        float sc = sc_tok, rc = rc_tok;
        if (GROUP == 128) {
            float mg = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) mg = max_num(mg, __builtin_fabsf(act[i][j]));
            mg = group_max_abs<16>(mg);
            sc = fp8_group_scale(mg);
            rc = recip_scale(sc);
        }
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = max_num(min_num(act[i][j] * rc, 448.0f), -448.0f);
        const uint32_t lo = cvt_pk4_e4m3(v[0], v[1], v[2], v[3]);
        const uint32_t hi = cvt_pk4_e4m3(v[4], v[5], v[6], v[7]);
        if (c < nch) {
            *reinterpret_cast<uint2*>(q + (int64_t)row * ldq + (int64_t)c * 8) = make_uint2(lo, hi);
            if (GROUP == 128 && (t & 15) == 0) s[(int64_t)row * lds + (c >> 4)] = sc;
        }
    }
}

}  // namespace hkq

// ============================================================================
// Host launchers (C ABI)
// ============================================================================
namespace {
using namespace hkq;

template <int MODE, int NC>
int launch_rmsnorm(const uint16_t* x, const uint16_t* w, uint8_t* q, void* s, int M, int D, int64_t ldx,
                   int64_t ldq, int64_t lds, float eps, hipStream_t st) {
    rmsnorm_quant_kernel<MODE, NC><<<(M + 3) / 4, 256, 0, st>>>(x, w, q, s, M, D, ldx, ldq, lds, eps);
    return hkq_launch_status();
}

template <int MODE>
int rmsnorm_nc(const uint16_t* x, const uint16_t* w, uint8_t* q, void* s, int M, int D, int64_t ldx, int64_t ldq,
               int64_t lds, float eps, hipStream_t st) {
    const int per_lane = (D / 8 + 63) / 64;
    if (per_lane <= 2) return launch_rmsnorm<MODE, 2>(x, w, q, s, M, D, ldx, ldq, lds, eps, st);
    if (per_lane <= 4) return launch_rmsnorm<MODE, 4>(x, w, q, s, M, D, ldx, ldq, lds, eps, st);
    if (per_lane <= 8) return launch_rmsnorm<MODE, 8>(x, w, q, s, M, D, ldx, ldq, lds, eps, st);
    return launch_rmsnorm<MODE, 16>(x, w, q, s, M, D, ldx, ldq, lds, eps, st);
}

template <int IL, int GROUP, int NC>
int launch_swiglu(const uint16_t* y, uint8_t* q, float* s, int M, int F, int64_t ldy, int64_t ldq, int64_t lds,
                  float alpha, hipStream_t st) {
    swiglu_quant_kernel<IL, GROUP, NC><<<M, 256, 0, st>>>(y, q, s, M, F, ldy, ldq, lds, alpha);
    return hkq_launch_status();
}

template <int IL, int GROUP>
int swiglu_nc(const uint16_t* y, uint8_t* q, float* s, int M, int F, int64_t ldy, int64_t ldq, int64_t lds,
              float alpha, hipStream_t st) {
    const int per_thread = (F / 8 + 255) / 256;
    if (per_thread <= 1) return launch_swiglu<IL, GROUP, 1>(y, q, s, M, F, ldy, ldq, lds, alpha, st);
    if (per_thread <= 2) return launch_swiglu<IL, GROUP, 2>(y, q, s, M, F, ldy, ldq, lds, alpha, st);
    if (per_thread <= 4) return launch_swiglu<IL, GROUP, 4>(y, q, s, M, F, ldy, ldq, lds, alpha, st);
    if (per_thread <= 8) return launch_swiglu<IL, GROUP, 8>(y, q, s, M, F, ldy, ldq, lds, alpha, st);
    return launch_swiglu<IL, GROUP, 16>(y, q, s, M, F, ldy, ldq, lds, alpha, st);
}

}  // namespace

extern "C" int hkq_rmsnorm_quant(const void* x, const void* w, void* q, void* s, int64_t M, int64_t D, int64_t ldx,
                                 int64_t ldq, int64_t lds, float eps, int kind, hkq_stream_t stream) {
    HKQ_CHECK_ARG(kind >= 0 && kind <= 2, "kind must be 0 (FP8 1x128), 1 (MXFP4, nearest) or 2 (MXFP4, floor)");
    HKQ_CHECK_ARG(M >= 0 && M <= INT32_MAX, "M must be in [0, 2^31)");
    HKQ_CHECK_ARG(D >= 128 && D <= 8192 && D % (kind == 0 ? 128 : 32) == 0,
                  "D must be a multiple of 128 (FP8) or 32 (MXFP4) in [128, 8192]");
    HKQ_CHECK_ARG(ldx >= D && ldx % 8 == 0, "ldx must be >= D and a multiple of 8");
    HKQ_CHECK_ARG(ldq >= (kind == 0 ? D : D / 2) && ldq % (kind == 0 ? 8 : 4) == 0,
                  "ldq must hold a row of codes and be a multiple of 8 (FP8) / 4 (MXFP4) bytes");
    HKQ_CHECK_ARG(lds >= (kind == 0 ? D / 128 : D / 32), "lds must hold a row of scales");
    HKQ_CHECK_ARG(eps >= 0.0f, "eps must be non-negative");
    if (M == 0) return 0;
    HKQ_CHECK_ARG(x && w && q && s, "x, w, q and s are required");
    HKQ_CHECK_ALIGN(x, 16);
    HKQ_CHECK_ALIGN(w, 16);
    HKQ_CHECK_ALIGN(q, kind == 0 ? 8 : 4);
    HKQ_CHECK_ALIGN(s, kind == 0 ? 4 : 1);
    const hipStream_t st = (hipStream_t)stream;
    if (kind == 0)
        return rmsnorm_nc<NQ_FP8_G128>((const uint16_t*)x, (const uint16_t*)w, (uint8_t*)q, s, (int)M, (int)D, ldx,
                                      ldq, lds, eps, st);
    if (kind == 2)
        return rmsnorm_nc<NQ_MXFP4_FLOOR>((const uint16_t*)x, (const uint16_t*)w, (uint8_t*)q, s, (int)M, (int)D, ldx,
                                          ldq, lds, eps, st);
    return rmsnorm_nc<NQ_MXFP4>((const uint16_t*)x, (const uint16_t*)w, (uint8_t*)q, s, (int)M, (int)D, ldx, ldq,
                                lds, eps, st);
}

extern "C" int hkq_swiglu_quant(const void* y, void* q, float* s, int64_t M, int64_t F, int64_t ldy, int64_t ldq,
                                int64_t lds, float alpha, int interleaved, int group, hkq_stream_t stream) {
    HKQ_CHECK_ARG(group == 0 || group == 128, "group must be 0 (per token) or 128");
    HKQ_CHECK_ARG(M >= 0 && M <= INT32_MAX, "M must be in [0, 2^31)");
    HKQ_CHECK_ARG(F >= 8 && F <= 32768 && F % (group ? 128 : 8) == 0,
                  "F must be a multiple of 8 (128 with groups) in [8, 32768]");
    HKQ_CHECK_ARG(ldy >= 2 * F && ldy % 8 == 0, "ldy must be >= 2F and a multiple of 8");
    HKQ_CHECK_ARG(ldq >= F && ldq % 8 == 0, "ldq must be >= F and a multiple of 8");
    HKQ_CHECK_ARG(group == 0 || lds >= F / 128, "lds must hold a row of group scales");
    if (M == 0) return 0;
    HKQ_CHECK_ARG(y && q && s, "y, q and s are required");
    HKQ_CHECK_ALIGN(y, 16);
    HKQ_CHECK_ALIGN(q, 8);
    HKQ_CHECK_ALIGN(s, 4);
    const hipStream_t st = (hipStream_t)stream;
    const uint16_t* yy = (const uint16_t*)y;
    uint8_t* qq = (uint8_t*)q;
    const int m = (int)M, f = (int)F;
    if (interleaved)
        return group ? swiglu_nc<1, 128>(yy, qq, s, m, f, ldy, ldq, lds, alpha, st)
                     : swiglu_nc<1, 0>(yy, qq, s, m, f, ldy, ldq, lds, alpha, st);
    return group ? swiglu_nc<0, 128>(yy, qq, s, m, f, ldy, ldq, lds, alpha, st)
                 : swiglu_nc<0, 0>(yy, qq, s, m, f, ldy, ldq, lds, alpha, st);
}
