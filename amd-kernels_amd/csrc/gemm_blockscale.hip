// gemm_blockscale.hip -- FP8 GEMM with per-K-group fp32 scales (DeepSeek-V3
// style), restating gemm-basic/gemm_a8w8_blockscale/kernel.cpp:129-153 (and
// the formula of gemm_a8w8_blockscale/test_parity.py:57-76):
//
//   C[m, n] = bf16( sum_g (A_g . B_g^T)[m, n] * sa[m, g] * sb[g, n / GN] ),
//   g = 128-wide K group, GN = 128 (128x128 weight blocks) or 1 (per column,
//   the layout of the reference test: b_scale [K/128, N]).
//
// fp32 scales cannot ride in the MFMA's e8m0 scale operands, so every K group
// is "promoted" on the VALU: per 32x32 sub-tile two chained MFMAs (the group's
// two 64-deep K-steps) produce a fresh partial P, then acc += P * sa * sb.
// M > 192 runs the 8-wave K loop of blockscale_core.h over 256 x 256 tiles;
// narrow M streams the weights through registers (blockscale_narrow_kernel).
#include <cstdlib>

#include "blockscale_core.h"
#include "hkq_host.h"

namespace hkq {

struct BlockScaleParams {
    const uint8_t* A;
    const uint8_t* B;
    uint16_t* C;
    const float* sa;  // [M, lsa]: column g = K group
    const float* sb;  // [K/128, lsb]: column n/128 (GN 128) or n (GN 1)
    int M, N, K;
    int64_t lda, ldb, ldc, lsa, lsb;
    int tiles_m, tiles_n, group_m, c16;
    // multiply-add epilogue C = ca * GEMM + cb, ca / cb bf16 [M, ldca] / [M, ldcb]
    // (nullptr: plain GEMM)
    const uint16_t* ca;
    const uint16_t* cb;
    int64_t ldca, ldcb;
};

// Multiply-add epilogue hook: v -> ca[m, n] * v + cb[m, n] on the fp32 sums.
// prefetch(i) loads the lane's 4 x TM groups of 4 bf16 of both operands for
// n-tile i in one batch (rows past M / columns past N: ca = 1, cb = 0).
template <int TM>
struct MulAddElem {
    const uint16_t *ca, *cb;
    int64_t ldca, ldcb;
    int M, N, mw, nw, lane;
    uint2 a[4][TM], b[4][TM];
    __device__ void prefetch(int i) {
        const int m0 = mw + (lane & 31), n0 = nw + i * 32 + 4 * (lane >> 5);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int m = m0 + j * 32, n = n0 + 8 * g;
                const bool in = m < M && n < N;
                a[g][j] = in ? *reinterpret_cast<const uint2*>(ca + (int64_t)m * ldca + n) : make_uint2(0x3F803F80u, 0x3F803F80u);
                b[g][j] = in ? *reinterpret_cast<const uint2*>(cb + (int64_t)m * ldcb + n) : make_uint2(0u, 0u);
            }
    }
    __device__ float4 operator()(int j, int, int g, float4 v) const {
        const uint2 x = a[g][j], y = b[g][j];
        return make_float4(bf16_to_f32(x.x & 0xFFFF) * v.x + bf16_to_f32(y.x & 0xFFFF),
                           bf16_to_f32(x.x >> 16) * v.y + bf16_to_f32(y.x >> 16),
                           bf16_to_f32(x.y & 0xFFFF) * v.z + bf16_to_f32(y.y & 0xFFFF),
                           bf16_to_f32(x.y >> 16) * v.w + bf16_to_f32(y.y >> 16));
    }
};

// Tiled kernel: the 8-wave K loop of blockscale_core.h over 256 x BN tiles.
// BN 256: waves of 64 x 128 (two per SIMD). BN 224, for grids that the
// 256-wide tiles would leave a CU short (2048 x 7168: 224 tiles of 256 x 256,
// 256 of 256 x 224): waves 0-3 take n-tiles 0-3 and waves 4-7 n-tiles 4-6 of
// their 64 rows, so that each SIMD holds one wave of each kind (the hardware
// places wave w on SIMD w % 4) and does 7/8 of a 256-wide tile's work; the B
// rows past 224 read zero. Scale slot: sa of the tile's 256 rows; sb GN 1 or
// BN 224: one value per tile column (GN 128: its block's), GN 128 with BN
// 256: the tile's two column blocks.
template <bool GN1, int BN>
__global__ __launch_bounds__(64 * BS_NW, 1) void blockscale_gemm_kernel(const BlockScaleParams p) {
    static_assert(BN == BS_BN || BN == BS_BN - 32, "tile widths of 256 or 224 columns");
    constexpr bool W224 = BN != BS_BN;
    constexpr int TM = BS_TM, TN = BS_TN, NW = BS_NW;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = W224 ? wave & 3 : wave / BS_WN, wn = W224 ? wave >> 2 : wave % BS_WN;

    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    const int m0 = tm * BS_BM, n0 = tn * BN;
    const int rows_a = min(p.M - m0, BS_BM), rows_b = min(p.N - n0, BN);

    // LDS-direct loads: load i of a wave fills rows (i*NW + wave)*8 .. +7 of
    // its operand tile
    uint32_t a_off[BS_LA], b_off[BS_LB];
#pragma unroll
    for (int i = 0; i < BS_LA; ++i) a_off[i] = dense_row_off<NW, BS_KT>(i, wave, lane, p.lda);
#pragma unroll
    for (int i = 0; i < BS_LB; ++i) b_off[i] = dense_row_off<NW, BS_KT>(i, wave, lane, p.ldb);
    const uint8_t* a_src = p.A + (int64_t)m0 * p.lda;
    const uint8_t* b_src = p.B + (int64_t)n0 * p.ldb;
    const int64_t a_bytes = min((int64_t)rows_a * p.lda, (int64_t)0x7FFFFFFF);
    const int64_t b_bytes = min((int64_t)rows_b * p.ldb, (int64_t)0x7FFFFFFF);
    // scales: sa rows (wave & 3) * 64 + lane; sb per column: tile column c =
    // (wave & 3)*64 + lane from sb's row of the K-tile (GN 128: its block's
    // value), per block (GN 128, BN 256): blocks n0/128 + {0, 1}. Waves 4-7
    // repeat the loads of 0-3 so that every wave issues the same loads.
    const float* sa_src = p.sa + (int64_t)m0 * p.lsa;
    const int64_t sa_bytes = min((int64_t)rows_a * p.lsa * 4, (int64_t)0x7FFFFFFF);
    const uint32_t sa_off = (uint32_t)(((wave & 3) * 64 + lane) * p.lsa * 4);
    constexpr bool PER_COL = GN1 || W224;
    const int sb_row = GN1 ? p.N : (p.N + 127) / 128;  // values per sb row
    const int sc = (wave & 3) * 64 + lane;
    const uint32_t sb_off = PER_COL ? (sc < rows_b ? (uint32_t)((GN1 ? n0 + sc : (n0 + sc) / 128) * 4) : OOB)
                                    : (lane < 2 ? (uint32_t)((n0 / 128 + lane) * 4) : OOB);
    const uint32_t lds_base = (uint32_t)(uintptr_t)smem;
    const int KTN = p.K / BS_KT;

    // load q (0 .. BS_NLD-1) of K-tile kt: A, B, then the sa and sb scales
    auto issue = [&](int kt, int q) {
        const bool live = kt < KTN;
        const uint32_t kb = (uint32_t)(kt * BS_KT);
        const int st = kt & 1;
        if (q < BS_LA + BS_LB) {
            HKQ_LDS uint8_t* dst = reinterpret_cast<HKQ_LDS uint8_t*>((uintptr_t)(lds_base + bs_load_dst(st, q, wave)));
            if (q < BS_LA)
                lds_load16(a_src + kb, live ? (uint32_t)(a_bytes - kb) : 0u, dst, a_off[q]);
            else
                lds_load16(b_src + kb, live ? (uint32_t)(b_bytes - kb) : 0u, dst, b_off[q - BS_LA]);
        } else {
            HKQ_LDS uint8_t* slot = smem + BS_SC + st * BS_SLOT;
            if (q == BS_LA + BS_LB)
                lds_load4(sa_src + kt, live ? (uint32_t)(sa_bytes - kt * 4) : 0u, slot + (wave & 3) * 256, sa_off);
            else
                lds_load4(p.sb + (int64_t)kt * p.lsb, live ? (uint32_t)(sb_row * 4) : 0u,
                          slot + 1024 + (PER_COL ? (wave & 3) * 256 : 0), sb_off);
        }
    };

    v16f acc[TN][TM];
    constexpr int SBM = GN1 ? BS_SB_COL : W224 ? BS_SB_NTILE : BS_SB_WAVE;
    if (W224 && wn == 1) {
        bs8_kloop<SBM, TN - 1>(smem, lane, wm, TN * 32, KTN, issue, reinterpret_cast<v16f(&)[TN - 1][TM]>(acc));
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[TN - 1][j] = v16f{};
    } else
        bs8_kloop<SBM, TN>(smem, lane, wm, wn * TN * 32, KTN, issue, acc);

    // BN 224: the last n-tile of waves 4-7 lies past the tile (never stored)
    const int mw = m0 + wm * TM * 32, nw = n0 + wn * TN * 32;
    const int n_end = W224 ? min(p.N, n0 + BN) : p.N;
    auto one = [](int) { return 1.0f; };
    auto ones = [](int, int) { return make_float4(1.f, 1.f, 1.f, 1.f); };
    if (p.ca) {
        MulAddElem<TM> e;
        e.ca = p.ca;
        e.cb = p.cb;
        e.ldca = p.ldca;
        e.ldcb = p.ldcb;
        e.M = p.M;
        e.N = n_end;
        e.mw = mw;
        e.nw = nw;
        e.lane = lane;
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, p.C, p.ldc, p.M, n_end, mw, nw, p.c16 != 0, one, ones, NoBias{}, e);
    } else {
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, p.C, p.ldc, p.M, n_end, mw, nw, p.c16 != 0, one, ones, NoBias{});
    }
}

// ---------------------------------------------------------------------------
// Narrow M (M <= 64): the streaming layout of the dense GEMMs' narrow path
// (workgroup = 16*NT columns for all rows, 4 waves splitting K, fragments
// loaded straight into registers for the 16x16x128 MFMA; lane l supplies row
// l % 16, bytes [16q, 16q+16) and [64+16q, 64+16q+16) of the step, q = l/16,
// and holds D[4q + i][l % 16]). A 128-value K-step is exactly one scale
// group, so each step's MFMA starts from zero and is promoted at once:
// acc += P * sa[m, g] * sb[g, n / GN]. Rows come in MT tiles of 16. The
// 256 x 256 tiles of the main kernel would give M <= 64 only N/256
// workgroups.
constexpr int BSN_WAVES = 4, BSN_MAX_M = 64;

template <bool GN1, int MT, int NT>
struct BsNarrowFrag {
    v4i b0[NT], b1[NT], a0[MT], a1[MT];
    float sa[MT];                // sa[m, g] of the lane's rows
    float sb[NT][GN1 ? 4 : 1];   // sb[g, n] of the lane's 4 columns (GN 1) or of the tile's column block
};

// Rows [64 * blockIdx.y, 64 * blockIdx.y + 64) of the GEMM as a GEMM of their own.
__device__ __forceinline__ BlockScaleParams bs_row_slice(const BlockScaleParams& pb) {
    BlockScaleParams p = pb;
    const int m0 = blockIdx.y * BSN_MAX_M;
    if (m0 > 0) {
        p.A += (int64_t)m0 * p.lda;
        p.sa += (int64_t)m0 * p.lsa;
        p.C += (int64_t)m0 * p.ldc;
        if (p.ca) {
            p.ca += (int64_t)m0 * p.ldca;
            p.cb += (int64_t)m0 * p.ldcb;
        }
    }
    // every row group (the first included) spans at most 64 rows, which keeps
    // its buffer ranges within the host's 64-row 2^31-byte bound
    p.M = min(BSN_MAX_M, p.M - m0);
    return p;
}

template <bool GN1, int MT, int NT>
__global__ __launch_bounds__(64 * BSN_WAVES) void blockscale_narrow_kernel(const BlockScaleParams pb) {
    const BlockScaleParams p = bs_row_slice(pb);
    constexpr int DEPTH = MT * NT == 1 ? 6 : 4;
    __shared__ v4f red[BSN_WAVES][NT][MT][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * 16 * NT;
    const int S = p.K / 128;
    const int s0 = wave * S / BSN_WAVES, s1 = (wave + 1) * S / BSN_WAVES;
    const int rows_b = min(16 * NT, p.N - n0);
    const auto rb = make_rsrc(p.B + (int64_t)n0 * p.ldb, (uint32_t)(rows_b * p.ldb));
    const auto ra = make_rsrc(p.A, (uint32_t)(p.M * p.lda));
    // scales: rows of sa past M and groups past S read zero
    const auto rsa = make_rsrc(p.sa, (uint32_t)(((int64_t)(p.M - 1) * p.lsa + S) * 4));
    const auto rsb = make_rsrc(p.sb, (uint32_t)(((int64_t)(S - 1) * p.lsb + (GN1 ? p.N : (p.N + 127) / 128)) * 4));
    uint32_t a_off[MT], sa_row[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        a_off[t] = (uint32_t)((t * 16 + r) * p.lda + 16 * q);
        sa_row[t] = t * 16 + r < p.M ? (uint32_t)((t * 16 + r) * p.lsa) * 4 : OOB;
    }
    uint32_t b_off[NT], sb_col[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        b_off[i] = (uint32_t)((i * 16 + r) * p.ldb + 16 * q);
        sb_col[i] = (uint32_t)(GN1 ? n0 + 16 * i + 4 * q : (n0 + 16 * i) / 128) * 4;
    }

    auto load = [&](int s, BsNarrowFrag<GN1, MT, NT>& f) {
        const uint32_t kill = s < s1 ? 0u : OOB;
        const uint32_t kb = (uint32_t)s * 128 | kill;
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            f.b0[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, b_off[i] + kb, 0, 0);
            f.b1[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, b_off[i] + kb + 64, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            f.a0[t] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[t] + kb, 0, 0);
            f.a1[t] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[t] + kb + 64, 0, 0);
            f.sa[t] = __builtin_bit_cast(float,
                                         __builtin_amdgcn_raw_buffer_load_b32(rsa, (sa_row[t] + 4 * (uint32_t)s) | kill, 0, 0));
        }
        const uint32_t srow = ((uint32_t)s * (uint32_t)p.lsb * 4) | kill;
#pragma unroll
        for (int i = 0; i < NT; ++i)
#pragma unroll
            for (int e = 0; e < (GN1 ? 4 : 1); ++e)
                f.sb[i][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsb, srow + sb_col[i] + 4 * e, 0, 0));
    };
    v4f acc[NT][MT];
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[i][t] = v4f{0.f, 0.f, 0.f, 0.f};
    auto mma = [&](const BsNarrowFrag<GN1, MT, NT>& f) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const v8i b = v8i{f.a0[t][0], f.a0[t][1], f.a0[t][2], f.a0[t][3], f.a1[t][0], f.a1[t][1], f.a1[t][2], f.a1[t][3]};
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                const v8i a = v8i{f.b0[i][0], f.b0[i][1], f.b0[i][2], f.b0[i][3],
                                  f.b1[i][0], f.b1[i][1], f.b1[i][2], f.b1[i][3]};
                const v4f P =
                    __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[i][t][e] = __builtin_fmaf(P[e], f.sa[t] * f.sb[i][GN1 ? e : 0], acc[i][t][e]);
            }
        }
    };
    BsNarrowFrag<GN1, MT, NT> f[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) load(s0 + d, f[d]);
    for (int s = s0; s < s1; s += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            mma(f[d]);
            load(s + d + DEPTH, f[d]);
        }
    }
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int t = 0; t < MT; ++t) red[wave][i][t][lane] = acc[i][t];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int n = n0 + 16 * i + 4 * q, m = t * 16 + r;
        if (n >= p.N || m >= p.M) continue;  // N % 4 == 0: n .. n+3 all in or all out
        v4f v = red[0][i][t][lane];
#pragma unroll
        for (int w = 1; w < BSN_WAVES; ++w) v += red[w][i][t][lane];
        if (p.ca) {
            const uint2 x = *reinterpret_cast<const uint2*>(p.ca + (int64_t)m * p.ldca + n);
            const uint2 y = *reinterpret_cast<const uint2*>(p.cb + (int64_t)m * p.ldcb + n);
            v = v4f{bf16_to_f32(x.x & 0xFFFF) * v[0] + bf16_to_f32(y.x & 0xFFFF),
                    bf16_to_f32(x.x >> 16) * v[1] + bf16_to_f32(y.x >> 16),
                    bf16_to_f32(x.y & 0xFFFF) * v[2] + bf16_to_f32(y.y & 0xFFFF),
                    bf16_to_f32(x.y >> 16) * v[3] + bf16_to_f32(y.y >> 16)};
        }
        *reinterpret_cast<v2i*>(p.C + (int64_t)m * p.ldc + n) = v2i{(int)pk_bf16(v[0], v[1]), (int)pk_bf16(v[2], v[3])};
    }
}

// M <= 64 in MT = 1, 2 or 4 row tiles, with 16-column (NT = 1) or 32-column
// (NT = 2, when N/16 workgroups exceed the CUs) slices; larger M in row groups
// of 64 (grid.y), each streaming the weights again. 32 weight rows and 64
// activation rows must span less than 2 GiB (32-bit buffer offsets).
template <bool GN1, int MT>
static int launch_blockscale_narrow_mt(const BlockScaleParams& p, hipStream_t stream) {
    const int64_t ncu = cu_count() > 0 ? cu_count() : 256;
    const int64_t wgs16 = (p.N + 15) / 16;
    const unsigned row_groups = (unsigned)((p.M + BSN_MAX_M - 1) / BSN_MAX_M);
    if (wgs16 > ncu)
        blockscale_narrow_kernel<GN1, MT, 2><<<dim3((unsigned)((p.N + 31) / 32), row_groups), 64 * BSN_WAVES, 0, stream>>>(p);
    else
        blockscale_narrow_kernel<GN1, MT, 1><<<dim3((unsigned)wgs16, row_groups), 64 * BSN_WAVES, 0, stream>>>(p);
    return hkq_launch_status();
}

template <bool GN1>
static int launch_blockscale_narrow(const BlockScaleParams& p, hipStream_t stream) {
    if (p.M <= 16) return launch_blockscale_narrow_mt<GN1, 1>(p, stream);
    if (p.M <= 32) return launch_blockscale_narrow_mt<GN1, 2>(p, stream);
    return launch_blockscale_narrow_mt<GN1, 4>(p, stream);
}

template <bool GN1, int BN>
static int launch_blockscale_bn(BlockScaleParams& p, hipStream_t stream) {
    constexpr int BM = BS_BM, LDS = BS_LDS;
    auto kern = blockscale_gemm_kernel<GN1, BN>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
        if (e != hipSuccess) {
            set_error("hipFuncSetAttribute(MaxDynamicSharedMemorySize=%d) failed: %s", LDS, hipGetErrorString(e));
            return (int)e;
        }
        attr_set = true;
    }
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + BN - 1) / BN;
    if (p.group_m <= 0) p.group_m = 8;
    p.c16 = (p.ldc % 8 == 0) && (reinterpret_cast<uintptr_t>(p.C) % 16 == 0);
    const int64_t nblk = (int64_t)p.tiles_m * p.tiles_n;
    if (nblk == 0) return 0;
    kern<<<dim3((unsigned)nblk), 64 * BS_NW, LDS, stream>>>(p);
    return hkq_launch_status();
}

// 224-column tiles when they take fewer SIMD-steps: rounds of tiles over the
// CUs times the n-tiles a SIMD computes per tile (8 for 256 columns, 7 for
// 224). HKQ_BLOCKSCALE_W224=0 (read at each call) keeps the 256-column tiles.
template <bool GN1>
static int launch_blockscale(BlockScaleParams& p, hipStream_t stream) {
    const char* w224_env = std::getenv("HKQ_BLOCKSCALE_W224");
    const bool w224_on = !(w224_env && w224_env[0] == '0');
    const int64_t ncu = cu_count() > 0 ? cu_count() : 256;
    const int64_t tm = (p.M + BS_BM - 1) / BS_BM;
    const int64_t r256 = (tm * ((p.N + BS_BN - 1) / BS_BN) + ncu - 1) / ncu;
    const int64_t r224 = (tm * ((p.N + BS_BN - 33) / (BS_BN - 32)) + ncu - 1) / ncu;
    if (w224_on && 7 * r224 < 8 * r256) return launch_blockscale_bn<GN1, BS_BN - 32>(p, stream);
    return launch_blockscale_bn<GN1, BS_BN>(p, stream);
}

}  // namespace hkq

using namespace hkq;

static int blockscale_call(const void* A, const void* B, const float* sa, const float* sb, void* C, const void* ca,
                           const void* cb, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t lsa,
                           int64_t lsb, int64_t ldc, int64_t ldca, int64_t ldcb, int64_t group_n, hipStream_t stream);

extern "C" int hkq_gemm_blockscale(const void* A, const void* B, const float* sa, const float* sb, void* C,
                                   int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t lsa,
                                   int64_t lsb, int64_t ldc, int64_t group_n, hipStream_t stream) {
    return blockscale_call(A, B, sa, sb, C, nullptr, nullptr, M, N, K, lda, ldb, lsa, lsb, ldc, 0, 0, group_n,
                           stream);
}

extern "C" int hkq_gemm_blockscale_mul_add(const void* A, const void* B, const float* sa, const float* sb, void* C,
                                           const void* c_a, const void* c_b, int64_t M, int64_t N, int64_t K,
                                           int64_t lda, int64_t ldb, int64_t lsa, int64_t lsb, int64_t ldc,
                                           int64_t ldca, int64_t ldcb, int64_t group_n, hipStream_t stream) {
    HKQ_CHECK_ARG(c_a && c_b, "c_a and c_b are required");
    HKQ_CHECK_ARG(ldca >= N && ldcb >= N && ldca % 4 == 0 && ldcb % 4 == 0,
                  "c_a / c_b row strides must be >= N and multiples of 4");
    HKQ_CHECK_ALIGN(c_a, 8);
    HKQ_CHECK_ALIGN(c_b, 8);
    return blockscale_call(A, B, sa, sb, C, c_a, c_b, M, N, K, lda, ldb, lsa, lsb, ldc, ldca, ldcb, group_n, stream);
}

static int blockscale_call(const void* A, const void* B, const float* sa, const float* sb, void* C, const void* ca,
                           const void* cb, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t lsa,
                           int64_t lsb, int64_t ldc, int64_t ldca, int64_t ldcb, int64_t group_n, hipStream_t stream) {
    HKQ_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "M, N must be >= 0 and K > 0");
    HKQ_CHECK_ARG(M < (1 << 30) && N < (1 << 30) && K < (1 << 30), "dimensions must be < 2^30");
    HKQ_CHECK_ARG(K % 128 == 0, "K must be a multiple of the 128-wide scale group");
    HKQ_CHECK_ARG(N % 4 == 0, "N must be a multiple of 4");
    HKQ_CHECK_ARG(group_n == 1 || group_n == 128, "group_n must be 1 or 128");
    HKQ_CHECK_ARG(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0, "lda/ldb must be >= K and multiples of 16");
    HKQ_CHECK_ARG(ldc >= N && ldc % 4 == 0, "ldc must be >= N and a multiple of 4");
    // a stride only matters when there is more than one row to step over
    HKQ_CHECK_ARG(M <= 1 || lsa >= K / 128, "a_scale row stride must be >= K/128");
    HKQ_CHECK_ARG(K / 128 <= 1 || lsb >= (group_n == 1 ? N : (N + 127) / 128),
                  "b_scale row stride must cover N / group_n columns");
    HKQ_CHECK_ALIGN(A, 16);
    HKQ_CHECK_ALIGN(B, 16);
    HKQ_CHECK_ALIGN(C, 8);
    HKQ_CHECK_ALIGN(sa, 4);
    HKQ_CHECK_ALIGN(sb, 4);
    BlockScaleParams p{};
    p.A = static_cast<const uint8_t*>(A);
    p.B = static_cast<const uint8_t*>(B);
    p.C = static_cast<uint16_t*>(C);
    p.sa = sa;
    p.sb = sb;
    p.M = (int)M; p.N = (int)N; p.K = (int)K;
    p.lda = lda; p.ldb = ldb; p.ldc = ldc; p.lsa = lsa; p.lsb = lsb;
    p.ca = static_cast<const uint16_t*>(ca);
    p.cb = static_cast<const uint16_t*>(cb);
    p.ldca = ldca; p.ldcb = ldcb;
    if (M == 0 || N == 0) return 0;
    // M <= 64; up to 192 rows (row groups of 64) while the 256 x 256 tiles
    // would give fewer than a quarter of the CUs work (at N = 7168, 28 tiles:
    // 16x7168x18432 took 321 us tiled, 31 us streamed; 128x7168x18432 325 vs
    // 140 us; at 256 rows the tiles win for K <= 7168)
    const int64_t ncu = cu_count() > 0 ? cu_count() : 256;
    const bool few_tiles = M <= 192 && ((N + 255) / 256) * 4 < ncu;
    if ((M <= BSN_MAX_M || few_tiles) && 32 * ldb < (1ll << 31) && BSN_MAX_M * lda < (1ll << 31) &&
        (int64_t)M * lsa < (1ll << 28) && (K / 128) * lsb < (1ll << 28))
        return group_n == 1 ? launch_blockscale_narrow<true>(p, stream) : launch_blockscale_narrow<false>(p, stream);
    return group_n == 1 ? launch_blockscale<true>(p, stream) : launch_blockscale<false>(p, stream);
}
