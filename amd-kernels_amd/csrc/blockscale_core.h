// blockscale_core.h -- the K loop of the 8-wave block-scale GEMMs (the dense
// GEMM and the MoE grouped GEMM): 256 x 256 tiles of 8 waves of 64 x 128
// (TM = 2 m-tiles, TN = 4 n-tiles of 32), two waves per SIMD, K-tiles of one
// 128-wide scale group.
//
// fp32 group scales cannot ride in the MFMA's e8m0 scale operands, so every
// K-tile is promoted on the VALU: per 32x32 sub-tile two chained MFMAs (the
// group's two 64-deep K-steps) make a fresh partial P, then
// acc += P * sa[row] * sb[column]. The accumulators stay in arch VGPRs (128
// fp32 per lane), so a promotion is one v_fma per element; the MFMAs write P
// straight to VGPRs. A wave's promotions run while the other wave of its SIMD
// issues MFMAs (measured on MI355X: one wave alternating 16 MFMA pairs with
// their promotions takes the sum of both times, two waves overlap them).
// The loop is bound by LDS traffic rather than by the matrix pipe: per K-tile
// the ring takes 64 KB of LDS-direct writes and the 8 waves read 192 KB of
// fragments (each A row by 2 waves, each B row by 4), about 2000 cycles at
// 128 B per clock against 1792 cycles of MFMAs (measured on MI355X: with
// the MFMAs taken out the loop still runs at 80% of its full time).
//
// LDS: a 2-stage ring of A and B K-tiles (stage: A 32 KB, then B as two 16 KB
// column halves, so every fragment offset fits the ds_read immediate), then 2
// scale slots of 2 KB: the tile's 256 row scales at 0, its column scales at
// 1024 (256 per-column values, or per-block values as the caller lays out).
#pragma once
#include "gemm_mainloop.h"

namespace hkq {

constexpr int BS_WM = 4, BS_WN = 2, BS_TM = 2, BS_TN = 4, BS_NW = BS_WM * BS_WN;
constexpr int BS_BM = BS_WM * BS_TM * 32, BS_BN = BS_WN * BS_TN * 32;
constexpr int BS_KT = 128, BS_NS = 2;
constexpr int BS_LA = BS_BM * BS_KT / 1024 / BS_NW, BS_LB = BS_BN * BS_KT / 1024 / BS_NW;  // 4, 4 loads per wave
constexpr int BS_NLD = BS_LA + BS_LB + 2;  // + one row-scale and one column-scale load per wave and K-tile
constexpr int BS_STAGE = (BS_BM + BS_BN) * BS_KT;                                       // 64 KB
constexpr int BS_BOFF = BS_BM * BS_KT;                                                  // 32 KB
constexpr int BS_SC = BS_NS * BS_STAGE;
constexpr int BS_SLOT = 2048;  // row scales at 0, column scales at 1024
constexpr int BS_RING = BS_SC + 2 * BS_SLOT;
constexpr int BS_EPI = BS_NW * BS_TM * 32 * (BS_TN * 32 * 2 + 16);
constexpr int BS_LDS = BS_RING > BS_EPI ? BS_RING : BS_EPI;
static_assert(BS_LDS <= 160 * 1024, "LDS budget of a CDNA4 CU");

// How the K loop reads the column scales of its slot (floats from 256):
//   BS_SB_COL:   one per column, tile column c at 256 + c
//   BS_SB_WAVE:  one per 128-column half of the tile, half h at 256 + h
//                (the wave's columns lie in one half)
//   BS_SB_NTILE: one per 32-column n-tile, read at 256 + (its first column)
enum : int { BS_SB_COL = 0, BS_SB_WAVE = 1, BS_SB_NTILE = 2 };

// LDS byte offset (from the ring base) of operand load q (< BS_LA + BS_LB) of
// a wave into stage st: loads fill 1 KB blocks (8 rows of 128 bytes), block
// q * NW + wave of the stage (the B loads' blocks start at BS_BOFF). Load q
// reads rows (q * NW + wave) * 8 .. +7 of its operand tile.
static_assert(BS_BOFF == BS_LA * BS_NW * 1024, "B blocks follow the A blocks");
__device__ __forceinline__ uint32_t bs_load_dst(int st, int q, int wave) {
    return (uint32_t)(st * BS_STAGE + q * BS_NW * 1024 + wave * 1024);
}

// The K loop over K-tiles [0, KTN). issue(kt, q) issues load q (0 ..
// BS_NLD-1: A rows, B rows, row scales, column scales) of K-tile kt into
// stage kt & 1 and scale slot kt & 1 (loads of kt >= KTN read zero). On
// return every load has landed and every wave is past its LDS reads.
// The wave computes tile rows wm*64 .. +63 and TN n-tiles from tile column cn
// (TN may differ between the waves of a workgroup: every wave issues the same
// loads and barriers). COMPUTE false: a wave whose rows all lie outside the
// tile only issues its share of the loads and takes the barriers (acc stays
// zero), leaving its SIMD's MFMA and VALU pipes to the other wave.
// BT: the B K-tiles are N-contiguous (KTileT: 128 rows of K x 256 columns at
// BS_BOFF of each stage), their operands built with transposed reads.
template <int SBM, int TN, bool COMPUTE = true, bool BT = false, class Issue>
__device__ __forceinline__ void bs8_kloop(HKQ_LDS uint8_t* smem, int lane, int wm, int cn, int KTN, Issue& issue,
                                          v16f (&acc)[TN][BS_TM]) {
    using KT = KTile<BS_KT>;
    constexpr int TM = BS_TM;
    static_assert(TN >= 1 && TN <= BS_TN, "n-tiles per wave");
    const int khalf = lane >> 5;
    if constexpr (!COMPUTE) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) acc[i][j] = v16f{};
#pragma unroll
        for (int q = 0; q < BS_NLD; ++q) issue(0, q);
        for (int kt = 0; kt < KTN; ++kt) {
            tile_barrier<0>();
#pragma unroll
            for (int q = 0; q < BS_NLD; ++q) issue(kt + 1, q);
        }
        tile_barrier<0>();
        return;
    }

    // Fragment reads: lane row lane%32 of m-tile / n-tile t, logical chunks
    // 4*ks + 2*khalf + {0, 1} of K-step ks. Rows 32 apart share the swizzle, so
    // per (K-step, part) one base per operand and t*4 KB as the immediate.
    uint32_t a_base[2][2], b_base[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int c = 4 * ks + 2 * khalf + h;
            a_base[ks][h] = (uint32_t)(uintptr_t)smem + (uint32_t)KT::swz(wm * TM * 32 + (lane & 31), c);
            b_base[ks][h] = (uint32_t)(uintptr_t)smem + (uint32_t)(BS_BOFF + cn * BS_KT) + (uint32_t)KT::swz(lane & 31, c);
        }
    // BT: per n-tile the lane's row 32 * khalf + (j >> 1) (j = lane % 16) and
    // byte 8 (j & 1) of logical chunk cn / 16 + 2t + g (g = (lane / 16) & 1);
    // K-step, part and read rows are immediates in multiples of 8 rows
    uint32_t bt_base[TN];
    if constexpr (BT) {
        const int j = lane & 15, g = (lane >> 4) & 1, row = 32 * khalf + (j >> 1);
#pragma unroll
        for (int t = 0; t < TN; ++t)
            bt_base[t] = (uint32_t)(uintptr_t)smem + (uint32_t)BS_BOFF +
                         (uint32_t)(row * KTileT::ROW + (KTileT::phys(row, cn / 16 + 2 * t + g) << 4) + 8 * (j & 1));
    }
    // the bases of stage st, rebuilt from opaque copies each K-tile: left
    // visible, the compiler hoists every piece address out of the loop
    struct Bases {
        uint32_t a[2][2], b[2][2], bt[TN];
    };
    auto bases = [&](int st) {
        Bases r;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                r.a[ks][h] = a_base[ks][h] + (uint32_t)(st * BS_STAGE);
                asm volatile("" : "+v"(r.a[ks][h]));
                if constexpr (!BT) {
                    r.b[ks][h] = b_base[ks][h] + (uint32_t)(st * BS_STAGE);
                    asm volatile("" : "+v"(r.b[ks][h]));
                }
            }
        if constexpr (BT) {
#pragma unroll
            for (int t = 0; t < TN; ++t) {
                r.bt[t] = bt_base[t] + (uint32_t)(st * BS_STAGE);
                asm volatile("" : "+v"(r.bt[t]));
            }
        }
        return r;
    };
    // a tile's operand for both K-steps: [K-step] of 8 dwords
    struct Op {
        v8i k[2];
    };
    auto read_step = [&](const uint32_t (&base)[2][2], int t, int ks) {
        const v4i lo = lds_read16(reinterpret_cast<const HKQ_LDS uint8_t*>((uintptr_t)(base[ks][0] + (uint32_t)(t * 32 * BS_KT))));
        const v4i hi = lds_read16(reinterpret_cast<const HKQ_LDS uint8_t*>((uintptr_t)(base[ks][1] + (uint32_t)(t * 32 * BS_KT))));
        return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    auto read_op = [&](const uint32_t (&base)[2][2], int t) {
        Op o;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) o.k[ks] = read_step(base, t, ks);
        return o;
    };
    // BT: K-step ks of n-tile t from the transposed tile, rows 64ks + 32khalf
    // + 8q (q = 0..3) of the lane's column
    auto read_step_t = [&](const Bases& rb, int t, int ks) {
        v2i q[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            q[r] = lds_read_tr8(reinterpret_cast<const HKQ_LDS uint8_t*>(
                (uintptr_t)(rb.bt[t] + (uint32_t)((64 * ks + 8 * r) * KTileT::ROW))));
        return v8i{q[0][0], q[0][1], q[1][0], q[1][1], q[2][0], q[2][1], q[3][0], q[3][1]};
    };
    auto read_b_step = [&](const Bases& rb, int t, int ks) {
        if constexpr (BT) return read_step_t(rb, t, ks);
        else return read_step(rb.b, t, ks);
    };
    auto read_b_op = [&](const Bases& rb, int t) {
        Op o;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) o.k[ks] = read_b_step(rb, t, ks);
        return o;
    };

#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = v16f{};

#pragma unroll
    for (int q = 0; q < BS_NLD; ++q) issue(0, q);
    for (int kt = 0; kt < KTN; ++kt) {
        // K-tile kt resident and every wave past its reads of stage (kt-1) & 1,
        // which takes K-tile kt+1 (its loads spread over the n-tiles below: a
        // burst at this point stalls the waves on the load queue)
        tile_barrier<0>();
        const int st = kt & 1;
        const HKQ_LDS float* sl = reinterpret_cast<const HKQ_LDS float*>(smem + BS_SC + st * BS_SLOT);
        float saj[TM];
#pragma unroll
        for (int j = 0; j < TM; ++j) saj[j] = sl[wm * TM * 32 + j * 32 + (lane & 31)];
        float sbt[TN];
#pragma unroll
        for (int i = 0; i < TN; ++i)
            sbt[i] = SBM == BS_SB_WAVE ? sl[256 + cn / 128] : SBM == BS_SB_NTILE ? sl[256 + cn + i * 32] : 0.f;
        const Bases rb = bases(st);
        // the first MFMA's operands (K-step 0 of n-tile 0 and m-tile 0) are
        // read first: the LDS counter is in order, so the MFMAs can start
        // while the other fragments are still in flight
        Op fa[TM], fb;
        fb.k[0] = read_b_step(rb, 0, 0);
        fa[0].k[0] = read_step(rb.a, 0, 0);
        fb.k[1] = read_b_step(rb, 0, 1);
        fa[0].k[1] = read_step(rb.a, 0, 1);
#pragma unroll
        for (int j = 1; j < TM; ++j) fa[j] = read_op(rb.a, j);
        // the group partial P of sub-tile (i, j), then acc += P * sa * sb. With
        // one scale per n-tile (not per column) the promotion of a sub-tile
        // waits until the MFMAs of the next one are issued, so that this wave's
        // VALU works while the matrix pipe runs them (measured on MI355X: 3-6%
        // faster at the DeepSeek shapes); per-column scales keep the direct
        // order (the deferred sub-tile's 16 column scales do not fit the
        // register budget).
        constexpr bool DEFER = SBM != BS_SB_COL;
        v16f Pq;
        int qi = 0, qj = 0;
        auto promote = [&](const v16f& P, int i, int j, const v4f* sbn) {
            const float sc = saj[j] * sbt[i];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float f = SBM == BS_SB_COL ? saj[j] * sbn[r >> 2][r & 3] : sc;
                acc[i][j][r] = __builtin_fmaf(P[r], f, acc[i][j][r]);
            }
        };
#pragma unroll
        for (int i = 0; i < TN; ++i) {
            constexpr int PER = (BS_NLD + TN - 1) / TN;
#pragma unroll
            for (int q = i * PER; q < (i + 1) * PER && q < BS_NLD; ++q) issue(kt + 1, q);
            // n-tile i+1's operand and column scales, read under this n-tile's MFMAs
            Op fb_next;
            if (i + 1 < TN) fb_next = read_b_op(rb, i + 1);
            v4f sbn[4];
            if constexpr (SBM == BS_SB_COL) {
#pragma unroll
                for (int g = 0; g < 4; ++g)
                    sbn[g] = *reinterpret_cast<const HKQ_LDS v4f*>(sl + 256 + cn + i * 32 + 8 * g + 4 * khalf);
            }
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const v16f p0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb.k[0], fa[j].k[0], v16f{}, 0, 0, 0,
                                                                              127, 0, 127);
                const v16f P = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb.k[1], fa[j].k[1], p0, 0, 0, 0, 127,
                                                                             0, 127);
                if constexpr (DEFER) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (i + j > 0) promote(Pq, qi, qj, nullptr);
                    __builtin_amdgcn_sched_barrier(0);
                    Pq = P;
                    qi = i;
                    qj = j;
                } else {
                    promote(P, i, j, sbn);
                }
            }
            if (i + 1 < TN) fb = fb_next;
        }
        if constexpr (DEFER) promote(Pq, qi, qj, nullptr);
    }
    tile_barrier<0>();  // no load in flight, every wave past its reads: the LDS takes the epilogue
}

}  // namespace hkq
