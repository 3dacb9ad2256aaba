// gemm_mainloop.h -- the pipelined K loop of the dense-operand scaled-MFMA
// GEMMs (A8W8, MXFP4 and the MoE grouped GEMM share it): tile configuration,
// LDS-direct K-tile ring, fragment double-buffering and MFMA issue order.
#pragma once
#include <type_traits>

#include "gemm_core.h"

namespace hkq {

template <int MODE, int WAVES_M, int WAVES_N, int TM, int TN, int KTB>
struct DenseCfg {
    using KT = KTile<KTB>;
    static constexpr int NW = WAVES_M * WAVES_N;
    static constexpr int BM = WAVES_M * TM * 32, BN = WAVES_N * TN * 32;
    static constexpr bool FP4 = MODE == MODE_MXFP4;
    static constexpr int SUB = (KTB / 64) * (FP4 ? 2 : 1);   // 64-deep MFMA K-steps per K-tile
    static constexpr int RPL = KT::ROWS_PER_LOAD;
    static constexpr int LA = BM / RPL / NW, LB = BN / RPL / NW;
    // FP4: the K-tile's e8m0 scales (KTB/16 bytes per row: one per 32 values)
    // ride in LDS after the data, as KTB/64 planes of one 4-byte word per row;
    // one 4-byte LDS-direct load per lane covers 64 rows of one plane. When a
    // tile has fewer (plane, 64-row group) pairs than waves, waves load the same
    // pair (identical bytes to the same place) so that every wave issues the
    // same number of loads per K-tile, which the vmcnt accounting relies on.
    static constexpr int PLANES = KTB / 64;
    static constexpr int SCA = FP4 ? BM * 4 * PLANES : 0, SCB = FP4 ? BN * 4 * PLANES : 0;
    static constexpr int GA = FP4 ? BM / 64 * PLANES : 1, GB = FP4 ? BN / 64 * PLANES : 1;
    static constexpr int LSA = FP4 ? (GA + NW - 1) / NW : 0, LSB = FP4 ? (GB + NW - 1) / NW : 0;
    static constexpr int STAGE = (BM + BN) * KTB + SCA + SCB;
    static constexpr int NLD = LA + LB + LSA + LSB;           // LDS-direct loads per wave per K-tile
    static constexpr int PARTS = FP4 ? 1 : 2;                 // ds_read_b128 per fragment per K-step
    static constexpr int NRD = 2 * PARTS * (TM > TN ? TM : TN);  // fragment read slots per K-step
    static constexpr int NSC = FP4 ? TM + TN : 0;             // scale reads per K-tile
    static constexpr int NMF = TM * TN, HALF = NMF / 2;       // MFMAs per K-step
    // epilogue: each wave stages its (TM*32) x (TN*32) bf16 sub-tile in LDS with a
    // padded row pitch, then writes whole 256-byte row segments of C
    static constexpr int EP_PITCH = TN * 32 * 2 + 16;
    static constexpr int EP_BYTES = NW * TM * 32 * EP_PITCH;
    static constexpr int lds_bytes(int ns) { return ns * STAGE > EP_BYTES ? ns * STAGE : EP_BYTES; }
    static_assert(LA >= 1 && LB >= 1, "tile too small for the wave count");
    static_assert(!FP4 || (GA % NW == 0 || NW % GA == 0), "A scale groups vs waves");
    static_assert(!FP4 || (GB % NW == 0 || NW % GB == 0), "B scale groups vs waves");
    static_assert((TN * 32 * 2) % 256 == 0, "epilogue rows are whole 256-byte segments");
};

// Where one workgroup's K-tiles come from. `a`/`b` point at the tile's first
// row (or at the tensor base when rows are gathered); loads at byte offsets at
// or beyond the *_bytes bounds read zero. FP4 only: the e8m0 scale rows.
struct LoopSrc {
    const uint8_t *a, *b;
    int64_t a_bytes, b_bytes;
    const uint8_t *as, *bs;
    int64_t as_bytes, bs_bytes, lsa, lsb;
    int KT;  // K-tiles
};

// Byte offset (row and logical chunk, excluding the K position) of LDS-direct
// load instruction i of `wave` for a plain row-major operand.
template <int NW, int KTB>
__device__ __forceinline__ uint32_t dense_row_off(int i, int wave, int lane, int64_t ld) {
    using KT = KTile<KTB>;
    const int r = (i * NW + wave) * KT::ROWS_PER_LOAD + lane / KT::CHUNKS;
    return (uint32_t)(r * ld) + (uint32_t)(KT::load_chunk(lane, r) << 4);
}

// Pipeline (per wave; one barrier per K-tile, NS ring stages):
//   K-tile kt lives in stage kt % NS. Its SUB K-steps run their MFMAs with
//   double-buffered fragments: the LDS reads of the next step are issued between
//   the MFMAs of the current one. Before the last step's MFMAs (SUB > 1) or
//   half-way through them (SUB == 1) a barrier (a) waits until K-tile kt+1 is
//   resident (at most NS-2 K-tiles of loads still in flight) and (b) retires
//   every wave's reads of stage kt % NS, which is then refilled with K-tile
//   kt+NS while the remaining MFMAs issue together with the reads of K-tile
//   kt+1's first step. sched_barrier between chunks keeps this order through
//   the compiler's scheduler.
//
// Fragments: lane half h (lane / 32) owns logical chunks [h * KTB/32, (h+1) *
// KTB/32) of every row; K-step ks uses chunks h*KTB/32 + 2ks + {0, 1} (FP8) or
// h*KTB/32 + ks (FP4). The order in which K enters the sums is the same for A
// and B, so the products are unchanged; for FP4 it makes the lane's e8m0 bytes
// of one K-tile contiguous (2 bytes for KTB 64, one 4-byte plane for KTB 128),
// and the MFMA's opsel picks byte ks.
//
// a_off/b_off: per load instruction, the byte offset of the lane's row and
// logical chunk inside src.a / src.b (OOB for rows that must read zero).
// On return acc holds the tile's fp32 sums and every wave is past a vmcnt(0)
// barrier, so the caller may reuse the LDS.
template <int MODE, int WAVES_M, int WAVES_N, int TM, int TN, int KTB, int NS>
__device__ __forceinline__ void gemm_mainloop(const LoopSrc& src,
                                              const uint32_t (&a_off)[DenseCfg<MODE, WAVES_M, WAVES_N, TM, TN, KTB>::LA],
                                              const uint32_t (&b_off)[DenseCfg<MODE, WAVES_M, WAVES_N, TM, TN, KTB>::LB],
                                              HKQ_LDS uint8_t* smem, int lane, int wave, v16f (&acc)[TN][TM]) {
    using Cfg = DenseCfg<MODE, WAVES_M, WAVES_N, TM, TN, KTB>;
    using KT = KTile<KTB>;
    constexpr int NW = Cfg::NW, BM = Cfg::BM, BN = Cfg::BN, SUB = Cfg::SUB;
    constexpr int LA = Cfg::LA, LB = Cfg::LB, LSA = Cfg::LSA, SCA = Cfg::SCA, STAGE = Cfg::STAGE;
    constexpr int GA = Cfg::GA, GB = Cfg::GB;
    constexpr int NLD = Cfg::NLD, PARTS = Cfg::PARTS, NRD = Cfg::NRD, NSC = Cfg::NSC;
    constexpr int NMF = Cfg::NMF, HALF = Cfg::HALF;
    constexpr bool FP4 = Cfg::FP4;
    constexpr int HCH = KTB / 32;  // logical chunks per lane half
    static_assert(NS >= 2 && (NS - 1) * NLD <= 63, "ring depth and vmcnt budget");
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int KTN = src.KT;

    // Load instruction idx of K-tile kt into `stage`: A rows, B rows, then (FP4)
    // scale words: group g covers plane g % PLANES of rows (g / PLANES)*64 + lane.
    // For kt >= KTN the buffers are empty, so the loads read zero (the loop needs
    // no branches).
    auto load_piece = [&](int kt, int stage, int idx) {
        const int kb = kt * KTB;
        const bool live = kt < KTN;
        HKQ_LDS uint8_t* st = smem + stage * STAGE;
        if (idx < LA) {
            lds_load16(src.a + kb, live ? (uint32_t)(src.a_bytes - kb) : 0u, st + (idx * NW + wave) * 1024, a_off[idx]);
        } else if (idx < LA + LB) {
            const int i = idx - LA;
            lds_load16(src.b + kb, live ? (uint32_t)(src.b_bytes - kb) : 0u, st + BM * KTB + (i * NW + wave) * 1024,
                       b_off[i]);
        } else if (idx < LA + LB + LSA) {
            constexpr int PL = Cfg::PLANES;
            const int g = ((idx - LA - LB) * NW + wave) % GA;
            const int plane = g % PL, rows = g / PL;
            const int kb4 = kt * 4 * PL + plane * 4;
            const uint32_t off = (uint32_t)((rows * 64 + lane) * src.lsa);
            lds_load4(src.as + kb4, live ? (uint32_t)(src.as_bytes - kb4) : 0u,
                      st + (BM + BN) * KTB + plane * BM * 4 + rows * 256, off);
        } else {
            constexpr int PL = Cfg::PLANES;
            const int g = ((idx - LA - LB - LSA) * NW + wave) % GB;
            const int plane = g % PL, rows = g / PL;
            const int kb4 = kt * 4 * PL + plane * 4;
            const uint32_t off = (uint32_t)((rows * 64 + lane) * src.lsb);
            lds_load4(src.bs + kb4, live ? (uint32_t)(src.bs_bytes - kb4) : 0u,
                      st + (BM + BN) * KTB + SCA + plane * BN * 4 + rows * 256, off);
        }
    };

    const int arow = wm * TM * 32 + (lane & 31);
    const int brow = wn * TN * 32 + (lane & 31);
    const int khalf = lane >> 5;

    struct Frags {
        v4i a[TM][PARTS], b[TN][PARTS];
    };
    // Fragment read slot idx of K-step ks, A and B tiles interleaved
    // (a0 b0 a1 b1 ...) so the first MFMAs' operands arrive first; slots past
    // TM (A) or TN (B) tiles are empty.
    auto read_piece = [&](int stage, int ks, Frags& f, int idx) {
        const HKQ_LDS uint8_t* At = smem + stage * STAGE;
        const int t = idx / (2 * PARTS), isb = (idx / PARTS) & 1, part = idx % PARTS;
        if ((isb ? TN : TM) <= t) return;
        const int row = (isb ? brow : arow) + t * 32;
        const int chunk = khalf * HCH + (FP4 ? ks : 2 * ks + part);
        const v4i v = lds_read16(At + (isb ? BM * KTB : 0) + KT::swz(row, chunk));
        if (isb) f.b[t][part] = v;
        else f.a[t][part] = v;
    };
    // MXFP4: per m/n-tile the lane's e8m0 bytes of the K-tile, byte ks for
    // K-step ks: 16 bits at byte 2h of the row's word (KTB 64) or the row's word
    // of plane h (KTB 128). The value goes to the MFMA unchanged.
    struct Scales {
        int a[TM], b[TN];
    };
    auto read_scale = [&](int stage, Scales& s, int idx) {
        if constexpr (FP4) {
            const HKQ_LDS uint8_t* sca = smem + stage * STAGE + (BM + BN) * KTB;
            const bool isa = idx < TM;
            const int t = isa ? idx : idx - TM;
            const int row = (isa ? arow : brow) + t * 32;
            const HKQ_LDS uint8_t* base = isa ? sca : sca + SCA;
            int w;
            if constexpr (KTB == 64) w = *reinterpret_cast<const HKQ_LDS uint16_t*>(base + row * 4 + khalf * 2);
            else w = *reinterpret_cast<const HKQ_LDS int*>(base + khalf * (isa ? BM : BN) * 4 + row * 4);
            if (isa) s.a[t] = w;
            else s.b[t] = w;
        }
    };

#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = v16f{};

    // MFMA idx (accumulator i*TM + j) of K-step ks
    auto mfma_one = [&](const Frags& f, int ks, const Scales& s, int idx) {
        const int i = idx / TM, j = idx % TM;
        v8i a, b;
        if constexpr (PARTS == 2) {
            b = v8i{f.b[i][0][0], f.b[i][0][1], f.b[i][0][2], f.b[i][0][3], f.b[i][1][0], f.b[i][1][1], f.b[i][1][2], f.b[i][1][3]};
            a = v8i{f.a[j][0][0], f.a[j][0][1], f.a[j][0][2], f.a[j][0][3], f.a[j][1][0], f.a[j][1][1], f.a[j][1][2], f.a[j][1][3]};
        } else {
            b = v8i{f.b[i][0][0], f.b[i][0][1], f.b[i][0][2], f.b[i][0][3], 0, 0, 0, 0};
            a = v8i{f.a[j][0][0], f.a[j][0][1], f.a[j][0][2], f.a[j][0][3], 0, 0, 0, 0};
        }
        if constexpr (FP4) {
            switch (ks & 3) {
                case 0: acc[i][j] = mfma_sel<true, 0, 0>(b, a, acc[i][j], s.b[i], s.a[j]); break;
                case 1: acc[i][j] = mfma_sel<true, 1, 1>(b, a, acc[i][j], s.b[i], s.a[j]); break;
                case 2: acc[i][j] = mfma_sel<true, 2, 2>(b, a, acc[i][j], s.b[i], s.a[j]); break;
                default: acc[i][j] = mfma_sel<true, 3, 3>(b, a, acc[i][j], s.b[i], s.a[j]); break;
            }
        } else {
            acc[i][j] = mfma_sel<false, 0, 0>(b, a, acc[i][j], 127, 127);
        }
    };

    Frags F[2];
    Scales S[2];
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int i = 0; i < NLD; ++i) load_piece(t, t, i);
    tile_barrier<(NS - 1) * NLD>();  // K-tile 0 resident
#pragma unroll
    for (int i = 0; i < NRD; ++i) read_piece(0, 0, F[0], i);
#pragma unroll
    for (int i = 0; i < NSC; ++i) read_scale(0, S[0], i);

    // One K-tile; P is the tile's parity (fragment and scale buffers alternate).
    auto ktile = [&](int kt, int stage, auto parity) {
        constexpr int P = decltype(parity)::value;
        const int next_stage = stage + 1 == NS ? 0 : stage + 1;
        // phase A: steps 0 .. SUB-2, the fragment reads of the next step spread
        // over the MFMAs
#pragma unroll
        for (int ks = 0; ks + 1 < SUB; ++ks) {
#pragma unroll
            for (int c = 0; c < NMF; ++c) {
                mfma_one(F[(P * SUB + ks) & 1], ks, S[P], c);
#pragma unroll
                for (int i = c * NRD / NMF; i < (c + 1) * NRD / NMF; ++i)
                    read_piece(stage, ks + 1, F[(P * SUB + ks + 1) & 1], i);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // phase B: last step. Its fragments were read during the previous step,
        // so with SUB > 1 the stage is retired as soon as phase A's reads are
        // done and the barrier comes first (the refill of the stage then spreads
        // over all of the step's MFMAs); with SUB == 1 half of the MFMAs are
        // issued before the barrier, keeping the matrix pipe busy meanwhile.
        constexpr int LAST = SUB - 1;
        constexpr int PRE = SUB > 1 ? 0 : HALF, POST = NMF - PRE;
        const Frags& cur = F[(P * SUB + LAST) & 1];
        Frags& nxt = F[(P * SUB + LAST + 1) & 1];
#pragma unroll
        for (int c = 0; c < PRE; ++c) mfma_one(cur, LAST, S[P], c);
        __builtin_amdgcn_sched_barrier(0);
        tile_barrier<(NS - 2) * NLD>();  // K-tile kt+1 resident; stage kt % NS retired
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < POST; ++c) {
            mfma_one(cur, LAST, S[P], PRE + c);
#pragma unroll
            for (int i = c * NLD / POST; i < (c + 1) * NLD / POST; ++i) load_piece(kt + NS, stage, i);
#pragma unroll
            for (int i = c * NRD / POST; i < (c + 1) * NRD / POST; ++i) read_piece(next_stage, 0, nxt, i);
#pragma unroll
            for (int i = c * NSC / POST; i < (c + 1) * NSC / POST; ++i) read_scale(next_stage, S[P ^ 1], i);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    int stage = 0;
    int kt = 0;
    for (; kt + 1 < KTN; kt += 2) {
        ktile(kt, stage, std::integral_constant<int, 0>{});
        stage = stage + 1 == NS ? 0 : stage + 1;
        ktile(kt + 1, stage, std::integral_constant<int, 1>{});
        stage = stage + 1 == NS ? 0 : stage + 1;
    }
    if (kt < KTN) ktile(kt, stage, std::integral_constant<int, 0>{});
    mfma_drain();
    tile_barrier<0>();  // every wave is done with the stages and no load is in flight
}

}  // namespace hkq
