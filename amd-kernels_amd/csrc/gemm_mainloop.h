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
    // K-steps per K-tile: 64 bytes of K per row each (FP8: one 64-deep MFMA per
    // output sub-tile; FP4: two, one per 32-byte half of the lane's fragment;
    // BF16: two 16-deep MFMAs, one per 16-byte part)
    static constexpr int SUB = KTB / 64;
    static constexpr int RPL = KT::ROWS_PER_LOAD;
    static constexpr int LA = BM / RPL / NW, LB = BN / RPL / NW;
    // FP4 e8m0 scales, KTB/16 bytes per row per K-tile (one per 32 values).
    // KTB 128 (SBLK): the scales of SB_KT = 4 K-tiles (32 bytes per row) form a
    // block, held in a 2-slot ring after the K-tile ring; a block is fetched in
    // 32-row groups (two lanes per row, 16 bytes each: 32 lines of 32 bytes per
    // load instead of 64 lines of 4 bytes), one group per wave per K-tile over
    // the 4 K-tiles before it is first read.
    // KTB 64: the K-tile's 4 scale bytes per row ride in its stage after the
    // data; one 4-byte LDS-direct load per lane covers 64 rows.
    // When there are fewer groups than load slots, slots load the same group
    // again (identical bytes to the same place) so that every wave issues the
    // same number of loads per K-tile, which the vmcnt accounting relies on.
    static constexpr bool SBLK = FP4 && KTB == 128;
    static constexpr int SB_KT = 4, SB_GROUPS = (BM + BN) / 32, SB_SLOT = (BM + BN) * 32;
    static constexpr int SB_BYTES = SBLK ? 2 * SB_SLOT : 0;
    static constexpr bool SK = FP4 && !SBLK;
    static constexpr int SCA = SK ? BM * 4 : 0, SCB = SK ? BN * 4 : 0;
    static constexpr int GA = SK ? BM / 64 : 1, GB = SK ? BN / 64 : 1;
    static constexpr int LSA = SK ? (GA + NW - 1) / NW : 0, LSB = SK ? (GB + NW - 1) / NW : 0;
    static constexpr int STAGE = (BM + BN) * KTB + SCA + SCB;
    // Ring layout of NS stages: the A tiles of all stages, then the B tiles,
    // then (64-byte FP4 K-tiles) their scales: every fragment read of one
    // operand then lies within a 64 KB immediate offset of one base register.
    static constexpr int A_ST = BM * KTB, B_ST = BN * KTB, S_ST = SCA + SCB;
    static constexpr int a_stage(int ns, int s) { return s * A_ST; }
    static constexpr int b_stage(int ns, int s) { return ns * A_ST + s * B_ST; }
    static constexpr int s_stage(int ns, int s) { return ns * (A_ST + B_ST) + s * S_ST; }
    static constexpr int NLD = LA + LB + LSA + LSB + (SBLK ? 1 : 0);  // LDS-direct loads per wave per K-tile
    static constexpr int PARTS = 2;                           // ds_read_b128 per fragment per K-step
    static constexpr int NRD = 2 * PARTS * (TM > TN ? TM : TN);  // fragment read slots per K-step
    static constexpr int NSC = FP4 ? TM + TN : 0;             // scale reads per K-tile
    static constexpr int NMF = TM * TN, HALF = NMF / 2;       // MFMAs per K-step
    // epilogue: each wave stages its (TM*32) x (TN*32) bf16 sub-tile in LDS with a
    // padded row pitch, then writes whole 256-byte row segments of C
    static constexpr int EP_PITCH = TN * 32 * 2 + 16;
    static constexpr int EP_BYTES = NW * TM * 32 * EP_PITCH;
    static constexpr int lds_bytes(int ns) { return ns * STAGE + SB_BYTES > EP_BYTES ? ns * STAGE + SB_BYTES : EP_BYTES; }
    static_assert(LA >= 1 && LB >= 1, "tile too small for the wave count");
    static_assert(!SK || (GA % NW == 0 || NW % GA == 0), "A scale groups vs waves");
    static_assert(!SK || (GB % NW == 0 || NW % GB == 0), "B scale groups vs waves");
    static_assert(!SBLK || (SB_GROUPS <= SB_KT * NW && BM % 32 == 0), "scale block groups vs load slots");
    static_assert((TN * 32 * 2) % 128 == 0, "epilogue rows are whole 128-byte segments");
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
    // FP4 with gathered A rows (sa_gathered): the byte offset inside `as` of the
    // A scale row this lane loads, per load slot (128-byte K-tiles: slot
    // u % SB_KT of scale unit u; 64-byte K-tiles: the k-th A scale load of a
    // K-tile), beyond as_bytes for rows that read zero. Otherwise tile row r's
    // scale row is at r * lsa.
    bool sa_gathered = false;
    uint32_t sa_row[4] = {0u, 0u, 0u, 0u};
    // N-contiguous B (BT): bytes from one K-tile of B to the next (128 rows of K)
    int64_t b_kstep = 0;
};

// Byte offset (row and logical chunk, excluding the K position) of LDS-direct
// load instruction i of `wave` for a plain row-major operand.
template <int NW, int KTB>
__device__ __forceinline__ uint32_t dense_row_off(int i, int wave, int lane, int64_t ld) {
    using KT = KTile<KTB>;
    const int r = (i * NW + wave) * KT::ROWS_PER_LOAD + lane / KT::CHUNKS;
    return (uint32_t)(r * ld) + (uint32_t)(KT::load_chunk(lane, r) << 4);
}

// Per-lane source offsets of an operand's LDS-direct loads within a K-tile:
// load i reads at byte v[i] (row and logical chunk; out of bounds for rows that
// must read zero). Loop-invariant, so the K loop keeps them in VGPRs.
template <int N>
struct TableOff {
    uint32_t v[N];
};
template <int NW, int KTB, int N>
__device__ __forceinline__ TableOff<N> dense_offs(int wave, int lane, int64_t ld) {
    TableOff<N> o;
#pragma unroll
    for (int i = 0; i < N; ++i) o.v[i] = dense_row_off<NW, KTB>(i, wave, lane, ld);
    return o;
}

// Load offsets of an N-contiguous B tile (KTileT; row stride ld bytes): load i
// of `wave` writes rows (i*NW + wave)*4 .. +3 of the K-tile; the lane carries
// physical chunk lane % 16 of row (i*NW + wave)*4 + lane / 16, i.e. logical
// chunk phys(r, lane % 16) (the swizzle is its own inverse).
template <int NW, int N>
__device__ __forceinline__ TableOff<N> dense_offs_t(int wave, int lane, int64_t ld) {
    TableOff<N> o;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int r = (i * NW + wave) * KTileT::ROWS_PER_LOAD + lane / 16;
        o.v[i] = (uint32_t)(r * ld) + (uint32_t)(KTileT::phys(r, lane % 16) << 4);
    }
    return o;
}

// LDS base addresses of the transposed B fragment reads (BT): per n-tile t
// of the wave, the lane's row 64h + (j >> 1) (h = lane / 32, j = lane % 16)
// and byte 8 (j & 1) of logical chunk (wave's first column)/16 + 2t + g
// (g = (lane / 16) & 1). The K-step / part / read rows ride as immediates in
// multiples of 8 rows, so the row's swizzle term is the lane constant
// 2 (j >> 1).
template <int TN>
struct TBase {
    uint32_t v[TN];
};
template <int TN>
__device__ __forceinline__ TBase<TN> tr_bases(uint32_t b_region, int wave_col, int lane) {
    TBase<TN> o;
    const int j = lane & 15, g = (lane >> 4) & 1, h = lane >> 5;
    const int row = 64 * h + (j >> 1);
#pragma unroll
    for (int t = 0; t < TN; ++t) {
        const int chunk = (wave_col >> 4) + 2 * t + g;
        o.v[t] = b_region + (uint32_t)(row * KTileT::ROW + (KTileT::phys(row, chunk) << 4) + 8 * (j & 1));
        asm volatile("" : "+v"(o.v[t]));
    }
    return o;
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
// KTB/32) of every row; K-step ks uses chunks h*KTB/32 + 2ks + {0, 1}, read as
// two 16-byte parts (FP8: the two halves of one MFMA operand; FP4 and BF16:
// one MFMA each). The order in which K enters the sums is the same for A and B, so the
// products are unchanged; for FP4 it makes the lane's e8m0 bytes of one K-tile
// contiguous (2 bytes for KTB 64, one 4-byte plane for KTB 128), and the MFMA's
// opsel picks byte 2ks + part.
//
// a_off/b_off: the lane's row and logical chunk offsets inside src.a / src.b of
// each load instruction (TableOff; out of bounds for rows that must read zero).
// On return acc holds the tile's fp32 sums and every wave is past a vmcnt(0)
// barrier, so the caller may reuse the LDS.
template <int MODE, int WAVES_M, int WAVES_N, int TM, int TN, int KTB, int NS, bool BT = false, typename AOff,
          typename BOff>
__device__ __forceinline__ void gemm_mainloop(const LoopSrc& src, const AOff& a_off, const BOff& b_off,
                                              HKQ_LDS uint8_t* smem, int lane, int wave, v16f (&acc)[TN][TM]) {
    using Cfg = DenseCfg<MODE, WAVES_M, WAVES_N, TM, TN, KTB>;
    using KT = KTile<KTB>;
    constexpr int NW = Cfg::NW, BM = Cfg::BM, BN = Cfg::BN, SUB = Cfg::SUB;
    constexpr int LA = Cfg::LA, LB = Cfg::LB, LSA = Cfg::LSA, SCA = Cfg::SCA, STAGE = Cfg::STAGE;
    constexpr int GA = Cfg::GA, GB = Cfg::GB;
    constexpr int NLD = Cfg::NLD, PARTS = Cfg::PARTS, NRD = Cfg::NRD, NSC = Cfg::NSC;
    constexpr int NMF = Cfg::NMF, HALF = Cfg::HALF;
    constexpr int RDS = NMF > 1 ? NMF / 2 : 1;  // MFMA slots that carry phase A's fragment reads
    constexpr bool FP4 = Cfg::FP4;
    constexpr int HCH = KTB / 32;  // logical chunks per lane half
    static_assert(NS >= 2 && (NS - 1) * NLD + 3 <= 63, "ring depth and vmcnt budget");
    static_assert(!Cfg::SBLK || NS == 2, "the scale-block schedule assumes a 2-stage ring");
    static_assert(Cfg::SB_KT <= 4 && LSA <= 4, "gathered scale rows: at most 4 load slots per lane");
    static_assert(!BT || (KTB == 128 && Cfg::BN == KTileT::ROW && (MODE == MODE_A8W8 || MODE == MODE_MXFP4)),
                  "N-contiguous B: FP8 or FP4, 128-byte K-tiles of 256 columns");
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int KTN = src.KT;

    // Scale unit u (SBLK): group slot k = u % SB_KT of block u / SB_KT; this
    // wave loads group (k * NW + wave) % SB_GROUPS of the block's [A; B] rows.
    // Per slot the group, its operand and the lane's row offset are fixed;
    // the block moves the offset by 32 bytes. Units of blocks past the last
    // one (the look-ahead past the end) land in a slot no remaining K-tile
    // reads.
    // BT (N-contiguous B scales, one row of N bytes per 32 values of K): the
    // block's B part holds its 32 rows of the tile's 256 columns in the KTileT
    // order (8 KB at BM * 32 in the slot); B group g - BM / 32 carries rows
    // 4 (g - BM / 32) + lane / 16, and a block moves them by 32 rows.
    HKQ_LDS uint8_t* sblk = smem + NS * STAGE;
    constexpr int SBK = Cfg::SBLK ? Cfg::SB_KT : 1;
    int su_g[SBK];
    bool su_a[SBK];
    uint32_t su_off[SBK];
#pragma unroll
    for (int k = 0; k < SBK; ++k) {
        const int g = (k * NW + wave) % Cfg::SB_GROUPS;
        const int r = g * 32 + (lane >> 1);
        su_g[k] = g;
        su_a[k] = g * 32 < BM;
        // row slot s = lane / 2 of the group; its two 16-byte halves are stored
        // swapped when bit 3 of s is set (see read_scale)
        const uint32_t half = (uint32_t)((lane & 1) ^ ((lane >> 4) & 1));
        const uint32_t a_row = src.sa_gathered ? src.sa_row[k & 3] : (uint32_t)(r * src.lsa);
        const uint32_t b_row = (uint32_t)((r - BM) * src.lsb);
        su_off[k] = (su_a[k] ? a_row : b_row) + half * 16u;
        if (BT && !su_a[k]) {
            const int rt = 4 * (g - BM / 32) + lane / 16;
            su_off[k] = (uint32_t)(rt * src.lsb) + (uint32_t)(KTileT::phys(rt, lane % 16) << 4);
        }
        asm volatile("" : "+v"(su_off[k]));
    }
    const v4i desc_as = buffer_desc(src.as, (uint32_t)(src.as_bytes < 0x7FFFFFFF ? (src.as_bytes > 0 ? src.as_bytes : 0) : 0x7FFFFFFF));
    const v4i desc_bs = buffer_desc(src.bs, (uint32_t)(src.bs_bytes < 0x7FFFFFFF ? (src.bs_bytes > 0 ? src.bs_bytes : 0) : 0x7FFFFFFF));
    auto load_scale_unit = [&](int u, auto kslot) {
        constexpr int k = decltype(kslot)::value;
        const int blk = u / Cfg::SB_KT;
        const uint32_t adv = BT && !su_a[k] ? (uint32_t)(blk * 32) * (uint32_t)src.lsb : (uint32_t)(blk * 32);
        lds_load16_d(su_a[k] ? desc_as : desc_bs, sblk + (blk & 1) * Cfg::SB_SLOT + su_g[k] * 1024, su_off[k] + adv);
    };

    // Operand buffers: the whole tile's rows, K positions in the lane offsets.
    // Rows that read zero have offsets at or past 2^31 (OOB), past every
    // extent; the loads of K-tiles kt >= KTN (the ring's look-ahead past the
    // end, into stages the loop never reads) take such an offset too, so they
    // count for vmcnt without fetching anything (a split's K range would
    // otherwise pull NS K-tiles of the next split's bytes).
    const v4i desc_a = buffer_desc(src.a, (uint32_t)(src.a_bytes < 0x7FFFFFFF ? (src.a_bytes > 0 ? src.a_bytes : 0) : 0x7FFFFFFF));
    const v4i desc_b = buffer_desc(src.b, (uint32_t)(src.b_bytes < 0x7FFFFFFF ? (src.b_bytes > 0 ? src.b_bytes : 0) : 0x7FFFFFFF));

    // Load instruction idx of K-tile kt into `stage`: A rows, B rows, then (FP4)
    // scales: KTB 64: group g covers rows g*64 + lane; KTB 128: one scale unit,
    // kt + SB_KT - 1 (with the 2-stage ring the loads issued in K-tile j are
    // those of K-tile j + 2, so K-tile j fetches unit j + SB_KT + 1: block b + 1
    // arrives during K-tiles 4b-1 .. 4b+2, after block b-1, which used the same
    // slot, was last read in K-tile 4b-2, and before K-tile 4b+3 reads it).
    // For kt >= KTN the scale buffers are empty, so those loads read zero (the
    // loop needs no branches).
    // kslot: (kt + SB_KT - 1) % SB_KT, the slot of the scale unit (SBLK)
    auto load_piece = [&](int kt, int stage, int idx, auto kslot) {
        const int kb = kt * KTB;
        const bool live = kt < KTN;
        if constexpr (Cfg::SBLK) {
            if (idx == LA + LB) {
                load_scale_unit(kt + Cfg::SB_KT - 1, kslot);
                return;
            }
        }
        if (idx < LA) {
            lds_load16_d(desc_a, smem + Cfg::a_stage(NS, stage) + (idx * NW + wave) * 1024,
                         live ? a_off.v[idx] + (uint32_t)kb : 0x80000000u);
        } else if (idx < LA + LB) {
            const int i = idx - LA;
            const uint32_t kbb = BT ? (uint32_t)(kt * src.b_kstep) : (uint32_t)kb;
            lds_load16_d(desc_b, smem + Cfg::b_stage(NS, stage) + (i * NW + wave) * 1024,
                         live ? b_off.v[i] + kbb : 0x80000000u);
        } else if (idx < LA + LB + LSA) {
            const int g = ((idx - LA - LB) * NW + wave) % GA;
            const int kb4 = kt * 4;
            const uint32_t off =
                src.sa_gathered ? src.sa_row[(idx - LA - LB) & 3] : (uint32_t)((g * 64 + lane) * src.lsa);
            lds_load4(src.as + kb4, live ? (uint32_t)(src.as_bytes - kb4) : 0u, smem + Cfg::s_stage(NS, stage) + g * 256,
                      off);
        } else {
            const int g = ((idx - LA - LB - LSA) * NW + wave) % GB;
            const int kb4 = kt * 4;
            const uint32_t off = (uint32_t)((g * 64 + lane) * src.lsb);
            lds_load4(src.bs + kb4, live ? (uint32_t)(src.bs_bytes - kb4) : 0u,
                      smem + Cfg::s_stage(NS, stage) + SCA + g * 256, off);
        }
    };

    const int khalf = lane >> 5;

    // LDS addresses of the fragment reads. The lane reads rows
    // (wave's first row) + t*32 + lane%32; rows 32 apart share the chunk
    // swizzle. Per (K-step, part) one base address per operand (its region,
    // the wave's rows and the lane's row and chunk); stage and row tile t are
    // immediate offsets below 64 KB. The empty asm keeps the compiler from
    // folding a region offset back into the immediates, which it would then
    // have to split into one register per row tile.
    uint32_t a_base[SUB][PARTS], b_base[SUB][PARTS];
#pragma unroll
    for (int ks = 0; ks < SUB; ++ks)
#pragma unroll
        for (int part = 0; part < PARTS; ++part) {
            const uint32_t lo = (uint32_t)KT::swz(lane & 31, khalf * HCH + 2 * ks + part);
            a_base[ks][part] = (uint32_t)(uintptr_t)smem + (uint32_t)(Cfg::a_stage(NS, 0) + wm * TM * 32 * KTB) + lo;
            b_base[ks][part] = (uint32_t)(uintptr_t)smem + (uint32_t)(Cfg::b_stage(NS, 0) + wn * TN * 32 * KTB) + lo;
            asm volatile("" : "+v"(a_base[ks][part]));
            asm volatile("" : "+v"(b_base[ks][part]));
        }

    const TBase<TN> bt = BT ? tr_bases<TN>((uint32_t)(uintptr_t)smem + (uint32_t)Cfg::b_stage(NS, 0), wn * TN * 32, lane)
                            : TBase<TN>{};

    struct Frags {
        v4i a[TM][PARTS], b[TN][PARTS];
    };
    // Fragment read slot idx of K-step ks, A and B tiles interleaved
    // (a0 b0 a1 b1 ...) so the first MFMAs' operands arrive first; slots past
    // TM (A) or TN (B) tiles are empty.
    auto read_piece = [&](int stage, int ks, Frags& f, int idx) {
        const int t = idx / (2 * PARTS), isb = (idx / PARTS) & 1, part = idx % PARTS;
        if ((isb ? TN : TM) <= t) return;
        if (BT && isb) {
            // the lane's 16 bytes of K [64h + 32ks + 16part, +16) of its column:
            // two transposed reads of 8 rows each
            const uint32_t b = bt.v[t] + (uint32_t)(Cfg::b_stage(NS, stage) - Cfg::b_stage(NS, 0)) +
                               (uint32_t)((32 * ks + 16 * part) * KTileT::ROW);
            const v2i lo = lds_read_tr8(reinterpret_cast<const HKQ_LDS uint8_t*>((uintptr_t)b));
            const v2i hi = lds_read_tr8(reinterpret_cast<const HKQ_LDS uint8_t*>((uintptr_t)(b + 8 * KTileT::ROW)));
            f.b[t][part] = v4i{lo[0], lo[1], hi[0], hi[1]};
            return;
        }
        const uint32_t base = isb ? b_base[ks][part] + (uint32_t)(Cfg::b_stage(NS, stage) - Cfg::b_stage(NS, 0))
                                  : a_base[ks][part] + (uint32_t)Cfg::a_stage(NS, stage);
        const v4i v = lds_read16(reinterpret_cast<const HKQ_LDS uint8_t*>((uintptr_t)(base + (uint32_t)(t * 32 * KTB))));
        if (isb) f.b[t][part] = v;
        else f.a[t][part] = v;
    };
    // MXFP4: per m/n-tile the lane's e8m0 bytes of K-tile kt, byte 2ks + part
    // for part `part` of K-step ks: KTB 64: 16 bits at byte 2h of the row's word
    // in the stage; KTB 128: the 4 bytes at 8 * (kt % SB_KT) + 4h of the row's
    // 32 bytes in the block slot. The value goes to the MFMA unchanged.
    struct Scales {
        int a[TM], b[TN];
    };
    // Scale reads: row ra = (wave's first row) + t*32 + lane%32 keeps bit 3 of
    // lane%32, so the swapped-half XOR below is a per-lane constant.
    const int sc_lo = (lane & 31) * 32 + khalf * 4, sc_x = (((lane & 31) >> 3) & 1) << 4;
    const int sk_lo = (lane & 31) * 4 + khalf * 2;
    // BT scales: per n-tile the lane's row (j >> 1) and byte 8 (j & 1) of
    // logical chunk (wave's first column)/16 + 2t + g of the block's B part; a
    // transposed read returns the column's 8 scale bytes of a K-tile (rows
    // 8 (kt % 4) + 0..7), of which lane half h takes bytes 4h .. 4h+3
    const TBase<TN> bts = BT && FP4 ? tr_bases<TN>((uint32_t)(uintptr_t)sblk + (uint32_t)(BM * 32) -
                                                        (uint32_t)(64 * khalf * KTileT::ROW),
                                                    wn * TN * 32, lane)
                                    : TBase<TN>{};
    auto read_scale = [&](int stage, int kt, Scales& s, int idx) {
        if constexpr (FP4) {
            const bool isa = idx < TM;
            const int t = isa ? idx : idx - TM;
            int w;
            if constexpr (Cfg::SBLK) {
                // byte o = 8 * (kt % 4) + 4h of the row's 32; the 16-byte halves of
                // rows with bit 3 set are swapped, so the 32 lanes of a read (32
                // consecutive rows, 32-byte pitch) hit 16 distinct bank pairs
                const HKQ_LDS uint8_t* slot = sblk + ((kt / Cfg::SB_KT) & 1) * Cfg::SB_SLOT;
                if (BT && !isa) {
                    const uint32_t b = bts.v[t] + (uint32_t)(((kt / Cfg::SB_KT) & 1) * Cfg::SB_SLOT) +
                                       (uint32_t)((kt % Cfg::SB_KT) * 8 * KTileT::ROW);
                    const v2i v = lds_read_tr8(reinterpret_cast<const HKQ_LDS uint8_t*>((uintptr_t)b));
                    w = khalf ? v[1] : v[0];
                } else {
                    const int wave_row = isa ? wm * TM * 32 : BM + wn * TN * 32;
                    const int o = ((kt % Cfg::SB_KT) * 8) ^ sc_x;
                    w = *reinterpret_cast<const HKQ_LDS int*>(slot + wave_row * 32 + sc_lo + o + t * 1024);
                }
            } else {
                const HKQ_LDS uint8_t* sca = smem + Cfg::s_stage(NS, stage) + (isa ? 0 : SCA);
                const int wave_row = isa ? wm * TM * 32 : wn * TN * 32;
                w = *reinterpret_cast<const HKQ_LDS uint16_t*>(sca + wave_row * 4 + sk_lo + t * 128);
            }
            if (isa) s.a[t] = w;
            else s.b[t] = w;
        }
    };

#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = v16f{};

    // MFMA slot idx (accumulator i*TM + j) of K-step ks: one FP8 MFMA on the
    // 32-byte fragments, two FP4 MFMAs (one per 16-byte half, scale bytes 2ks
    // and 2ks + 1 of the lane's scale word) or two BF16 MFMAs (one per half)
    auto mfma_one = [&](const Frags& f, int ks, const Scales& s, int idx) {
        const int i = idx / TM, j = idx % TM;
        if constexpr (MODE == MODE_BF16) {
            acc[i][j] = mfma_bf16(f.b[i][0], f.a[j][0], acc[i][j]);
            acc[i][j] = mfma_bf16(f.b[i][1], f.a[j][1], acc[i][j]);
        } else if constexpr (FP4) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const v8i b = v8i{f.b[i][q][0], f.b[i][q][1], f.b[i][q][2], f.b[i][q][3], 0, 0, 0, 0};
                const v8i a = v8i{f.a[j][q][0], f.a[j][q][1], f.a[j][q][2], f.a[j][q][3], 0, 0, 0, 0};
                switch ((2 * ks + q) & 3) {
                    case 0: acc[i][j] = mfma_sel<true, 0, 0>(b, a, acc[i][j], s.b[i], s.a[j]); break;
                    case 1: acc[i][j] = mfma_sel<true, 1, 1>(b, a, acc[i][j], s.b[i], s.a[j]); break;
                    case 2: acc[i][j] = mfma_sel<true, 2, 2>(b, a, acc[i][j], s.b[i], s.a[j]); break;
                    default: acc[i][j] = mfma_sel<true, 3, 3>(b, a, acc[i][j], s.b[i], s.a[j]); break;
                }
            }
        } else {
            const v8i b = v8i{f.b[i][0][0], f.b[i][0][1], f.b[i][0][2], f.b[i][0][3], f.b[i][1][0], f.b[i][1][1], f.b[i][1][2], f.b[i][1][3]};
            const v8i a = v8i{f.a[j][0][0], f.a[j][0][1], f.a[j][0][2], f.a[j][0][3], f.a[j][1][0], f.a[j][1][1], f.a[j][1][2], f.a[j][1][3]};
            acc[i][j] = mfma_sel<false, 0, 0>(b, a, acc[i][j], 127, 127);
        }
    };

    Frags F[2];
    Scales S[2];
    // prologue: (SBLK) units 0 .. SB_KT-2 of scale block 0, then K-tiles 0 .. NS-1
    // (whose loads carry units SB_KT-1, SB_KT: the rest of block 0, the start of 1)
    using Q0 = std::integral_constant<int, 0>;
    using Q1 = std::integral_constant<int, 1>;
    using Q2 = std::integral_constant<int, 2>;
    using Q3 = std::integral_constant<int, 3>;
    if constexpr (Cfg::SBLK) {
        static_assert(Cfg::SB_KT == 4 && NS == 2, "scale slots of the prologue");
        load_scale_unit(0, Q0{});
        load_scale_unit(1, Q1{});
        load_scale_unit(2, Q2{});
#pragma unroll
        for (int i = 0; i < NLD; ++i) load_piece(0, 0, i, Q3{});
#pragma unroll
        for (int i = 0; i < NLD; ++i) load_piece(1, 1, i, Q0{});
    } else {
#pragma unroll
        for (int t = 0; t < NS; ++t)
#pragma unroll
            for (int i = 0; i < NLD; ++i) load_piece(t, t, i, Q0{});
    }
    tile_barrier<(NS - 1) * NLD>();  // K-tile 0 (and everything issued before it) resident
#pragma unroll
    for (int i = 0; i < NRD; ++i) read_piece(0, 0, F[0], i);
#pragma unroll
    for (int i = 0; i < NSC; ++i) read_scale(0, 0, S[0], i);

    // One K-tile; P is the tile's parity (fragment and scale buffers alternate),
    // Q (SBLK) kt % 4: its loads carry scale unit kt + NS + 3, slot (Q + 1) % 4.
    auto ktile = [&](int kt, int stage, auto parity, auto qslot) {
        constexpr int P = decltype(parity)::value;
        using KS = std::integral_constant<int, (decltype(qslot)::value + NS + Cfg::SB_KT - 1) % 4>;
        const int next_stage = stage + 1 == NS ? 0 : stage + 1;
        // phase A: steps 0 .. SUB-2, the fragment reads of the next step spread
        // over the first RDS MFMA slots, so that they have landed when the
        // barrier below waits for every LDS read of the stage
#pragma unroll
        for (int ks = 0; ks + 1 < SUB; ++ks) {
#pragma unroll
            for (int c = 0; c < NMF; ++c) {
                mfma_one(F[(P * SUB + ks) & 1], ks, S[P], c);
#pragma unroll
                for (int i = c * NRD / RDS; i < (c + 1) * NRD / RDS && i < NRD; ++i)
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
            for (int i = c * NLD / POST; i < (c + 1) * NLD / POST; ++i) load_piece(kt + NS, stage, i, KS{});
#pragma unroll
            for (int i = c * NRD / POST; i < (c + 1) * NRD / POST; ++i) read_piece(next_stage, 0, nxt, i);
#pragma unroll
            for (int i = c * NSC / POST; i < (c + 1) * NSC / POST; ++i) read_scale(next_stage, kt + 1, S[P ^ 1], i);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    int kt = 0;
    if constexpr (Cfg::SBLK) {
        // four K-tiles per iteration: the scale slot of each is a constant
        for (; kt + 3 < KTN; kt += 4) {
            ktile(kt, 0, Q0{}, Q0{});
            ktile(kt + 1, 1, Q1{}, Q1{});
            ktile(kt + 2, 0, Q0{}, Q2{});
            ktile(kt + 3, 1, Q1{}, Q3{});
        }
        if (kt < KTN) ktile(kt, 0, Q0{}, Q0{});
        if (kt + 1 < KTN) ktile(kt + 1, 1, Q1{}, Q1{});
        if (kt + 2 < KTN) ktile(kt + 2, 0, Q0{}, Q2{});
    } else {
        int stage = 0;
        for (; kt + 1 < KTN; kt += 2) {
            ktile(kt, stage, Q0{}, Q0{});
            stage = stage + 1 == NS ? 0 : stage + 1;
            ktile(kt + 1, stage, Q1{}, Q0{});
            stage = stage + 1 == NS ? 0 : stage + 1;
        }
        if (kt < KTN) ktile(kt, stage, Q0{}, Q0{});
    }
    mfma_drain();
    tile_barrier<0>();  // every wave is done with the stages and no load is in flight
}

}  // namespace hkq
