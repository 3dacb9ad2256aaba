// gemm_stream.h -- the pipelined K loop of gemm_mainloop.h run over a stream of
// output tiles by one persistent workgroup: the K-tiles of consecutive tiles
// form one sequence through the LDS ring, so the loads of tile t+1's first
// K-tiles are issued during tile t's last ones and the ring never drains.
// Between two tiles the epilogue runs from registers only (the ring already
// holds the next tile's first K-tiles), and the next tile's first K-step
// starts its accumulators from zero (a literal-zero MFMA accumulator input),
// so no accumulator is cleared.
//
// Restrictions (the caller checks them): 128-byte K-tiles in a 2-stage ring,
// and a K-tile count per tile that is a multiple of 8, so that tiles start at
// stage 0 with the fragment parity 0 and (MXFP4) the scale blocks of 4 K-tiles
// never straddle two tiles and alternate their ring slot across tiles.
#pragma once
#include <type_traits>

#include "gemm_mainloop.h"

namespace hkq {

// Where one tile's K-tiles come from (the fields of LoopSrc a dense tile needs,
// with 32-bit extents: two of these stay in SGPRs across the stream).
struct StreamSrc {
    const uint8_t *a, *b;    // the tile's first A / B row
    const uint8_t *as, *bs;  // MXFP4: its first e8m0 scale rows
    uint32_t a_bytes, b_bytes, as_bytes, bs_bytes;  // loads at or past these read zero
};

// Seq: { int tiles; int KT; uint32_t lsa, lsb; __device__ StreamSrc src(int t) const;  (t < tiles)
//        static constexpr bool GATHER;   // true: the A rows differ per tile and
//        __device__ void a_rows(int t, AOff& a_off) const;  // sets tile t's load offsets;
//        called where the loads switch to tile t (two K-tiles before the end of
//        tile t - 1), after at least one vmcnt(0) barrier of tile t - 1 }
// Epi: { __device__ void begin(int t); __device__ void end(int t, v16f (&acc)[TN][TM]); }
//   begin(t) runs before tile t's first K-tile is computed (e.g. to prefetch
//   the tile's epilogue scales; loads it issues are waited for by the loop's
//   next barrier), end(t, acc) after tile t's last MFMA has drained; it must
//   not touch the LDS ring. On return every wave is past a vmcnt(0) barrier.
// BT: B tiles N-contiguous (KTileT layout, transposed fragment reads; the
// sequence then provides b_kstep, the bytes from one K-tile of B to the next).
template <int MODE, int WAVES_M, int WAVES_N, int TM, int TN, bool BT = false, typename AOff, typename BOff,
          typename Seq, typename Epi>
__device__ __forceinline__ void gemm_stream(const Seq& seq, AOff& a_off, const BOff& b_off, HKQ_LDS uint8_t* smem,
                                            int lane, int wave, v16f (&acc)[TN][TM], Epi& epi) {
    constexpr int KTB = 128, NS = 2;
    using Cfg = DenseCfg<MODE, WAVES_M, WAVES_N, TM, TN, KTB>;
    using KT = KTile<KTB>;
    constexpr int NW = Cfg::NW, BM = Cfg::BM, SUB = Cfg::SUB;
    constexpr int LA = Cfg::LA, LB = Cfg::LB, STAGE = Cfg::STAGE;
    constexpr int NLD = Cfg::NLD, PARTS = Cfg::PARTS, NRD = Cfg::NRD, NSC = Cfg::NSC;
    constexpr int NMF = Cfg::NMF;
    constexpr bool FP4 = Cfg::FP4;
    constexpr int HCH = KTB / 32;
    static_assert(SUB == 2 && !Cfg::SK, "128-byte K-tiles");
    static_assert((NS - 1) * NLD + 3 <= 63, "vmcnt budget");
    static_assert(!BT || (Cfg::BN == KTileT::ROW && MODE == MODE_A8W8), "N-contiguous B: FP8 tiles of 256 columns");
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int KTN = seq.KT;

    // Loads run NS K-tiles (data) and NS + SB_KT - 1 scale units (MXFP4) ahead
    // of the compute, so near the end of a tile they read the next tile: `ld`
    // is the source the data loads read (K-tile kl of it, `ld_live` false past
    // the last tile), `ls` the one the scale units read. Each switches to the
    // next tile at the top of a K-tile body, before its MFMAs (a branch there
    // leaves the body's MFMA/load interleave in one basic block).
    StreamSrc ld = seq.src(0), ls = ld;
    bool ld_live = true, ls_live = true;

    HKQ_LDS uint8_t* sblk = smem + NS * STAGE;
    // LDS destination of a load: the wave's base plus a constant, rebuilt from
    // an opaque copy at each load so that the compiler keeps one register
    // instead of hoisting every (stage, piece) destination out of the loop.
    const uint32_t lds_wave = (uint32_t)(uintptr_t)smem + (uint32_t)wave * 1024u;
    auto wave_dst = [&](uint32_t c) {
        uint32_t d = lds_wave;
        asm volatile("" : "+s"(d));
        return reinterpret_cast<HKQ_LDS uint8_t*>(d + c);
    };
    // MXFP4 scale units (see gemm_mainloop): unit u of a block is loaded by
    // every wave into group ((u % SB_KT) * NW + wave) % SB_GROUPS, so per unit
    // slot k = u % SB_KT a wave's group and its lanes' row offsets are fixed:
    // computed once here (the 32-bit row offsets relative to the tile's first
    // scale row), the slot is a template argument at every use.
    constexpr int SBK = Cfg::SBLK ? Cfg::SB_KT : 1;
    int su_g[SBK];
    bool su_a[SBK];
    uint32_t su_off[SBK];
#pragma unroll
    for (int k = 0; k < SBK; ++k) {
        const int g = (k * NW + wave) % (Cfg::SBLK ? Cfg::SB_GROUPS : 1);
        const int r = g * 32 + (lane >> 1);
        su_g[k] = g;
        su_a[k] = g * 32 < BM;
        // row slot s = lane / 2 of the group; its two 16-byte halves are stored
        // swapped when bit 3 of s is set (see read_scale)
        const uint32_t half = (uint32_t)((lane & 1) ^ ((lane >> 4) & 1));
        su_off[k] = (su_a[k] ? (uint32_t)r * seq.lsa : (uint32_t)(r - BM) * seq.lsb) + half * 16u;
        asm volatile("" : "+v"(su_off[k]));
    }
    // scale unit u (slot K = u % SB_KT) of the tile `ls`
    auto load_scale_unit = [&](int u, auto kslot) {
        constexpr int K = decltype(kslot)::value;
        const int blk = u / Cfg::SB_KT;
        const bool live = ls_live && blk * Cfg::SB_KT < KTN;
        const uint8_t* base = (su_a[K] ? ls.as : ls.bs) + blk * 32;
        const uint32_t ext = su_a[K] ? ls.as_bytes : ls.bs_bytes, kb = (uint32_t)blk * 32u;
        lds_load16_u(base, live && ext > kb ? ext - kb : 0u, sblk + (blk & 1) * Cfg::SB_SLOT + su_g[K] * 1024,
                     su_off[K]);
    };

    // load instruction idx of K-tile kl of `ld` into `stage`; MXFP4: scale
    // unit kl + SB_KT - 1 of `ls` (slot KS), counted in `ls`'s own K-tiles
    // (kl + SB_KT - 1 - KTN once `ls` has switched ahead of `ld`)
    auto load_piece = [&](int kl, int ul, int stage, int idx, auto kslot) {
        if constexpr (Cfg::SBLK) {
            if (idx == LA + LB) {
                load_scale_unit(ul, kslot);
                return;
            }
        }
        const uint32_t kb = (uint32_t)(kl * KTB);
        if (idx < LA) {
            lds_load16_u(ld.a + kb, ld_live && ld.a_bytes > kb ? ld.a_bytes - kb : 0u,
                         wave_dst(Cfg::a_stage(NS, stage) + idx * NW * 1024), a_off.v[idx]);
        } else {
            const int i = idx - LA;
            uint32_t kbb = kb;
            if constexpr (BT) kbb = (uint32_t)kl * seq.b_kstep;
            lds_load16_u(ld.b + kbb, ld_live && ld.b_bytes > kbb ? ld.b_bytes - kbb : 0u,
                         wave_dst(Cfg::b_stage(NS, stage) + i * NW * 1024), b_off.v[i]);
        }
    };

    const int khalf = lane >> 5;
    // Per (K-step, part) one base address per operand (its region, the wave's
    // rows and the lane's row and chunk); stage and row tile are immediate
    // offsets below 64 KB. The empty asm keeps the compiler from folding a
    // region offset back into the immediates, which it would then have to
    // split into one register per row tile.
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

    // A lane's operand of one 64-byte K-step: two 16-byte parts (FP8: the two
    // halves of one MFMA operand; FP4 and BF16: one operand each).
    const TBase<TN> bt = BT ? tr_bases<TN>((uint32_t)(uintptr_t)smem + (uint32_t)Cfg::b_stage(NS, 0), wn * TN * 32, lane)
                            : TBase<TN>{};
    struct Frags {
        v4i a[TM][PARTS], b[TN][PARTS];
    };
    auto read_piece = [&](int stage, int ks, Frags& f, int idx) {
        const int t = idx / (2 * PARTS), isb = (idx / PARTS) & 1, part = idx % PARTS;
        if ((isb ? TN : TM) <= t) return;
        if (BT && isb) {
            // see gemm_mainloop: two transposed reads of 8 rows of K each
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
    struct Scales {
        int a[TM], b[TN];
    };
    const int sc_lo = (lane & 31) * 32 + khalf * 4, sc_x = (((lane & 31) >> 3) & 1) << 4;
    // the scale words of K-tile kt (slot Q = kt % SB_KT of its block)
    auto read_scale = [&](int kt, Scales& s, int idx, auto qslot) {
        if constexpr (FP4) {
            constexpr int Q = decltype(qslot)::value;
            const bool isa = idx < TM;
            const int t = isa ? idx : idx - TM;
            const HKQ_LDS uint8_t* slot = sblk + ((kt / Cfg::SB_KT) & 1) * Cfg::SB_SLOT;
            const int wave_row = isa ? wm * TM * 32 : BM + wn * TN * 32;
            const int o = (Q * 8) ^ sc_x;
            const int w = *reinterpret_cast<const HKQ_LDS int*>(slot + wave_row * 32 + sc_lo + o + t * 1024);
            if (isa) s.a[t] = w;
            else s.b[t] = w;
        }
    };

    // MFMA slot idx of K-step ks; ZERO: the accumulator input is zero (the
    // first K-step of a tile)
    auto mfma_one = [&](const Frags& f, int ks, const Scales& s, int idx, auto zero) {
        constexpr bool ZERO = decltype(zero)::value;
        const int i = idx / TM, j = idx % TM;
        if constexpr (MODE == MODE_BF16) {
            acc[i][j] = mfma_bf16(f.b[i][0], f.a[j][0], ZERO ? v16f{} : acc[i][j]);
            acc[i][j] = mfma_bf16(f.b[i][1], f.a[j][1], acc[i][j]);
        } else if constexpr (FP4) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const v8i b = v8i{f.b[i][q][0], f.b[i][q][1], f.b[i][q][2], f.b[i][q][3], 0, 0, 0, 0};
                const v8i a = v8i{f.a[j][q][0], f.a[j][q][1], f.a[j][q][2], f.a[j][q][3], 0, 0, 0, 0};
                const v16f c = (ZERO && q == 0) ? v16f{} : acc[i][j];
                switch ((2 * ks + q) & 3) {
                    case 0: acc[i][j] = mfma_sel<true, 0, 0>(b, a, c, s.b[i], s.a[j]); break;
                    case 1: acc[i][j] = mfma_sel<true, 1, 1>(b, a, c, s.b[i], s.a[j]); break;
                    case 2: acc[i][j] = mfma_sel<true, 2, 2>(b, a, c, s.b[i], s.a[j]); break;
                    default: acc[i][j] = mfma_sel<true, 3, 3>(b, a, c, s.b[i], s.a[j]); break;
                }
            }
        } else {
            const v8i b = v8i{f.b[i][0][0], f.b[i][0][1], f.b[i][0][2], f.b[i][0][3], f.b[i][1][0], f.b[i][1][1], f.b[i][1][2], f.b[i][1][3]};
            const v8i a = v8i{f.a[j][0][0], f.a[j][0][1], f.a[j][0][2], f.a[j][0][3], f.a[j][1][0], f.a[j][1][1], f.a[j][1][2], f.a[j][1][3]};
            acc[i][j] = mfma_sel<false, 0, 0>(b, a, ZERO ? v16f{} : acc[i][j], 127, 127);
        }
    };

    using Q0 = std::integral_constant<int, 0>;
    using Q1 = std::integral_constant<int, 1>;
    using Q2 = std::integral_constant<int, 2>;
    using Q3 = std::integral_constant<int, 3>;
    Frags F[2];
    Scales S[2];
    epi.begin(0);
    // units 0 .. SB_KT-2 of block 0, then K-tiles 0 and 1, whose loads carry
    // units SB_KT-1 and SB_KT (slots 3 and 0)
    if constexpr (Cfg::SBLK) {
        load_scale_unit(0, Q0{});
        load_scale_unit(1, Q1{});
        load_scale_unit(2, Q2{});
    }
#pragma unroll
    for (int i = 0; i < NLD; ++i) load_piece(0, Cfg::SB_KT - 1, 0, i, Q3{});
#pragma unroll
    for (int i = 0; i < NLD; ++i) load_piece(1, Cfg::SB_KT, 1, i, Q0{});
    tile_barrier<(NS - 1) * NLD>();
#pragma unroll
    for (int i = 0; i < NRD; ++i) read_piece(0, 0, F[0], i);
#pragma unroll
    for (int i = 0; i < NSC; ++i) read_scale(0, S[0], i, Q0{});

    int cur = 0;  // the tile being computed
    // One K-tile (see gemm_mainloop); FIRST: the tile's first K-tile, whose
    // first step starts the accumulators from zero; LAST: the tile's last
    // K-tile, which leaves the next tile's first fragments to be read after
    // the epilogue (keeping them live through it would exceed the registers).
    // VM: vector-memory operations younger than K-tile kt+1's loads when the
    // body waits for them (the C stores and scale loads of an epilogue that ran
    // after those loads were issued may stay in flight)
    // Q: kt % SB_KT (MXFP4's scale slots; K-tiles per tile are a multiple of
    // 8, so it also fixes the stage and the fragment parity)
    auto ktile_vm = [&](int kt, auto qslot, auto first, auto last, auto vm) {
        constexpr int Q = decltype(qslot)::value;
        constexpr int P = Q & 1;
        constexpr bool FIRST = decltype(first)::value;
        constexpr bool LAST = decltype(last)::value;
        constexpr int VM = decltype(vm)::value;
        using KS = std::integral_constant<int, (Q + 1) % 4>;  // kt + NS + SB_KT - 1 = kt + 5
        using QN = std::integral_constant<int, (Q + 1) % 4>;  // K-tile kt + 1
        const int stage = P, next_stage = P ^ 1;
        const int kl = kt + NS < KTN ? kt + NS : kt + NS - KTN;
        const int ul = kt + NS + Cfg::SB_KT - 1 < KTN ? kt + NS + Cfg::SB_KT - 1 : kt + NS + Cfg::SB_KT - 1 - KTN;
        // K-step 1's fragment reads go out over the first half of K-step 0's
        // MFMAs: the barrier below waits for every LDS read of the stage
        constexpr int RDS = NMF > 1 ? NMF / 2 : 1;
#pragma unroll
        for (int c = 0; c < NMF; ++c) {
            mfma_one(F[0], 0, S[P], c, std::integral_constant<bool, FIRST>{});
#pragma unroll
            for (int i = c * NRD / RDS; i < (c + 1) * NRD / RDS && i < NRD; ++i) read_piece(stage, 1, F[1], i);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_sched_barrier(0);
        tile_barrier<VM>();  // K-tile kt+1 resident; this stage retired
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < NMF; ++c) {
            mfma_one(F[1], 1, S[P], c, std::false_type{});
#pragma unroll
            for (int i = c * NLD / NMF; i < (c + 1) * NLD / NMF; ++i) load_piece(kl, ul, stage, i, KS{});
            if constexpr (!LAST) {
#pragma unroll
                for (int i = c * NRD / NMF; i < (c + 1) * NRD / NMF; ++i) read_piece(next_stage, 0, F[0], i);
#pragma unroll
                for (int i = c * NSC / NMF; i < (c + 1) * NSC / NMF; ++i) read_scale(kt + 1, S[P ^ 1], i, QN{});
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto ktile = [&](int kt, auto qslot, auto first, auto last) {
        ktile_vm(kt, qslot, first, last, std::integral_constant<int, (NS - 2) * NLD>{});
    };

    using F0 = std::false_type;
    for (int t = 0; t < seq.tiles; ++t) {
        cur = t;
        if (t > 0) {
            epi.begin(t);
            // K-tile 1's loads went out before the previous tile's epilogue:
            // its C stores (and this tile's scale loads) need not be waited for
            constexpr int VM_EPI = (NS - 2) * NLD + Epi::VM_ISSUED;
            ktile_vm(0, Q0{}, std::true_type{}, F0{}, std::integral_constant<int, VM_EPI < 63 ? VM_EPI : 63>{});
        } else {
            ktile(0, Q0{}, std::true_type{}, F0{});
        }
        ktile(1, Q1{}, F0{}, F0{});
        // The sources switch between K-tile bodies (a branch inside one would
        // split its MFMA/load interleave): the scale units of the next tile
        // start with K-tile KTN - 5 (MXFP4), its data with K-tile KTN - 2.
        // MXFP4 runs four K-tiles per iteration, so that every scale slot is a
        // constant (KTN % 8 == 0: the loop ends at KTN - 6).
        if constexpr (Cfg::SBLK) {
            for (int kt = 2; kt + 6 < KTN; kt += 4) {
                ktile(kt, Q2{}, F0{}, F0{});
                ktile(kt + 1, Q3{}, F0{}, F0{});
                ktile(kt + 2, Q0{}, F0{}, F0{});
                ktile(kt + 3, Q1{}, F0{}, F0{});
            }
            ktile(KTN - 6, Q2{}, F0{}, F0{});
            ls_live = t + 1 < seq.tiles;
            ls = seq.src(min(t + 1, seq.tiles - 1));
            ktile(KTN - 5, Q3{}, F0{}, F0{});
            ktile(KTN - 4, Q0{}, F0{}, F0{});
            ktile(KTN - 3, Q1{}, F0{}, F0{});
        } else {
            for (int kt = 2; kt + 2 < KTN; kt += 2) {
                ktile(kt, Q0{}, F0{}, F0{});
                ktile(kt + 1, Q1{}, F0{}, F0{});
            }
        }
        ld_live = t + 1 < seq.tiles;
        ld = seq.src(min(t + 1, seq.tiles - 1));
        if constexpr (Seq::GATHER) seq.a_rows(min(t + 1, seq.tiles - 1), a_off);
        ktile(KTN - 2, Q2{}, F0{}, F0{});
        ktile(KTN - 1, Q3{}, F0{}, std::true_type{});
        mfma_drain();
        // Pin the finished accumulators here: without it the compiler sinks
        // the last K-tile's MFMAs past their scheduling barriers into the
        // epilogue (and into its copy on the loop exit), where their operands
        // and the epilogue's values together exceed the registers.
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) asm volatile("" ::"a"(acc[i][j]));
        epi.end(t, acc);
        // The next tile's K-tile 0 (stage 0) is resident: the last K-tile's
        // barrier waited for it. Read unconditionally (after the last tile the
        // values go unused): a condition here would let the compiler assume the
        // previous fragments stay live through the epilogue.
#pragma unroll
        for (int i = 0; i < NRD; ++i) read_piece(0, 0, F[0], i);
#pragma unroll
        for (int i = 0; i < NSC; ++i) read_scale(0, S[0], i, Q0{});
    }
    tile_barrier<0>();  // no load in flight, every wave past its reads
}

// Epilogue stores of a stream tile, shared by the stream kernels: per (n-tile
// pair ip, m-tile j) the wave's 32 rows x 64 columns (2 n-tiles: one 128-byte
// line per row) are scaled, converted and written to the wave's staging area
// (row pitch STREAM_STG_PITCH; each lane writes its 4 consecutive columns of a
// register group as 8 bytes), then read back so that lane l holds 16 bytes of
// row l / 8 at column 8 * (l % 8), and written with four 16-byte buffer
// stores, each covering 8 whole 128-byte lines of C (32 per wave and tile).
// Stores of 32-byte pieces straight from the accumulator layout (32 partial
// lines per instruction) held the epilogue up for longer: all CUs store their
// tiles at about the same time and those partial lines cost the memory path
// more requests. The stores are non-temporal: C is not read again by the
// kernel, and kept out of the caches it leaves them to the operands (measured
// on MI355X, A8W8 4096x28672x4096: 362.6 -> 332.0 us; 8192x28672x4096: 708 ->
// 662 us; 4096x14336x4096 within noise); whole lines keep them merged (the
// same policy on 32-byte pieces was 24% slower).
// Lanes whose row or columns lie outside C get an offset past the buffer, so
// every wave issues the same stores whatever the tile's edge. N % 4 == 0
// leaves one partial case: 8 columns of which the last 4 lie past N (the
// store would run into the next row); in a wave whose columns end there, such
// lanes write their first 4 columns with an extra 8-byte store.
//   base: C at the wave's first row and column, ldc its row pitch (elements);
//   rows / cols: of the wave's sub-tile inside C; rs[j]: the row scale of the
//   lane's row (lane % 32) of m-tile j; col_scale(i, g): the 4 column scales of
//   n-tile i, columns 8g + 4 (lane / 32) + 0..3.
constexpr int STREAM_STG_PITCH = 144;              // staged row: 64 bf16 columns + 16 bytes
constexpr int STREAM_STG = 32 * STREAM_STG_PITCH;  // one wave's staging area: 32 rows
constexpr int CPOL_NT = 2;                         // buffer-store cache policy: non-temporal

template <int TM, int TN, typename ColScale>
__device__ __forceinline__ void stream_store_tile(v16f (&acc)[TN][TM], HKQ_LDS uint8_t* stg, uint16_t* base, int64_t ldc,
                                                  int rows, int cols, const float (&rs)[TM], ColScale col_scale,
                                                  int lane) {
    static_assert(TN % 2 == 0, "n-tiles in pairs");
    const int khalf = lane >> 5, r = lane & 31;
    const auto rc = make_rsrc(base, 0x7FFFFFFFu);
    const bool ragged = cols < TN * 32 && (cols & 7) != 0;
    // The lane's offsets come from an opaque copy of the lane each tile: left
    // visible, the compiler hoists them out of the tile loop as invariants and
    // spills them.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int sr = ln >> 3, sc = (ln & 7) * 8;  // the store lane's row in an 8-row group, first column
    const uint32_t so = (uint32_t)((sr * ldc + sc) * 2);
    const uint32_t wr_lo = (uint32_t)(r * STREAM_STG_PITCH + 8 * khalf);
    const uint32_t rd_lo = (uint32_t)(sr * STREAM_STG_PITCH + (ln & 7) * 16);
#pragma unroll
    for (int ip = 0; ip < TN; ip += 2) {
        v4f cs[2][4];
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
            for (int g = 0; g < 4; ++g) cs[ii][g] = col_scale(ip + ii, g);
#pragma unroll
        for (int j = 0; j < TM; ++j) {
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
                // Explicit reads out of the accumulator registers, in store
                // order: the compiler's own copies tend to be hoisted to the
                // start of the epilogue, all 256 of them live at once.
                float v[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v[e]) : "a"(acc[ip + ii][j][e]));
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float a = rs[j];
                    const uint32_t lo = pk_bf16(v[4 * g + 0] * a * cs[ii][g][0], v[4 * g + 1] * a * cs[ii][g][1]);
                    const uint32_t hi = pk_bf16(v[4 * g + 2] * a * cs[ii][g][2], v[4 * g + 3] * a * cs[ii][g][3]);
                    *reinterpret_cast<HKQ_LDS v2i*>(stg + wr_lo + (ii * 32 + 8 * g) * 2) = v2i{(int)lo, (int)hi};
                }
            }
            // LDS operations of a wave complete in order: the reads see the
            // writes above, and the next group's writes follow these reads
            v4i dv[4];
#pragma unroll
            for (int pp = 0; pp < 4; ++pp)
                dv[pp] = *reinterpret_cast<const HKQ_LDS v4i*>(stg + rd_lo + pp * 8 * STREAM_STG_PITCH);
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
                const int m = j * 32 + pp * 8 + sr, c = ip * 32 + sc;
                const uint32_t at = so + (uint32_t)(((j * 32 + pp * 8) * ldc + ip * 32) * 2);
                __builtin_amdgcn_raw_buffer_store_b128(dv[pp], rc, m < rows && c + 8 <= cols ? at : OOB, 0, CPOL_NT);
                if (ragged)
                    __builtin_amdgcn_raw_buffer_store_b64(v2i{dv[pp][0], dv[pp][1]}, rc,
                                                          m < rows && c + 4 == cols ? at : OOB, 0, CPOL_NT);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

}  // namespace hkq
