// gemm.hip -- dense scaled GEMMs on CDNA4 matrix cores.
//
//   hkq_gemm_a8w8        C = bf16((A . B^T) * sa[m] * sb[n]), A/B E4M3FN codes
//                        (gemm-basic/gemm_a8w8/kernel.cpp:46-160 and
//                        gemm_a8w8_per_token_scale/kernel.cpp:49-156; formula
//                        tests/test_gemm.py:116);
//   hkq_gemm_mxfp4       C = bf16(sum_k e2m1(a) 2^(sa-127) e2m1(b) 2^(sb-127)),
//                        e8m0 scales per 32 K-values fed to the MFMA scale
//                        operands (gemm-basic/gemm_afp4wfp4/kernel.cpp:1-12 for
//                        the data format; the reference kernel itself consumes
//                        pre-dequantized bf16);
//   hkq_gemm_bf16,       C = bf16(A . B^T (+ bias[n])), bf16 operands
//   hkq_batched_gemm_*   (gemm_a16w16, formula tests/test_gemm.py:21-42),
//                        batched over grid.y (gemm-batched/batched_gemm_a8w8/
//                        kernel.cpp:59-203, batched_gemm_bf16/kernel.cpp:53-187;
//                        formulas tests/test_gemm.py:316-390).
#include <algorithm>
#include <mutex>

#include <cstdlib>

#include "gemm_stream.h"
#include "hkq_host.h"

namespace hkq {

struct DenseParams {
    const uint8_t* A;
    const uint8_t* B;
    uint16_t* C;
    const void* sa;
    const void* sb;
    int M, N, K;          // K in elements
    int kbytes;           // K in bytes per row of A/B (a multiple of the K-tile)
    int64_t lda, ldb;     // bytes
    int64_t ldc;          // elements
    int64_t lsa, lsb;     // MXFP4 scale row strides (bytes)
    int tiles_m, tiles_n, group_m;
    int n_whole;          // workgroups [0, n_whole) compute whole tiles 0 .. n_whole-1
    int n_split;          // tiles n_whole .. n_whole+n_split-1 are computed as two M halves
    int c16;              // rows of C are 16-byte aligned (ldc % 8 == 0, C 16-byte aligned)
    int splits;           // K splits of the split/skinny path (1: none)
    int kt_split;         // K-tiles per split
    float* ws;            // split partials (splits > 1)
    uint64_t* split_cnt;  // splits > 1: per tile, the arrival counter of its splits
    // batched A8W8 GEMMs: grid.y walks the batch; the operands of batch z start
    // z * bs_* further (bytes for A/B, elements for the others); bias bf16 [N]
    // per batch (nullptr: none), added after the scales
    int batch;  // 0 or 1: one GEMM
    const uint16_t* bias;
    int64_t bs_a, bs_b, bs_c, bs_sa, bs_sb, bs_bias;
};

// The parameters of this workgroup's batch (blockIdx.y).
__device__ __forceinline__ DenseParams batch_slice(const DenseParams& p) {
    DenseParams q = p;
    if (gridDim.y > 1) {
        const int64_t z = blockIdx.y;
        q.A += z * p.bs_a;
        q.B += z * p.bs_b;
        q.C += z * p.bs_c;
        q.sa = static_cast<const float*>(p.sa) + z * p.bs_sa;
        q.sb = static_cast<const float*>(p.sb) + z * p.bs_sb;
        if (p.bias) q.bias += z * p.bs_bias;
    }
    return q;
}

// bias of columns n .. n+3 (zero when there is none or n is past N; N % 4 == 0)
__device__ __forceinline__ float4 bias4(const DenseParams& p, int n) {
    if (!p.bias || n >= p.N) return make_float4(0.f, 0.f, 0.f, 0.f);
    const uint2 b = *reinterpret_cast<const uint2*>(p.bias + n);
    return make_float4(bf16_to_f32(b.x & 0xFFFF), bf16_to_f32(b.x >> 16), bf16_to_f32(b.y & 0xFFFF),
                       bf16_to_f32(b.y >> 16));
}

// Tile geometry of the dense GEMMs: 256 x 256 tiles computed by 4 waves of
// 128 x 128 (whole tiles) or 64 x 128 (M halves of a tile, 128 x 256). K-tiles
// are 128 bytes per row (whole 128-byte lines per row and load: half the
// cache-line requests of 64-byte K-tiles) in a 2-stage ring when K allows,
// else 64 bytes in a 4-stage ring.
constexpr int DENSE_WAVES_M = 2, DENSE_WAVES_N = 2, DENSE_TM = 4, DENSE_TN = 4;
constexpr int DENSE_BM = DENSE_WAVES_M * DENSE_TM * 32, DENSE_BN = DENSE_WAVES_N * DENSE_TN * 32;
// Skinny geometry (M <= 64): one row of (TM*32) x 256 tiles, 4 waves of
// (TM*32) x 64 side by side.
constexpr int SKINNY_WAVES_N = 4, SKINNY_TN = 2, SKINNY_BN = SKINNY_WAVES_N * SKINNY_TN * 32;
template <int KTB>
constexpr int dense_ns() { return KTB == 128 ? 2 : 4; }

// LDS of a dense workgroup: the K-tile ring / epilogue staging (the larger of
// the whole- and half-tile configurations), then (A8W8) the tile's row and
// column scales, 256 floats each, fetched at the start of the tile.
template <int MODE, int KTB>
constexpr int dense_ring_lds() {
    using Whole = DenseCfg<MODE, DENSE_WAVES_M, DENSE_WAVES_N, DENSE_TM, DENSE_TN, KTB>;
    using Half = DenseCfg<MODE, DENSE_WAVES_M, DENSE_WAVES_N, DENSE_TM / 2, DENSE_TN, KTB>;
    constexpr int NS = dense_ns<KTB>();
    return Whole::lds_bytes(NS) > Half::lds_bytes(NS) ? Whole::lds_bytes(NS) : Half::lds_bytes(NS);
}
template <int MODE, int KTB>
constexpr int dense_lds() { return dense_ring_lds<MODE, KTB>() + (MODE == MODE_A8W8 ? 2 * DENSE_BM * 4 : 0); }

// K loop of one (WM*TM*32) x (WN*TN*32) block of C at (m0, n0) over K-tiles
// [kt0, kt1): the operand sources start kt0 K-tiles into the rows, so the
// loop (and its scale-block schedule) counts K-tiles from 0.
template <int MODE, int WM, int WN, int TM, int TN, int KTB, int NS = dense_ns<KTB>()>
__device__ __forceinline__ void dense_kloop(const DenseParams& p, int m0, int n0, int kt0, int kt1, HKQ_LDS uint8_t* smem,
                                            v16f (&acc)[TN][TM]) {
    using Cfg = DenseCfg<MODE, WM, WN, TM, TN, KTB>;
    constexpr int NW = Cfg::NW, BM = Cfg::BM, BN = Cfg::BN;
    constexpr bool FP4 = Cfg::FP4;
    constexpr int SCB_PER_KT = KTB / 16;  // FP4 scale bytes per row per K-tile
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rows_a = min(p.M - m0, BM), rows_b = min(p.N - n0, BN);
    const int64_t kb0 = (int64_t)kt0 * KTB, ks0 = (int64_t)kt0 * SCB_PER_KT;

    LoopSrc src;
    src.a = p.A + (int64_t)m0 * p.lda + kb0;
    src.b = p.B + (int64_t)n0 * p.ldb + kb0;
    src.a_bytes = min((int64_t)rows_a * p.lda - kb0, (int64_t)0x7FFFFFFF);
    src.b_bytes = min((int64_t)rows_b * p.ldb - kb0, (int64_t)0x7FFFFFFF);
    src.as = FP4 ? static_cast<const uint8_t*>(p.sa) + (int64_t)m0 * p.lsa + ks0 : nullptr;
    src.bs = FP4 ? static_cast<const uint8_t*>(p.sb) + (int64_t)n0 * p.lsb + ks0 : nullptr;
    src.as_bytes = FP4 ? min((int64_t)rows_a * p.lsa - ks0, (int64_t)0x7FFFFFFF) : 0;
    src.bs_bytes = FP4 ? min((int64_t)rows_b * p.lsb - ks0, (int64_t)0x7FFFFFFF) : 0;
    src.lsa = p.lsa;
    src.lsb = p.lsb;
    src.KT = kt1 - kt0;
    const auto a_off = dense_offs<NW, KTB, Cfg::LA>(wave, lane, p.lda);
    const auto b_off = dense_offs<NW, KTB, Cfg::LB>(wave, lane, p.ldb);
    gemm_mainloop<MODE, WM, WN, TM, TN, KTB, NS>(src, a_off, b_off, smem, lane, wave, acc);
}

// One (TM*64) x 256 block of C: rows [m0, m0 + TM*64) of tile (tm, tn) of the
// 256 x 256 tile grid, starting `half` * 128 rows into the tile, on an NS-stage
// K-tile ring (the tile's row and column scales follow the ring).
template <int MODE, int TM, int KTB, int NS = dense_ns<KTB>()>
__device__ __forceinline__ void dense_block(const DenseParams& p, int tm, int tn, int half, HKQ_LDS uint8_t* smem) {
    constexpr int WAVES_M = DENSE_WAVES_M, WAVES_N = DENSE_WAVES_N, TN = DENSE_TN;
    using Cfg = DenseCfg<MODE, WAVES_M, WAVES_N, TM, TN, KTB>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN;
    constexpr int RING = NS == dense_ns<KTB>() ? dense_ring_lds<MODE, KTB>() : Cfg::lds_bytes(NS);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int khalf = lane >> 5;

    const int m0 = tm * DENSE_BM + half * BM, n0 = tn * BN;
    const int rows_a = min(p.M - m0, BM), rows_b = min(p.N - n0, BN);
    if (rows_a <= 0) return;  // the M half below the last row (uniform per workgroup)

    // A8W8: the tile's row and column scales go to LDS while the K loop runs
    // (rows past M / columns past N read zero); each wave loads 64 of each.
    // These loads are older than the K-tile loads, so the loop's vmcnt waits
    // cover them, and its final vmcnt(0) barrier makes them visible.
    HKQ_LDS uint8_t* scl = smem + RING;
    if constexpr (MODE == MODE_A8W8) {
        const float* sa = static_cast<const float*>(p.sa) + m0;
        const float* sb = static_cast<const float*>(p.sb) + n0;
        lds_load4(sa, (uint32_t)rows_a * 4u, scl + wave * 256, (uint32_t)(wave * 64 + lane) * 4u);
        lds_load4(sb, (uint32_t)rows_b * 4u, scl + DENSE_BM * 4 + wave * 256, (uint32_t)(wave * 64 + lane) * 4u);
    }

    v16f acc[TN][TM];
    dense_kloop<MODE, WAVES_M, WAVES_N, TM, TN, KTB, NS>(p, m0, n0, 0, p.kbytes / KTB, smem, acc);

    // Epilogue (scales of A8W8 applied in registers; MXFP4 has none left)
    const int mw = m0 + wm * TM * 32, nw = n0 + wn * TN * 32;
    auto row_scale = [&](int j) {
        const int r = wm * TM * 32 + j * 32 + (lane & 31);
        return MODE == MODE_A8W8 ? *reinterpret_cast<const HKQ_LDS float*>(scl + r * 4) : 1.0f;
    };
    auto col_scale4 = [&](int i, int g) {
        const int n = wn * TN * 32 + i * 32 + 8 * g + 4 * khalf;
        if constexpr (MODE == MODE_A8W8) {
            const v4f c = *reinterpret_cast<const HKQ_LDS v4f*>(scl + DENSE_BM * 4 + n * 4);
            return make_float4(c[0], c[1], c[2], c[3]);
        }
        return make_float4(1.f, 1.f, 1.f, 1.f);
    };
    if (p.bias)
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, p.C, p.ldc, p.M, p.N, mw, nw, p.c16 != 0, row_scale, col_scale4,
                                [&](int i, int g) { return bias4(p, nw + i * 32 + 8 * g + 4 * khalf); });
    else
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, p.C, p.ldc, p.M, p.N, mw, nw, p.c16 != 0, row_scale, col_scale4,
                                NoBias{});
}

// Workgroup u < n_whole computes tile u. When the last round of tiles would
// leave at least half of the CUs idle, its tiles are instead computed as M
// halves by twice as many workgroups: unit v = u - n_whole (XCD v & 7, as the
// dispatcher assigns workgroups round-robin) computes half (v >> 3) & 1 of tile
// n_whole + 8 * (v >> 4) + (v & 7), so both halves of a tile run on one XCD.
// Tile ids then go through tile_coords' XCD-aware order.
template <int MODE, int KTB>
__global__ __launch_bounds__(64 * DENSE_WAVES_M * DENSE_WAVES_N, 1) void dense_gemm_kernel(const DenseParams pb) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;
    const DenseParams p = batch_slice(pb);
    const int u = blockIdx.x;
    int whole = -1, t = -1, half = 0;
    if (u < p.n_whole) {
        whole = u;
    } else {
        const int v = u - p.n_whole;
        t = 8 * (v >> 4) + (v & 7);
        half = (v >> 3) & 1;
        if (t >= p.n_split) return;
    }
    int tm, tn;
    if (whole >= 0) {
        tile_coords(whole, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
        dense_block<MODE, DENSE_TM, KTB>(p, tm, tn, 0, smem);
    } else {
        tile_coords(p.n_whole + t, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
        dense_block<MODE, DENSE_TM / 2, KTB>(p, tm, tn, half, smem);
    }
}

// ---------------------------------------------------------------------------
// Persistent streaming kernel (128-byte K-tiles, K-tiles per tile a multiple
// of 8, one 2-D GEMM without bias): workgroup b of G computes whole tiles
// b, b + G, ... < n_whole as one K-tile stream (gemm_stream.h) and, when the
// last round is split, the M half (b >> 3) & 1 of tile n_whole + 8*(b >> 4) +
// (b & 7) (before or after the whole tiles). Epilogues store C from registers
// through a per-wave LDS staging area (DirectEpi). A8W8 row/column scales of
// tile k are prefetched into LDS slot k & 1 when the tile starts.
//
// A half tile (128 x 256) runs on the one-tile K loop with a 3-stage ring:
// per K-tile it moves 48 KB through the LDS for half of a whole tile's MFMAs,
// and its K loop is bound by that traffic; the deeper ring gives the loads
// two K-tiles of lead (measured on MI355X, with the staged epilogue below:
// 4096 x 14336 x 4096 308.8K -> 293.7K cycles per workgroup, 179.4 -> 173.8 us).
constexpr int STREAM_SCL = 2 * DENSE_BM * 4;  // one scale slot: 256 row + 256 column scales
constexpr int HALF_NS = 3;                    // ring stages of a half tile

template <int MODE>
constexpr int stream_ring_lds() {
    using Whole = DenseCfg<MODE, DENSE_WAVES_M, DENSE_WAVES_N, DENSE_TM, DENSE_TN, 128>;
    return 2 * Whole::STAGE + Whole::SB_BYTES;
}
// The staging areas follow the ring and (A8W8) the two scale slots.
template <int MODE>
constexpr int stream_stg_off() { return stream_ring_lds<MODE>() + (MODE == MODE_A8W8 ? 2 * STREAM_SCL : 0); }
template <int MODE>
constexpr int stream_lds() {
    using Half = DenseCfg<MODE, DENSE_WAVES_M, DENSE_WAVES_N, DENSE_TM / 2, DENSE_TN, 128>;
    constexpr int whole = stream_stg_off<MODE>() + DENSE_WAVES_M * DENSE_WAVES_N * STREAM_STG;
    constexpr int half = Half::lds_bytes(HALF_NS) + (MODE == MODE_A8W8 ? 2 * DENSE_BM * 4 : 0);
    return whole > half ? whole : half;
}

// Tile k of the stream: tile id first + k * stride in tile_coords order,
// rows [tm*256 + half*BM, +BM) of it.
template <int BM>
struct DenseSeq {
    static constexpr bool GATHER = false;
    const DenseParams* p;
    int tiles, KT;
    uint32_t lsa, lsb;
    int first, stride, half;
    __device__ void coords(int k, int& m0, int& n0) const {
        int tm, tn;
        tile_coords(first + k * stride, p->tiles_m, p->tiles_n, p->group_m, tm, tn);
        m0 = tm * DENSE_BM + half * BM;
        n0 = tn * DENSE_BN;
    }
    __device__ StreamSrc src(int k) const {
        int m0, n0;
        coords(k, m0, n0);
        const int rows_a = min(p->M - m0, BM), rows_b = min(p->N - n0, DENSE_BN);
        StreamSrc s;
        s.a = p->A + (int64_t)m0 * p->lda;
        s.b = p->B + (int64_t)n0 * p->ldb;
        s.a_bytes = (uint32_t)min((int64_t)rows_a * p->lda, (int64_t)0x7FFFFFFF);
        s.b_bytes = (uint32_t)min((int64_t)rows_b * p->ldb, (int64_t)0x7FFFFFFF);
        s.as = static_cast<const uint8_t*>(p->sa) + (int64_t)m0 * p->lsa;
        s.bs = static_cast<const uint8_t*>(p->sb) + (int64_t)n0 * p->lsb;
        s.as_bytes = (uint32_t)min((int64_t)rows_a * p->lsa, (int64_t)0x7FFFFFFF);
        s.bs_bytes = (uint32_t)min((int64_t)rows_b * p->lsb, (int64_t)0x7FFFFFFF);
        return s;
    }
};

template <int MODE, int TM, int BM>
struct DirectEpi {
    static constexpr int TN = DENSE_TN;
    // vector-memory instructions a wave issues in end() (at least: ragged
    // tiles add 8-byte stores) plus the next begin(); the stream's first
    // barrier after an epilogue leaves that many in flight
    static constexpr int VM_ISSUED = TN * TM * 2 + (MODE == MODE_A8W8 ? 2 : 0);
    const DenseSeq<BM>* seq;
    const DenseParams* p;
    HKQ_LDS uint8_t* scl;  // 2 slots of STREAM_SCL bytes
    HKQ_LDS uint8_t* stg;  // this wave's STREAM_STG bytes of staging
    int lane, wave;
    __device__ void begin(int k) {
        if constexpr (MODE == MODE_A8W8) {
            int m0, n0;
            seq->coords(k, m0, n0);
            const int rows_a = min(p->M - m0, BM), rows_b = min(p->N - n0, DENSE_BN);
            HKQ_LDS uint8_t* slot = scl + (k & 1) * STREAM_SCL;
            const uint32_t off = (uint32_t)(wave * 64 + lane) * 4u;
            lds_load4(static_cast<const float*>(p->sa) + m0, (uint32_t)rows_a * 4u, slot + wave * 256, off);
            lds_load4(static_cast<const float*>(p->sb) + n0, (uint32_t)rows_b * 4u, slot + DENSE_BM * 4 + wave * 256, off);
        }
    }
    // Stores through the wave's staging area (stream_store_tile), with the
    // tile's row and column scales from its LDS slot.
    __device__ void end(int k, v16f (&acc)[TN][TM]) {
        int m0, n0;
        seq->coords(k, m0, n0);
        const int wm = wave / DENSE_WAVES_N, wn = wave % DENSE_WAVES_N;
        const int khalf = lane >> 5, r = lane & 31;
        const HKQ_LDS float* sl = reinterpret_cast<const HKQ_LDS float*>(scl + (k & 1) * STREAM_SCL);
        const int mw0 = m0 + wm * TM * 32, nw0 = n0 + wn * TN * 32;
        float rs[TM];
#pragma unroll
        for (int j = 0; j < TM; ++j) rs[j] = MODE == MODE_A8W8 ? sl[wm * TM * 32 + j * 32 + r] : 1.0f;
        stream_store_tile<TM, TN>(
            acc, stg, p->C + (int64_t)mw0 * p->ldc + nw0, p->ldc, p->M - mw0, p->N - nw0, rs,
            [&](int i, int g) {
                return MODE == MODE_A8W8 ? *reinterpret_cast<const HKQ_LDS v4f*>(sl + DENSE_BM + wn * TN * 32 + i * 32 +
                                                                                 8 * g + 4 * khalf)
                                         : v4f{1.f, 1.f, 1.f, 1.f};
            },
            lane);
    }
};

template <int MODE, int TM>
__device__ __forceinline__ void dense_stream(const DenseParams& p, int tiles, int first, int stride, int half,
                                             HKQ_LDS uint8_t* smem) {
    constexpr int WM = DENSE_WAVES_M, WN = DENSE_WAVES_N, TN = DENSE_TN;
    using Cfg = DenseCfg<MODE, WM, WN, TM, TN, 128>;
    constexpr int BM = Cfg::BM;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    DenseSeq<BM> seq{&p, tiles, p.kbytes / 128, (uint32_t)p.lsa, (uint32_t)p.lsb, first, stride, half};
    DirectEpi<MODE, TM, BM> epi{&seq, &p, smem + stream_ring_lds<MODE>(),
                                smem + stream_stg_off<MODE>() + wave * STREAM_STG, lane, wave};
    auto a_off = dense_offs<Cfg::NW, 128, Cfg::LA>(wave, lane, p.lda);
    const auto b_off = dense_offs<Cfg::NW, 128, Cfg::LB>(wave, lane, p.ldb);
    v16f acc[TN][TM];
    gemm_stream<MODE, WM, WN, TM, TN>(seq, a_off, b_off, smem, lane, wave, acc, epi);
}

template <int MODE>
__global__ __launch_bounds__(64 * DENSE_WAVES_M * DENSE_WAVES_N, 1) void dense_stream_kernel(const DenseParams p) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;
    const int b = blockIdx.x, G = gridDim.x;
    const int mine = b < p.n_whole ? (p.n_whole - 1 - b) / G + 1 : 0;
    const int t = 8 * (b >> 4) + (b & 7);
    // Half of the workgroups (half of each XCD's) take their half tile first:
    // their tile boundaries then fall between the others', so the epilogues'
    // bursts of C stores come in two waves (measured on MI355X: 4096 x 14336
    // x 4096, 190.3 -> 186.9 us)
    const bool half_first = (b >> 4) & 1;
    const bool has_half = t < p.n_split;
    int tm = 0, tn = 0;
    if (has_half) tile_coords(p.n_whole + t, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    if (half_first && has_half) {
        dense_block<MODE, DENSE_TM / 2, 128, HALF_NS>(p, tm, tn, (b >> 3) & 1, smem);
        // the stream's first loads overwrite the half tile's staging: every
        // wave's LDS reads are done first (its C stores may still drain)
        lds_barrier();
    }
    if (mine > 0) dense_stream<MODE, DENSE_TM>(p, mine, b, G, 0, smem);
    if (!half_first && has_half) dense_block<MODE, DENSE_TM / 2, 128, HALF_NS>(p, tm, tn, (b >> 3) & 1, smem);
}

// ---------------------------------------------------------------------------
// Smaller tiles and split K. A grid of 256 x 256 tiles that would fill at most
// half of the CUs runs on 128 x 128 tiles (4 waves of 64 x 64; FP8 with
// M <= 128 and K <= 16384: 128 x 64 tiles, 4 waves of 32 x 64), and M <= 64
// on one row of (32 or 64) x 256 tiles (4 waves side by side); if that still
// fills at most half of the CUs, K is split as well: workgroup u computes tile
// u % tiles over K-tiles [s * kt_split, (s+1) * kt_split), s = u / tiles, and
// writes its fp32 sums to the workspace in register order (per wave, float4 q
// of lane l at (q * 64 + l) * 16 bytes: every store is a contiguous 1 KB).
// Then it counts itself in at the tile's arrival counter; the split that
// arrives last (ticket splits - 1) adds the partials of all splits in split
// order (s = 0, 1, ...: the same fp32 sums whichever split arrives last), runs
// the epilogue and puts the counter back to SPLIT_IDLE. Without a split the
// workgroup runs the epilogue itself.

// The scales of a wave's (TM*32) x (TN*32) block (A8W8: rows past M and
// columns past N read 1; other modes: 1), loaded into registers before the K
// loop so that the epilogue waits on none of them.
template <int MODE, int TM, int TN>
struct EpiScales {
    float r[TM];
    float4 c[TN][4];
    __device__ __forceinline__ void load(const DenseParams& p, int lane, int mw, int nw) {
        const int khalf = lane >> 5;
#pragma unroll
        for (int j = 0; j < TM; ++j) {
            const int m = mw + j * 32 + (lane & 31);
            r[j] = (MODE == MODE_A8W8 && m < p.M) ? static_cast<const float*>(p.sa)[m] : 1.0f;
        }
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = nw + i * 32 + 8 * g + 4 * khalf;
                c[i][g] = (MODE == MODE_A8W8 && n < p.N)
                              ? *reinterpret_cast<const float4*>(static_cast<const float*>(p.sb) + n)
                              : make_float4(1.f, 1.f, 1.f, 1.f);
            }
    }
};

template <int MODE, int WM, int WN, int TM, int TN>
__device__ __forceinline__ void dense_epilogue_global(const DenseParams& p, v16f (&acc)[TN][TM],
                                                      const EpiScales<MODE, TM, TN>& sc, HKQ_LDS uint8_t* smem,
                                                      int wave, int lane, int mw, int nw) {
    const int khalf = lane >> 5;
    auto row_scale = [&](int j) { return sc.r[j]; };
    auto col_scale4 = [&](int i, int g) { return sc.c[i][g]; };
    if (p.bias)
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, p.C, p.ldc, p.M, p.N, mw, nw, p.c16 != 0, row_scale, col_scale4,
                                [&](int i, int g) { return bias4(p, nw + i * 32 + 8 * g + 4 * khalf); });
    else
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, p.C, p.ldc, p.M, p.N, mw, nw, p.c16 != 0, row_scale, col_scale4,
                                NoBias{});
}

// Split partials cross XCDs, whose L2s are not coherent with each other: they
// are written and read with device-scope cache policy (sc1: the store writes
// through to the coherent level, the load does not hit a line another XCD may
// have changed), so no whole-L2 write-back or invalidate is needed; a wave's
// stores are complete (vmcnt 0) before its workgroup counts in.
constexpr int CPOL_SC1 = 16;

// Arrival counters of split tiles: bits 63..16 hold the SPLIT_MAGIC mark,
// 15..0 the number of splits counted in. An idle counter is SPLIT_MAGIC << 16
// (count 0), and the last split of a call leaves it so; one arrival then costs
// a single fetch-and-add. A counter without the mark (a workspace never used
// for a split plan, or memory another tensor held) is claimed by compare-and-
// swap: the arrival whose swap installs a count of 1 is counted by it, every
// other arrival that found the counter unmarked counts itself in again once it
// sees the mark. Exactly `splits` arrivals are counted, so exactly one draws
// the last ticket.
constexpr uint64_t SPLIT_MAGIC = 0x686B71535054ull;  // 48 bits
constexpr uint64_t SPLIT_IDLE = SPLIT_MAGIC << 16;
// Counters sit at the start of the split workspace, one per tile, for at most
// SPLIT_MAX_TILES tiles (every plan uses the same ones, so partial sums of
// another plan never overwrite them); the partial sums follow.
constexpr int SPLIT_MAX_TILES = 512;
constexpr size_t SPLIT_CNT_BYTES = SPLIT_MAX_TILES * 8;

__device__ __forceinline__ int split_ticket(uint64_t* cnt, int splits) {
    auto fresh = [&](uint64_t v) { return (v >> 16) == SPLIT_MAGIC && (int)(v & 0xFFFF) < splits; };
    const uint64_t old = __hip_atomic_fetch_add(cnt, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (fresh(old)) return (int)(old & 0xFFFF);
    uint64_t cur = old + 1;
    for (;;) {  // ends: a swap fails only when another arrival changed the counter
        if (__hip_atomic_compare_exchange_strong(cnt, &cur, SPLIT_IDLE | 1ull, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT))
            return 0;
        if (fresh(cur)) {  // claimed by another arrival: this one's increment was dropped with the old value
            const uint64_t o = __hip_atomic_fetch_add(cnt, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return (int)(o & 0xFFFF);
        }
    }
}

template <int MODE, int WM, int WN, int TM, int TN, int KTB, int MINB, int NS>
__global__ __launch_bounds__(64 * WM * WN, MINB) void dense_tile_kernel(const DenseParams pb) {
    using Cfg = DenseCfg<MODE, WM, WN, TM, TN, KTB>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, NW = Cfg::NW;
    constexpr int NQ = TN * TM * 4;  // float4 of accumulators per lane
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;
    const DenseParams p = batch_slice(pb);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tiles = p.tiles_m * p.tiles_n;
    const int tile = blockIdx.x % tiles, split = blockIdx.x / tiles;
    int tm, tn;
    tile_coords(tile, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KT = p.kbytes / KTB;
    const int kt0 = split * p.kt_split, kt1 = min(KT, kt0 + p.kt_split);
    const int wm = wave / WN, wn = wave % WN;
    const int mw = m0 + wm * TM * 32, nw = n0 + wn * TN * 32;

    // older than the K-tile loads: the loop's vmcnt waits cover them
    EpiScales<MODE, TM, TN> sc;
    sc.load(p, lane, mw, nw);

    v16f acc[TN][TM];
    dense_kloop<MODE, WM, WN, TM, TN, KTB, NS>(p, m0, n0, kt0, kt1, smem, acc);

    if (p.splits == 1) {
        dense_epilogue_global<MODE, WM, WN, TM, TN>(p, acc, sc, smem, wave, lane, mw, nw);
        return;
    }
    // this split's partial: float4 q of lane l of wave w at
    // ((s * tiles + tile) * NW + w) * NQ * 64 + q * 64 + l
    const uint32_t wave_slot = (uint32_t)(((int64_t)tile * NW + wave) * NQ * 64 + lane) * 16u;
    const uint32_t split_stride = (uint32_t)tiles * NW * NQ * 64 * 16u;
    const __amdgpu_buffer_rsrc_t ws =
        __builtin_amdgcn_make_buffer_rsrc(p.ws, 0, (int)(split_stride * (uint32_t)p.splits), 0x00020000);
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const v4f v = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, v), ws,
                                                       (uint32_t)split * split_stride + wave_slot +
                                                           (uint32_t)(((i * TM + j) * 4 + g) * 64 * 16),
                                                       0, CPOL_SC1);
            }
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
    // count this split in (one thread per workgroup); the flag lies past the
    // epilogue's staging, in the (idle) K-tile ring
    static_assert(Cfg::EP_BYTES + 16 <= Cfg::lds_bytes(NS), "room for the split flag");
    HKQ_LDS int& last_split = *reinterpret_cast<HKQ_LDS int*>(smem + Cfg::lds_bytes(NS) - 16);
    __syncthreads();
    if (threadIdx.x == 0) {
        const bool last = split_ticket(p.split_cnt + tile, p.splits) == p.splits - 1;
        if (last) __hip_atomic_store(p.split_cnt + tile, SPLIT_IDLE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_split = last;
    }
    __syncthreads();
    if (!last_split) return;
    // sum in split order; the other splits' float4 come in chunks of RCH
    // splits, all loads of a chunk in flight together (three splits' worth of
    // registers where the budget allows: 8 float4 per lane, or one workgroup
    // per CU)
    constexpr int RCH = (NQ <= 8 || MINB == 1) ? 3 : 1;
    v16f sum[TN][TM];
    for (int s0 = 0; s0 < p.splits; s0 += RCH) {
        v4f part[RCH][NQ] = {};
#pragma unroll
        for (int c = 0; c < RCH; ++c) {
            const int s = s0 + c;
            if (s < p.splits && s != split) {
#pragma unroll
                for (int q = 0; q < NQ; ++q)
                    part[c][q] = __builtin_bit_cast(
                        v4f, __builtin_amdgcn_raw_buffer_load_b128(ws, (uint32_t)s * split_stride + wave_slot +
                                                                           (uint32_t)(q * 64 * 16),
                                                                   0, CPOL_SC1));
            }
        }
#pragma unroll
        for (int c = 0; c < RCH; ++c) {
            const int s = s0 + c;
            if (s >= p.splits) break;
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int q = (i * TM + j) * 4 + g;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float x = s == split ? acc[i][j][4 * g + e] : part[c][q][e];
                            sum[i][j][4 * g + e] = s == 0 ? x : sum[i][j][4 * g + e] + x;
                        }
                    }
        }
    }
    dense_epilogue_global<MODE, WM, WN, TM, TN>(p, sum, sc, smem, wave, lane, mw, nw);
}

// ---------------------------------------------------------------------------
// Narrow M (M <= 32, FP8 and FP4): a streaming path on the 16x16x128 MFMA.
// Workgroup u owns the 16*NT columns [16*NT*u, 16*NT*(u+1)) of C for all M
// rows; its 4 waves split K (wave w takes the 128-value K-steps
// [w*S/4, (w+1)*S/4) of S) and load their operand fragments from memory
// straight into registers, DEPTH steps ahead. The waves' sums meet in LDS, and
// wave 0 adds them in wave order, applies the scales and writes C. Each weight
// byte is read once, by one workgroup, in a single launch (no split-K
// partials, no second kernel). NT > 1 reuses each activation fragment for NT
// weight tiles when N gives more workgroups than CUs.
//
// Fragment layout of the 16x16x128 MFMA (verified on gfx950): lane l supplies
// row l % 16 and the 32 K-values [32*(l/16), 32*(l/16) + 32) of the 128-deep
// slice (FP8: 32 bytes; FP4: 16 bytes in the low 4 VGPRs, scaled per lane by
// its 32-value block's e8m0); lane l, register i of the result holds
// D[4*(l/16) + i][l % 16]. The MFMA A operand is the weight rows (n), B the
// activation rows (m): a lane holds 4 consecutive n of one m. An FP8 sum over
// K does not depend on which lane supplies which K-value as long as both
// operands agree, so an FP8 lane takes bytes [16q, 16q+16) and [64+16q,
// 64+16q+16) of the step (q = l/16): each 16-byte load covers 64 contiguous
// bytes of 16 rows.
constexpr int NARROW_WAVES = 4, NARROW_MAX_M = 32;

template <int MODE, int MT, int NT>
struct NarrowFrag {
    v4i b0[NT], b1[NT];  // weight rows (b1: FP8 only)
    v4i a0[MT], a1[MT];  // activation rows (a1: FP8 only)
    uint32_t sb[NT], sa[MT];  // FP4: e8m0 scales of the step's 4 blocks (byte q is the lane's)
};

// K-steps of loads in flight per wave (measured on MI355X: FP8 with two
// column tiles per workgroup 8 rather than 6, 1x6144x4096 8.33 -> 7.94 us;
// deeper rings for one or four column tiles, and for FP4, were slower)
template <int MODE, int MT, int NT>
constexpr int narrow_depth() { return NT >= 4 ? 4 : NT == 2 ? (MODE == MODE_MXFP4 ? 6 : 8) : 8; }

template <int MODE, int MT, int NT>
__global__ __launch_bounds__(64 * NARROW_WAVES) void narrow_gemm_kernel(const DenseParams pb) {
    constexpr bool FP4 = MODE == MODE_MXFP4;
    constexpr int SB = FP4 ? 64 : 128;  // bytes of a row per 128-value K-step
    constexpr int DEPTH = narrow_depth<MODE, MT, NT>();
    __shared__ v4f red[NARROW_WAVES][NT][MT][64];
    const DenseParams p = batch_slice(pb);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * 16 * NT;
    const int S = p.kbytes / SB;
    const int s0 = wave * S / NARROW_WAVES, s1 = (wave + 1) * S / NARROW_WAVES;
    const int rows_b = min(16 * NT, p.N - n0);
    const auto rb = make_rsrc(p.B + (int64_t)n0 * p.ldb, (uint32_t)(rows_b * p.ldb));
    const auto ra = make_rsrc(p.A, (uint32_t)(p.M * p.lda));
    const uint8_t* bs = static_cast<const uint8_t*>(p.sb);
    const auto rsb = make_rsrc(FP4 ? bs + (int64_t)n0 * p.lsb : p.B, FP4 ? (uint32_t)(rows_b * p.lsb) : 0u);
    const auto rsa = make_rsrc(FP4 ? p.sa : p.A, FP4 ? (uint32_t)(p.M * p.lsa) : 0u);
    uint32_t b_off[NT], a_off[MT];
#pragma unroll
    for (int t = 0; t < NT; ++t) b_off[t] = (uint32_t)((t * 16 + r) * p.ldb + 16 * q);
#pragma unroll
    for (int t = 0; t < MT; ++t) a_off[t] = (uint32_t)((t * 16 + r) * p.lda + 16 * q);

    // Steps at or past s1 read zeros (their MFMAs add nothing): offsets with
    // the OOB bit set are past every buffer's range.
    auto load = [&](int s, NarrowFrag<MODE, MT, NT>& f) {
        const uint32_t kb = (uint32_t)s * SB | (s < s1 ? 0u : OOB);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            f.b0[t] = __builtin_amdgcn_raw_buffer_load_b128(rb, b_off[t] + kb, 0, 0);
            if constexpr (!FP4) f.b1[t] = __builtin_amdgcn_raw_buffer_load_b128(rb, b_off[t] + kb + 64, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            f.a0[t] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[t] + kb, 0, 0);
            if constexpr (!FP4) f.a1[t] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[t] + kb + 64, 0, 0);
        }
        if constexpr (FP4) {
            const uint32_t ks = 4 * (uint32_t)s | (s < s1 ? 0u : OOB);
#pragma unroll
            for (int t = 0; t < NT; ++t)
                f.sb[t] = __builtin_amdgcn_raw_buffer_load_b32(rsb, (uint32_t)((t * 16 + r) * p.lsb) + ks, 0, 0);
#pragma unroll
            for (int t = 0; t < MT; ++t)
                f.sa[t] = __builtin_amdgcn_raw_buffer_load_b32(rsa, (uint32_t)((t * 16 + r) * p.lsa) + ks, 0, 0);
        }
    };
    v4f acc[NT][MT];
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[i][t] = v4f{0.f, 0.f, 0.f, 0.f};
    auto mma = [&](const NarrowFrag<MODE, MT, NT>& f) {
#pragma unroll
        for (int i = 0; i < NT; ++i)
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                if constexpr (FP4) {
                    const v8i a = v8i{f.b0[i][0], f.b0[i][1], f.b0[i][2], f.b0[i][3], 0, 0, 0, 0};
                    const v8i b = v8i{f.a0[t][0], f.a0[t][1], f.a0[t][2], f.a0[t][3], 0, 0, 0, 0};
                    acc[i][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        a, b, acc[i][t], 4, 4, 0, (int)(f.sb[i] >> (8 * q)), 0, (int)(f.sa[t] >> (8 * q)));
                } else {
                    const v8i a = v8i{f.b0[i][0], f.b0[i][1], f.b0[i][2], f.b0[i][3],
                                      f.b1[i][0], f.b1[i][1], f.b1[i][2], f.b1[i][3]};
                    const v8i b = v8i{f.a0[t][0], f.a0[t][1], f.a0[t][2], f.a0[t][3],
                                      f.a1[t][0], f.a1[t][1], f.a1[t][2], f.a1[t][3]};
                    acc[i][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[i][t], 0, 0, 0, 127, 0, 127);
                }
            }
    };
    NarrowFrag<MODE, MT, NT> f[DEPTH];
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
    const float* sa = static_cast<const float*>(p.sa);
    const float* sb = static_cast<const float*>(p.sb);
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int n = n0 + 16 * i + 4 * q;
        if (n >= p.N) break;  // N % 4 == 0: n .. n+3 all in or all out
        float4 cs = make_float4(1.f, 1.f, 1.f, 1.f);
        if constexpr (MODE == MODE_A8W8) cs = *reinterpret_cast<const float4*>(sb + n);
        const float4 c = bias4(p, n);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int m = t * 16 + r;
            if (m >= p.M) break;
            v4f v = red[0][i][t][lane];
#pragma unroll
            for (int w = 1; w < NARROW_WAVES; ++w) v += red[w][i][t][lane];
            const float a = MODE == MODE_A8W8 ? sa[m] : 1.f;
            *reinterpret_cast<v2i*>(p.C + (int64_t)m * p.ldc + n) =
                v2i{(int)pk_bf16(v[0] * a * cs.x + c.x, v[1] * a * cs.y + c.y),
                    (int)pk_bf16(v[2] * a * cs.z + c.z, v[3] * a * cs.w + c.w)};
        }
    }
}

template <typename K>
static int set_lds(K kern, int lds, bool& done) {
    if (done) return 0;
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) {
        set_error("hipFuncSetAttribute(MaxDynamicSharedMemorySize=%d) failed: %s", lds, hipGetErrorString(e));
        return (int)e;
    }
    done = true;
    return 0;
}

// Plan of a dense GEMM: the tile geometry, how many K splits, and the
// workspace the splits need (bytes). The same function answers the workspace
// query, so a caller's workspace always matches the launch.
enum DenseGeo { GEO_256 = 0, GEO_128 = 1, GEO_SKINNY = 2, GEO_128x64 = 3 };
struct DensePlan {
    int geo;
    int skinny_tm;  // GEO_SKINNY: TM = 1 or 2
    int64_t tiles;
    int splits, kt_split;
    size_t ws_bytes;
};

static DensePlan dense_plan(int mode, int64_t M, int64_t N, int64_t kbytes, bool allow_split, int64_t batch = 1) {
    DensePlan pl{};
    const int ktb = kbytes % 128 == 0 ? 128 : 64;
    const int64_t KT = kbytes / ktb;
    const int ncu = cu_count() > 0 ? cu_count() : 256;
    // tiles of the whole launch (all batches)
    auto ntiles = [&](int64_t bm, int64_t bn) { return batch * ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    int64_t bm = DENSE_BM, bn = DENSE_BN;
    pl.geo = GEO_256;
    if (ktb == 128 && M <= 64) {
        pl.geo = GEO_SKINNY;
        pl.skinny_tm = M <= 32 ? 1 : 2;
        bm = 32 * pl.skinny_tm;
        bn = SKINNY_BN;
    } else if (ktb == 128 && 2 * ntiles(DENSE_BM, DENSE_BN) <= ncu) {
        pl.geo = GEO_128;
        bm = bn = 128;
        // FP8 with M <= 128 and K <= 16384: 128 x 64 tiles (4 waves of 32 x 64),
        // twice the workgroups for the same K split and a quarter of the
        // partial sums the last split reads (measured on MI355X: 128x4096x4096
        // 10.0 us, 128x4096x14336 18.0 us against 24.1 on 128 x 128 tiles)
        if (mode == MODE_A8W8 && M <= 128 && KT <= 128) {
            pl.geo = GEO_128x64;
            bn = 64;
        }
    }
    pl.tiles = ntiles(bm, bn);
    pl.splits = 1;
    pl.kt_split = (int)KT;
    // split K when the tiles fill at most half of the CUs, keeping at least 4
    // K-tiles per split
    if (allow_split && pl.geo != GEO_256 && pl.tiles > 0 && 2 * pl.tiles <= ncu && pl.tiles <= SPLIT_MAX_TILES &&
        KT >= 8) {
        int64_t s = (ncu + pl.tiles - 1) / pl.tiles;
        s = std::min<int64_t>(s, KT / 4);
        if (s > 1) {
            const int64_t per = (KT + s - 1) / s;
            pl.splits = (int)((KT + per - 1) / per);
            pl.kt_split = (int)per;
        }
    }
    // the arrival counters, then the partial sums
    if (pl.splits > 1) pl.ws_bytes = SPLIT_CNT_BYTES + (size_t)pl.splits * (size_t)pl.tiles * (size_t)(bm * bn) * 4;
    return pl;
}

template <int MODE, int WM, int WN, int TM, int TN, int KTB, int MINB, int NS = dense_ns<KTB>()>
static int launch_dense_tiles(DenseParams& p, const DensePlan& pl, hipStream_t stream) {
    using Cfg = DenseCfg<MODE, WM, WN, TM, TN, KTB>;
    constexpr int LDS = Cfg::lds_bytes(NS);
    static_assert(LDS * MINB <= 160 * 1024, "LDS budget of a CDNA4 CU");
    auto kern = dense_tile_kernel<MODE, WM, WN, TM, TN, KTB, MINB, NS>;
    static bool attr_set = false;
    if (int e = set_lds(kern, LDS, attr_set)) return e;
    p.tiles_m = (p.M + Cfg::BM - 1) / Cfg::BM;
    p.tiles_n = (p.N + Cfg::BN - 1) / Cfg::BN;
    if (p.group_m <= 0) p.group_m = 8;
    p.splits = pl.splits;
    p.kt_split = pl.kt_split;
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    if (tiles == 0) return 0;
    if (p.splits > 1) {  // dense_plan's workspace: the arrival counters, then the partial sums
        p.split_cnt = reinterpret_cast<uint64_t*>(p.ws);
        p.ws = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(p.ws) + SPLIT_CNT_BYTES);
    }
    kern<<<dim3((unsigned)(tiles * p.splits), (unsigned)std::max(1, p.batch)), 64 * WM * WN, LDS, stream>>>(p);
    return hkq_launch_status();
}

template <int MODE, int KTB>
static int launch_dense_whole(DenseParams& p, hipStream_t stream) {
    constexpr int LDS = dense_lds<MODE, KTB>();
    static_assert(LDS <= 160 * 1024, "LDS budget of a CDNA4 CU");
    auto kern = dense_gemm_kernel<MODE, KTB>;
    static bool attr_set = false;  // per instantiation; the attribute is per-process
    if (int e = set_lds(kern, LDS, attr_set)) return e;
    p.tiles_m = (p.M + DENSE_BM - 1) / DENSE_BM;
    p.tiles_n = (p.N + DENSE_BN - 1) / DENSE_BN;
    // tile rows per group of the walk (measured best: 8 for FP8, 4 for FP4)
    if (p.group_m <= 0) p.group_m = MODE == MODE_MXFP4 ? 4 : 8;
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    if (tiles == 0) return 0;
    // Split the last round into M halves when it would fill at most half of the
    // CUs and the tiles have rows in both halves.
    const int ncu = cu_count();
    const int64_t last = ncu > 0 ? tiles % ncu : 0;
    const bool batched = p.batch > 1;  // a batch fills the GPU by itself: no half tiles
    const int64_t split = (!batched && last > 0 && 2 * last <= ncu && p.M > DENSE_BM / 2) ? last : 0;
    p.n_whole = (int)(tiles - split);
    p.n_split = (int)split;
    // MXFP4 stays on the one-tile kernel: its stream (the K loop below with
    // compile-time scale slots, C stored from registers since the ring and the
    // scale blocks fill the LDS) spills and measured 1.8x slower on MI355X.
    if constexpr (KTB == 128 && MODE != MODE_MXFP4) {
        // the persistent streaming kernel: one workgroup per CU, whole tiles as
        // a K-tile stream (needs K-tiles per tile % 8 == 0; one 2-D GEMM without
        // bias, C's rows 16-byte aligned); HKQ_DENSE_STREAM=0 selects the
        // one-tile-per-workgroup kernel
        static const bool stream_on = [] {
            const char* e = std::getenv("HKQ_DENSE_STREAM");
            return !(e && e[0] == '0');
        }();
        // Measured on MI355X against the one-tile-per-workgroup kernel: 1-3%
        // faster at 1.75-3.5 rounds of tiles, 1-2% at 7 and 14 rounds
        // (4096x28672, 8192x14336 and 8192x28672, K = 4096).
        // Half tile t belongs to workgroup b with t = 8 * (b >> 4) + (b & 7), so
        // the split needs 2 * roundup8(split) workgroups: grids that cannot hold
        // them within one per CU take the one-tile kernel.
        const int64_t g = std::min<int64_t>(ncu, std::max<int64_t>(p.n_whole, 2 * ((split + 7) / 8 * 8)));
        if (stream_on && ncu > 0 && !batched && p.bias == nullptr && (p.kbytes / 128) % 8 == 0 && p.c16 &&
            2 * ((split + 7) / 8 * 8) <= g) {
            constexpr int SLDS = stream_lds<MODE>();
            static_assert(SLDS <= 160 * 1024, "LDS budget of a CDNA4 CU");
            auto skern = dense_stream_kernel<MODE>;
            static bool sattr = false;
            if (int e = set_lds(skern, SLDS, sattr)) return e;
            skern<<<dim3((unsigned)g), 64 * DENSE_WAVES_M * DENSE_WAVES_N, SLDS, stream>>>(p);
            return hkq_launch_status();
        }
    }
    const int64_t nblk = p.n_whole + 2 * ((split + 7) / 8 * 8);
    kern<<<dim3((unsigned)nblk, (unsigned)std::max(1, p.batch)), 64 * DENSE_WAVES_M * DENSE_WAVES_N, LDS, stream>>>(p);
    return hkq_launch_status();
}

// The narrow path serves the FP8 and FP4 GEMMs whose rows hold whole 128-value
// K-steps: all of M <= 16, and M <= 32 while the 16-column workgroups number
// fewer than two per CU and K is at most 32 steps (beyond that, every
// workgroup re-reading the activation rows costs more than the tiled path's
// LDS-shared activation tile; measured on MI355X). Its buffer offsets are
// 32-bit: 16*NT weight rows and 32 activation rows must span less than 2 GiB.
static bool use_narrow(int mode, int64_t M, int64_t N, int64_t kbytes, int64_t lda, int64_t ldb, int64_t batch) {
    if (mode != MODE_A8W8 && mode != MODE_MXFP4) return false;
    const int64_t step = mode == MODE_MXFP4 ? 64 : 128;
    if (M < 1 || M > NARROW_MAX_M || kbytes % step != 0 || 64 * ldb >= (1ll << 31) || NARROW_MAX_M * lda >= (1ll << 31))
        return false;
    if (M <= 16) return true;
    const int64_t ncu = cu_count() > 0 ? cu_count() : 256;
    return std::max<int64_t>(1, batch) * ((N + 15) / 16) < 2 * ncu && kbytes / step <= 32;
}

template <int MODE, int MT, int NT>
static int launch_narrow_nt(const DenseParams& p, hipStream_t stream) {
    const dim3 grid((unsigned)((p.N + 16 * NT - 1) / (16 * NT)), (unsigned)std::max(1, p.batch));
    narrow_gemm_kernel<MODE, MT, NT><<<grid, 64 * NARROW_WAVES, 0, stream>>>(p);
    return hkq_launch_status();
}

// Columns per workgroup: 16 * NT. One round of 16-column workgroups: NT = 1;
// up to three rounds: NT = 2 (one round, activation fragments used twice);
// more: NT = 4 (measured on MI355X at N = 4096 .. 28672).
template <int MODE>
static int launch_narrow(const DenseParams& p, hipStream_t stream) {
    if constexpr (MODE == MODE_A8W8 || MODE == MODE_MXFP4) {
        if (p.N == 0) return 0;
        const int64_t ncu = cu_count() > 0 ? cu_count() : 256;
        const int64_t wgs16 = (int64_t)std::max(1, p.batch) * ((p.N + 15) / 16);
        const int nt = wgs16 <= ncu ? 1 : wgs16 <= 3 * ncu ? 2 : 4;
        if (p.M <= 16) {
            if (nt == 4) return launch_narrow_nt<MODE, 1, 4>(p, stream);
            if (nt == 2) return launch_narrow_nt<MODE, 1, 2>(p, stream);
            return launch_narrow_nt<MODE, 1, 1>(p, stream);
        }
        if (nt == 4) return launch_narrow_nt<MODE, 2, 4>(p, stream);
        if (nt == 2) return launch_narrow_nt<MODE, 2, 2>(p, stream);
        return launch_narrow_nt<MODE, 2, 1>(p, stream);
    }
    return 0;
}

// 128-byte K-tiles need whole 128-byte K-tiles in every row: a partial last
// K-tile would read the next row's bytes instead of zeros.
template <int MODE, int KTB>
static int launch_dense_ktb(DenseParams& p, void* ws, size_t ws_bytes, hipStream_t stream) {
    if (use_narrow(MODE, p.M, p.N, p.kbytes, p.lda, p.ldb, p.batch)) return launch_narrow<MODE>(p, stream);
    p.c16 = (p.ldc % 8 == 0) && (reinterpret_cast<uintptr_t>(p.C) % 16 == 0);
    // batches and bias run unsplit (the split partials and their reduction are per 2-D GEMM)
    const bool plain = p.batch <= 1 && p.bias == nullptr;
    DensePlan pl = dense_plan(MODE, p.M, p.N, p.kbytes, plain, std::max(1, p.batch));
    if (pl.splits > 1 && (ws == nullptr || ws_bytes < pl.ws_bytes))
        pl = dense_plan(MODE, p.M, p.N, p.kbytes, false, std::max(1, p.batch));
    p.ws = static_cast<float*>(ws);
    if constexpr (KTB == 128) {  // smaller tiles need a full 16-byte load per lane for their A rows
        if (pl.geo == GEO_SKINNY) {
            if (pl.skinny_tm == 1) return launch_dense_tiles<MODE, 1, SKINNY_WAVES_N, 1, SKINNY_TN, KTB, 1>(p, pl, stream);
            return launch_dense_tiles<MODE, 1, SKINNY_WAVES_N, 2, SKINNY_TN, KTB, 1>(p, pl, stream);
        }
        // Grids of at most one workgroup per CU run one workgroup each with a
        // 3-stage ring (two K-tiles of loads in flight) rather than two per CU
        // with 2-stage rings (measured on MI355X: 128 x 128 tiles at
        // 1024x4096x4096 25.8 -> 21.2 us, 1024x4096x14336 75.1 -> 58.1,
        // 512x4096x4096 21.4 -> 15.8; 128 x 64 tiles at 128x4096x4096 12.7 ->
        // 11.3, 128x6144x4096 13.3 -> 11.4; at 1.5 rounds, 1024x6144x4096,
        // two per CU win: 29.6 vs 36.5). MXFP4's scale blocks assume 2 stages.
        const int ncu = cu_count() > 0 ? cu_count() : 256;
        const bool one_round = pl.tiles * pl.splits * std::max(1, p.batch) <= ncu;
        if (pl.geo == GEO_128) {
            if (one_round) {
                if constexpr (MODE == MODE_MXFP4) {  // the scale blocks keep 2 stages
                    return launch_dense_tiles<MODE, 2, 2, 2, 2, KTB, 1, 2>(p, pl, stream);
                } else {
                    if (pl.kt_split >= 4) return launch_dense_tiles<MODE, 2, 2, 2, 2, KTB, 1, 4>(p, pl, stream);
                    return launch_dense_tiles<MODE, 2, 2, 2, 2, KTB, 1, 3>(p, pl, stream);
                }
            }
            return launch_dense_tiles<MODE, 2, 2, 2, 2, KTB, 2>(p, pl, stream);
        }
        if constexpr (MODE == MODE_A8W8)
            if (pl.geo == GEO_128x64) {
                if (one_round) {
                    if (pl.kt_split >= 6) return launch_dense_tiles<MODE, 4, 1, 1, 2, KTB, 1, 6>(p, pl, stream);
                    return launch_dense_tiles<MODE, 4, 1, 1, 2, KTB, 1, 3>(p, pl, stream);
                }
                return launch_dense_tiles<MODE, 4, 1, 1, 2, KTB, 2>(p, pl, stream);
            }
    }
    return launch_dense_whole<MODE, KTB>(p, stream);
}

template <int MODE>
static int launch_dense(DenseParams& p, void* ws, size_t ws_bytes, hipStream_t stream) {
    return p.kbytes % 128 == 0 ? launch_dense_ktb<MODE, 128>(p, ws, ws_bytes, stream)
                               : launch_dense_ktb<MODE, 64>(p, ws, ws_bytes, stream);
}

}  // namespace hkq

using namespace hkq;

static int check_common(int64_t M, int64_t N, int64_t K, int64_t ldc, const void* C) {
    HKQ_CHECK_ARG(M >= 0 && N >= 0 && K > 0, "M, N must be >= 0 and K > 0");
    HKQ_CHECK_ARG(M < (1 << 30) && N < (1 << 30) && K < (1 << 30), "dimensions must be < 2^30");
    HKQ_CHECK_ARG(N % 4 == 0, "N must be a multiple of 4");
    HKQ_CHECK_ARG(ldc >= N && ldc % 4 == 0, "ldc must be >= N and a multiple of 4");
    HKQ_CHECK_ALIGN(C, 8);
    return 0;
}

extern "C" {

size_t hkq_gemm_a8w8_workspace(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 64 != 0 || use_narrow(MODE_A8W8, M, N, K, K, K, 1)) return 0;
    return dense_plan(MODE_A8W8, M, N, K, true).ws_bytes;
}

int hkq_gemm_a8w8_ws(const void* A, const void* B, const float* sa, const float* sb, void* C, int64_t M, int64_t N,
                     int64_t K, int64_t lda, int64_t ldb, int64_t ldc, void* workspace, size_t workspace_bytes,
                     hipStream_t stream) {
    if (int e = check_common(M, N, K, ldc, C)) return e;
    HKQ_CHECK_ARG(K % 64 == 0, "K must be a multiple of 64");
    HKQ_CHECK_ARG(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0,
                  "lda/ldb must be >= K and multiples of 16");
    HKQ_CHECK_ALIGN(A, 16);
    HKQ_CHECK_ALIGN(B, 16);
    HKQ_CHECK_ALIGN(sb, 16);
    HKQ_CHECK_ALIGN(workspace, 16);
    DenseParams p{};
    p.A = static_cast<const uint8_t*>(A);
    p.B = static_cast<const uint8_t*>(B);
    p.C = static_cast<uint16_t*>(C);
    p.sa = sa;
    p.sb = sb;
    p.M = (int)M; p.N = (int)N; p.K = (int)K; p.kbytes = (int)K;
    p.lda = lda; p.ldb = ldb; p.ldc = ldc;
    return launch_dense<MODE_A8W8>(p, workspace, workspace_bytes, stream);
}

int hkq_gemm_a8w8(const void* A, const void* B, const float* sa, const float* sb, void* C, int64_t M, int64_t N,
                  int64_t K, int64_t lda, int64_t ldb, int64_t ldc, hipStream_t stream) {
    return hkq_gemm_a8w8_ws(A, B, sa, sb, C, M, N, K, lda, ldb, ldc, nullptr, 0, stream);
}

}  // extern "C"

// Split-K counters and partial sums of hkq_gemm_a8w8_noalloc: a library-owned
// workspace that each GPU holds from the library's load to the end of the
// process, so that the entry point allocates nothing. Its size bounds every
// split plan on 256 CUs (at most 1.5 * 256 tile splits of 128 x 128 fp32
// sums: 25.2 MB, after 4 KB of counters).
constexpr size_t HKQ_SCRATCH_BYTES = size_t(32) << 20;
static __device__ __align__(256) uint8_t scratch[HKQ_SCRATCH_BYTES];

// Device address of `scratch` on the current device, looked up once per device
// with that device current (the host-side name is only a stand-in for it).
static int scratch_address(void** out) {
    constexpr int MAXDEV = 64;
    static void* addr[MAXDEV] = {};
    static std::mutex mu;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= MAXDEV) {
        set_error("hkq_gemm_a8w8_noalloc: no usable current device (%s)", hipGetErrorString(e));
        return e != hipSuccess ? (int)e : (int)hipErrorInvalidDevice;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            set_error("hkq_gemm_a8w8_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
            return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
        }
        addr[dev] = p;
    }
    *out = addr[dev];
    return 0;
}

extern "C" {

size_t hkq_gemm_a8w8_noalloc_max_workspace(void) { return HKQ_SCRATCH_BYTES; }

int hkq_gemm_a8w8_noalloc(const void* A, const void* B, const float* sa, const float* sb, void* C, int64_t M,
                          int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc, hipStream_t stream) {
    // the same argument checks and plan as hkq_gemm_a8w8_ws, whose launches run
    // unchanged on the library's scratch workspace
    const size_t need = hkq_gemm_a8w8_workspace(M, N, K);
    if (need > HKQ_SCRATCH_BYTES) {
        set_error("hkq_gemm_a8w8_noalloc: the split plan of %lldx%lldx%lld needs %zu workspace bytes, more than the "
                  "%zu-byte library scratch; use hkq_gemm_a8w8_ws with a caller workspace",
                  (long long)M, (long long)N, (long long)K, need, HKQ_SCRATCH_BYTES);
        return (int)hipErrorInvalidValue;
    }
    void* ws = nullptr;
    if (need > 0)
        if (int e = scratch_address(&ws)) return e;
    return hkq_gemm_a8w8_ws(A, B, sa, sb, C, M, N, K, lda, ldb, ldc, ws, need, stream);
}

size_t hkq_gemm_mxfp4_workspace(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 128 != 0 || use_narrow(MODE_MXFP4, M, N, K / 2, K / 2, K / 2, 1)) return 0;
    return dense_plan(MODE_MXFP4, M, N, K / 2, true).ws_bytes;
}

int hkq_gemm_mxfp4_ws(const void* A, const void* As, const void* B, const void* Bs, void* C, int64_t M, int64_t N,
                      int64_t K, int64_t lda, int64_t ldb, int64_t ldsa, int64_t ldsb, int64_t ldc, void* workspace,
                      size_t workspace_bytes, hipStream_t stream) {
    if (int e = check_common(M, N, K, ldc, C)) return e;
    HKQ_CHECK_ARG(K % 128 == 0, "K must be a multiple of 128");
    HKQ_CHECK_ARG(lda >= K / 2 && ldb >= K / 2 && lda % 16 == 0 && ldb % 16 == 0,
                  "lda/ldb (bytes) must be >= K/2 and multiples of 16");
    HKQ_CHECK_ARG(ldsa >= K / 32 && ldsb >= K / 32 && ldsa % 4 == 0 && ldsb % 4 == 0,
                  "scale row strides must be >= K/32 and multiples of 4");
    HKQ_CHECK_ALIGN(A, 16);
    HKQ_CHECK_ALIGN(B, 16);
    HKQ_CHECK_ALIGN(As, 4);
    HKQ_CHECK_ALIGN(Bs, 4);
    HKQ_CHECK_ALIGN(workspace, 16);
    DenseParams p{};
    p.A = static_cast<const uint8_t*>(A);
    p.B = static_cast<const uint8_t*>(B);
    p.C = static_cast<uint16_t*>(C);
    p.sa = As;
    p.sb = Bs;
    p.M = (int)M; p.N = (int)N; p.K = (int)K; p.kbytes = (int)(K / 2);
    p.lda = lda; p.ldb = ldb; p.ldc = ldc;
    p.lsa = ldsa; p.lsb = ldsb;
    return launch_dense<MODE_MXFP4>(p, workspace, workspace_bytes, stream);
}

int hkq_gemm_mxfp4(const void* A, const void* As, const void* B, const void* Bs, void* C, int64_t M, int64_t N,
                   int64_t K, int64_t lda, int64_t ldb, int64_t ldsa, int64_t ldsb, int64_t ldc, hipStream_t stream) {
    return hkq_gemm_mxfp4_ws(A, As, B, Bs, C, M, N, K, lda, ldb, ldsa, ldsb, ldc, nullptr, 0, stream);
}

int hkq_batched_gemm_a8w8(const void* A, const void* B, const float* sa, const float* sb, const void* bias, void* C,
                          int64_t batch, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb, int64_t ldc,
                          int64_t batch_stride_a, int64_t batch_stride_b, int64_t batch_stride_c,
                          int64_t batch_stride_sa, int64_t batch_stride_sb, int64_t batch_stride_bias,
                          hipStream_t stream) {
    if (int e = check_common(M, N, K, ldc, C)) return e;
    HKQ_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535]");
    HKQ_CHECK_ARG(K % 64 == 0, "K must be a multiple of 64");
    HKQ_CHECK_ARG(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0,
                  "lda/ldb must be >= K and multiples of 16");
    HKQ_CHECK_ARG(batch <= 1 || (batch_stride_a % 16 == 0 && batch_stride_b % 16 == 0 && batch_stride_c % 8 == 0 &&
                                 batch_stride_sb % 4 == 0 && batch_stride_bias % 4 == 0),
                  "batch strides must keep every batch's operands aligned (A, B: 16 bytes; C: 8 elements; "
                  "b_scale, bias: 4 elements)");
    HKQ_CHECK_ALIGN(A, 16);
    HKQ_CHECK_ALIGN(B, 16);
    HKQ_CHECK_ALIGN(sb, 16);
    HKQ_CHECK_ALIGN(bias, 8);
    if (batch == 0) return 0;
    DenseParams p{};
    p.A = static_cast<const uint8_t*>(A);
    p.B = static_cast<const uint8_t*>(B);
    p.C = static_cast<uint16_t*>(C);
    p.sa = sa;
    p.sb = sb;
    p.M = (int)M; p.N = (int)N; p.K = (int)K; p.kbytes = (int)K;
    p.lda = lda; p.ldb = ldb; p.ldc = ldc;
    p.batch = (int)batch;
    p.bias = static_cast<const uint16_t*>(bias);
    p.bs_a = batch_stride_a; p.bs_b = batch_stride_b; p.bs_c = batch_stride_c;
    p.bs_sa = batch_stride_sa; p.bs_sb = batch_stride_sb; p.bs_bias = batch_stride_bias;
    return launch_dense<MODE_A8W8>(p, nullptr, 0, stream);
}

size_t hkq_gemm_bf16_workspace(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 32 != 0) return 0;
    return dense_plan(MODE_BF16, M, N, 2 * K, true).ws_bytes;
}

int hkq_batched_gemm_bf16(const void* A, const void* B, const void* bias, void* C, int64_t batch, int64_t M, int64_t N,
                          int64_t K, int64_t lda, int64_t ldb, int64_t ldc, int64_t batch_stride_a,
                          int64_t batch_stride_b, int64_t batch_stride_c, int64_t batch_stride_bias, void* workspace,
                          size_t workspace_bytes, hipStream_t stream) {
    if (int e = check_common(M, N, K, ldc, C)) return e;
    HKQ_CHECK_ARG(batch >= 0 && batch <= 65535, "batch must be in [0, 65535]");
    HKQ_CHECK_ARG(K % 32 == 0, "K must be a multiple of 32");
    HKQ_CHECK_ARG(lda >= K && ldb >= K && lda % 8 == 0 && ldb % 8 == 0,
                  "lda/ldb (elements) must be >= K and multiples of 8");
    HKQ_CHECK_ARG(batch <= 1 || (batch_stride_a % 8 == 0 && batch_stride_b % 8 == 0 && batch_stride_c % 8 == 0 &&
                                 batch_stride_bias % 4 == 0),
                  "batch strides must keep every batch's operands aligned (A, B, C: 8 elements; bias: 4)");
    HKQ_CHECK_ALIGN(A, 16);
    HKQ_CHECK_ALIGN(B, 16);
    HKQ_CHECK_ALIGN(bias, 8);
    HKQ_CHECK_ALIGN(workspace, 16);
    if (batch == 0) return 0;
    DenseParams p{};
    p.A = static_cast<const uint8_t*>(A);
    p.B = static_cast<const uint8_t*>(B);
    p.C = static_cast<uint16_t*>(C);
    p.M = (int)M; p.N = (int)N; p.K = (int)K; p.kbytes = (int)(2 * K);
    p.lda = 2 * lda; p.ldb = 2 * ldb; p.ldc = ldc;
    p.batch = (int)batch;
    p.bias = static_cast<const uint16_t*>(bias);
    p.bs_a = 2 * batch_stride_a; p.bs_b = 2 * batch_stride_b; p.bs_c = batch_stride_c;
    p.bs_bias = batch_stride_bias;
    return launch_dense<MODE_BF16>(p, workspace, workspace_bytes, stream);
}

int hkq_gemm_bf16(const void* A, const void* B, void* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldb,
                  int64_t ldc, hipStream_t stream) {
    return hkq_batched_gemm_bf16(A, B, nullptr, C, 1, M, N, K, lda, ldb, ldc, 0, 0, 0, 0, nullptr, 0, stream);
}

}  // extern "C"
