// moe.hip -- A8W8 MoE grouped GEMM over OGS routing metadata
// (moe-gemm/moe_op_gemm_a8w8/kernel.cpp:61-169 and the per-token x
// per-channel case of moe_op_gemm_a8w8_blockscale/kernel.cpp:54-167, i.e.
// group_k = K):
//
//   for each tile entry ExptData[pm] = e | (b << 16) (-1: skip), rows
//   gm = b*128 + r < ExptHist[e], sorted index s = ExptOffs[e] + gm,
//   token = GatherIndx[s] / topk (or s without a gather):
//     Y[s, n] = bf16( (sum_k X[token, k] W[e, n, k]) * xs(token) * ws(e, n) + bias[e, n] )
//
// with xs per tensor (xs[0]) or per token (xs[token * xs_tok]) and ws per
// expert (ws[e]) or per output channel group (ws[e * ws_e + (n / ws_gn) * ws_n]).
// Output rows stay in expert-sorted order, as in the reference (no combine).
//
// Tiles are 256 columns by two consecutive OGS blocks of one expert (256 rows,
// the dense GEMM's tile) or, where a pair of blocks straddles two experts, by
// one block (128 rows); the K loop is the shared pipelined main loop with the
// A rows gathered per lane through the routing index (rows of other tokens
// never enter LDS). Metadata is bounds-checked: entries naming an expert >= E,
// rows past the gather index or tokens past T read zero or are skipped instead
// of faulting.
#include <algorithm>
#include <cstdlib>

#include "gemm_stream.h"
#include "hkq_host.h"

namespace hkq {

struct MoeParams {
    const uint8_t* X;        // [T, sxm] E4M3FN, K contiguous
    const uint8_t* W;        // expert e at W + e*swe; wt == 0: row n at + n*swn, K contiguous;
                             // wt == 1 (N-contiguous [K, N]): row k at + k*swk, N contiguous
    uint16_t* Y;             // sorted row s at Y + s*sym
    const float* xs;         // nullptr: 1
    const float* ws;         // nullptr: 1
    const float* bias;       // nullptr: 0; else bias[e * bias_e + n]
    const int32_t* gather;   // nullptr: token = s
    const int32_t* hist;
    const int32_t* offs;
    const int32_t* expt_data;
    int T, E, N, K, topk, grid_m, y_rows, g_len;
    double rtopk;  // 1.0 / topk (div_recip)
    int64_t sxm, swe, swn, swk, sym;
    int wt;
    int64_t xs_tok, ws_e, ws_n, ws_gn, bias_e;
    int tiles_n, group_m, c16;
    int xcd_cols;  // pair_walk's column order
    // per-channel scales / bias readable as float4 (16-byte aligned rows of
    // contiguous channels, one scale per channel)
    int ws_vec, bias_vec;
};

constexpr int MOE_BM = 128;  // rows per OGS routing block

// Tiles: 256 columns x 256 rows = two consecutive routing blocks of one expert
// (4 waves of 128 x 128, the dense GEMM's geometry), or x 128 rows = one block
// (4 waves of 64 x 128) where a pair of blocks straddles two experts.
constexpr int MOE_WM = 2, MOE_WN = 2, MOE_TN = 4, MOE_BN = MOE_WN * MOE_TN * 32;

// Rows [row0, row0 + TM*64) of expert e (sorted rows start + row0 + r) times
// columns [n0, n0 + TN*64). LEAN: no bias, and the column scales absent, one
// per expert or one per channel readable as float4 (ws_vec); the epilogue
// then carries no code for the other layouts.
template <int TM, int KTB, int NS, bool LEAN, bool BT = false, int TN = MOE_TN>
__device__ __forceinline__ void moe_block(const MoeParams& p, int e, int row0, int n0, HKQ_LDS uint8_t* smem) {
    using Cfg = DenseCfg<MODE_A8W8, MOE_WM, MOE_WN, TM, TN, KTB>;
    constexpr int NW = Cfg::NW, BM = Cfg::BM, BN = Cfg::BN, LA = Cfg::LA, LB = Cfg::LB;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / MOE_WN, wn = wave % MOE_WN;
    const int khalf = lane >> 5;

    const int m_e = p.hist[e], start = p.offs[e];
    const int rows = min(m_e - row0, BM);
    if (rows <= 0 || start < 0) return;  // uniform over the workgroup
    const int rows_b = min(p.N - n0, BN);

    // token of tile row r (-1 when the row is past the expert's rows or the metadata)
    auto token_of = [&](int r) {
        const int s = start + row0 + r;
        if (r >= rows || s >= p.g_len) return -1;
        const int t = p.gather ? div_recip(p.gather[s], p.rtopk) : s;
        return (t >= 0 && t < p.T) ? t : -1;
    };

    LoopSrc src;
    src.a = p.X;
    src.a_bytes = min((int64_t)p.T * p.sxm, (int64_t)0x7FFFFFFF);
    if constexpr (BT) {
        // N-contiguous weights: the tile's columns of every row of K (columns
        // past N read the next row's bytes, which only reach output columns
        // that are never stored; the last row's read zero)
        src.b = p.W + (int64_t)e * p.swe + n0;
        src.b_bytes = min((int64_t)(p.K - 1) * p.swk + rows_b, (int64_t)0x7FFFFFFF);
        src.b_kstep = (int64_t)KTB * p.swk;
    } else {
        src.b = p.W + (int64_t)e * p.swe + (int64_t)n0 * p.swn;
        src.b_bytes = min((int64_t)rows_b * p.swn, (int64_t)0x7FFFFFFF);
    }
    src.as = src.bs = nullptr;
    src.as_bytes = src.bs_bytes = src.lsa = src.lsb = 0;
    src.KT = p.K / KTB;
    TableOff<LA> a_off;
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int r = (i * NW + wave) * Cfg::RPL + lane / Cfg::KT::CHUNKS;
        const int t = token_of(r);
        a_off.v[i] = t < 0 ? OOB : (uint32_t)(t * p.sxm) + (uint32_t)(Cfg::KT::load_chunk(lane, r) << 4);
    }
    TableOff<LB> b_off;
    if constexpr (BT) b_off = dense_offs_t<NW, LB>(wave, lane, p.swk);
    else b_off = dense_offs<NW, KTB, LB>(wave, lane, p.swn);

    // the epilogue's row scales, fetched before the K loop so that their
    // dependent loads (gather index, then scale) are not on the tile's tail
    float rs[TM];
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int t = p.xs ? token_of(wm * TM * 32 + j * 32 + (lane & 31)) : -1;
        rs[j] = !p.xs ? 1.0f : (t < 0 ? 0.0f : p.xs[(int64_t)t * p.xs_tok]);
    }

    v16f acc[TN][TM];
    gemm_mainloop<MODE_A8W8, MOE_WM, MOE_WN, TM, TN, KTB, NS, BT>(src, a_off, b_off, smem, lane, wave, acc);

    const int s0 = start + row0;
    const int nw = n0 + wn * TN * 32;
    const int out_rows = min(rows, p.y_rows - s0);
    auto col_scale4 = [&](int i, int g) {
        // n .. n+3 lie inside C together (N % 4 == 0)
        const int n = nw + i * 32 + 8 * g + 4 * khalf;
        if (!p.ws) return make_float4(1.f, 1.f, 1.f, 1.f);
        if (n >= p.N) return make_float4(0.f, 0.f, 0.f, 0.f);
        const float* w = p.ws + (int64_t)e * p.ws_e;
        if (p.ws_n == 0) {  // one scale per expert
            const float v = w[0];
            return make_float4(v, v, v, v);
        }
        if (LEAN || p.ws_vec) return *reinterpret_cast<const float4*>(w + n);
        // column groups (ws_gn >= 2, clamped to N by the host: 32-bit quotients)
        const int gn = (int)p.ws_gn;
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = w[(int64_t)((n + c) / gn) * p.ws_n];
        return make_float4(v[0], v[1], v[2], v[3]);
    };
    auto row_scale = [&](int j) { return rs[j]; };
    uint16_t* Y = p.Y + (int64_t)s0 * p.sym;
    if (!LEAN && p.bias)
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, Y, p.sym, out_rows, p.N, wm * TM * 32, nw, p.c16 != 0, row_scale,
                                col_scale4, [&](int i, int g) {
                                    const int n = nw + i * 32 + 8 * g + 4 * khalf;
                                    if (n >= p.N) return make_float4(0.f, 0.f, 0.f, 0.f);
                                    const float* b = p.bias + (int64_t)e * p.bias_e + n;
                                    if (p.bias_vec) return *reinterpret_cast<const float4*>(b);
                                    return make_float4(b[0], b[1], b[2], b[3]);
                                });
    else
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, Y, p.sym, out_rows, p.N, wm * TM * 32, nw, p.c16 != 0, row_scale,
                                col_scale4, NoBias{});
}

// Workgroup id -> (routing-block pair q, column tile tn): the ids walk the
// columns of `group` pairs at a time in dispatch order, so the CUs of every XCD
// work on the same few pairs (one expert) together. The experts' block counts
// differ, and giving each XCD its own range of experts (as tile_coords does for
// the dense GEMMs) left XCDs idle: the A8W8 gate/up and down projections ran
// 9% and 31% slower that way, the MXFP4 ones 16% and 33%.
// xcd_cols: within a group the columns go in blocks of 8, one column of the
// block per consecutive id and the group's pairs one after the other, so that
// (dispatch placing id u on XCD u % 8, and group * tiles_n % 8 == 0) each XCD
// holds every pair of the group on the same columns: the pairs share each
// weight tile and each pair's activation rows in that XCD's L2. Otherwise the
// group's pairs alternate id by id (a weight tile's pairs on neighbouring XCDs).
__device__ __forceinline__ void pair_walk(int bid, int pairs, int tiles_n, int group, int xcd_cols, int& q, int& tn) {
    const int per = group * tiles_n;
    const int grp = bid / per, first = grp * group;
    const int gsize = min(pairs - first, group), in_g = bid - grp * per;
    if (!xcd_cols) {
        q = first + in_g % gsize;
        tn = in_g / gsize;
        return;
    }
    const int nfull = tiles_n >> 3, blk = 8 * gsize;
    const int cb = min(in_g / blk, nfull);  // column block; the last one may be narrower
    const int rem = in_g - cb * blk;
    const int w = cb < nfull ? 8 : tiles_n - 8 * nfull;
    q = first + rem / w;
    tn = 8 * cb + rem % w;
}

// Work unit of workgroup bid: tile t (pair q, column tn) in pair_walk order,
// whole (half -1) or one of its two blocks (half 0 / 1). When the last round
// of the launch's tiles would fill at most half of the CUs, each of its tiles
// is cut into its two blocks, run by two workgroups (the padding entries come
// last, so these are the last live tiles and the empty ones after them):
//   units [0, s0): tile u; then block (u - s0) & 1 of tile s0 + (u - s0) / 2.
// Returns false for the spare units past the last tile.
__device__ __forceinline__ bool pair_unit(int bid, int pairs, int tiles_n, int group, int xcd_cols, int split, int& q,
                                          int& tn, int& half) {
    const int total = pairs * tiles_n;
    const int s0 = total - split;
    int t;
    half = -1;
    if (bid < s0) {
        t = bid;
    } else {
        t = s0 + (bid - s0) / 2;
        half = (bid - s0) & 1;
        if (t >= total) return false;
    }
    pair_walk(t, pairs, tiles_n, group, xcd_cols, q, tn);
    return true;
}

// pair_walk's column order (host side): XCD-aligned columns for wide
// projections (measured on MI355X, Mixtral A8W8 gate/up, N = 28672: 0.981 ->
// 0.963 ms, L2 hit rate 44% -> 55%; with 8 x 1024 rows per expert 0.858 ->
// 0.825 ms, 35% -> 62%), the alternating order for narrow ones (down, N =
// 4096: 0.540 vs 0.552 ms).
static int moe_xcd_cols(int tiles_n) { return tiles_n >= 32 ? 1 : 0; }

// Tiles of the last round that pair_unit cuts in two (host side).
static int64_t moe_tail_split(int64_t tiles) {
    const int ncu = cu_count();
    const int64_t last = ncu > 0 ? tiles % ncu : 0;
    return (last > 0 && 2 * last <= ncu) ? last : 0;
}

// Workgroup: routing entries (2q, 2q + 1) x column tile tn. Two consecutive
// blocks of one expert form one 256-row tile; otherwise each valid entry is a
// 128-row tile (64 rows when it holds at most 64 of its expert's rows), one
// after the other.
template <int KTB, int NS, bool LEAN, bool BT = false>
__global__ __launch_bounds__(64 * MOE_WM * MOE_WN, 1) void moe_gemm_kernel(const MoeParams p) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;
    int q, tn;
    pair_walk(blockIdx.x, (p.grid_m + 1) / 2, p.tiles_n, p.group_m, p.xcd_cols, q, tn);
    const int n0 = tn * MOE_BN;
    const int pm0 = 2 * q, pm1 = 2 * q + 1;
    const int ed0 = p.expt_data[pm0], ed1 = pm1 < p.grid_m ? p.expt_data[pm1] : -1;
    // an entry with bit 31 set (-1 or any malformed word) is skipped: its block
    // id would be negative
    const int e0 = ed0 & 0xFFFF, e1 = ed1 & 0xFFFF;
    const bool v0 = ed0 >= 0 && e0 < p.E, v1 = ed1 >= 0 && e1 < p.E;
    const int b0 = ed0 >> 16, b1 = ed1 >> 16;
    if (v0 && v1 && e0 == e1 && b1 == b0 + 1) {
        moe_block<4, KTB, NS, LEAN, BT>(p, e0, b0 * MOE_BM, n0, smem);
        return;
    }
    // a block holding at most 64 of its expert's rows (an expert's last block)
    // runs as a 64-row tile, with 128-byte K-tiles on a 3-stage ring (its
    // little MFMA work hides less of the load latency)
    constexpr int NS1 = KTB == 128 && NS == 2 ? 3 : NS;
    static_assert(DenseCfg<MODE_A8W8, MOE_WM, MOE_WN, 1, MOE_TN, KTB>::lds_bytes(NS1) <=
                      DenseCfg<MODE_A8W8, MOE_WM, MOE_WN, 4, MOE_TN, KTB>::lds_bytes(NS),
                  "the 64-row ring fits the launch's LDS");
    auto block = [&](int e, int b) {
        if (p.hist[e] - b * MOE_BM <= MOE_BM / 2)
            moe_block<1, KTB, NS1, LEAN, BT>(p, e, b * MOE_BM, n0, smem);
        else
            moe_block<2, KTB, NS, LEAN, BT>(p, e, b * MOE_BM, n0, smem);
    };
    if (v0) block(e0, b0);
    if (v1) {
        __syncthreads();  // every wave is done with the first block's epilogue staging
        block(e1, b1);
    }
}

// ---------------------------------------------------------------------------
// Decode-size MoE (at most 64 routed rows in all, so at most 64 per block):
// the streaming layout of the dense GEMMs' narrow path. Workgroup u takes
// routing entry u / slices and the 16*NT columns of slice u % slices; its 4
// waves split K and load fragments from memory straight into registers for
// the 16x16x128 MFMA (lane l: row l % 16 of each 16-row group, bytes
// [16q, 16q+16) and [64+16q, 64+16q+16) of a K-step, q = l/16; result
// D[4q + i][l % 16]), the rows gathered per lane through the routing index.
// Every weight row of an active expert is read once; the tiled kernel would
// give each block of a few rows a whole 256 x 256 tile and leave most CUs idle.
constexpr int MOE_NARROW_WAVES = 4, MOE_NARROW_MAX_ROWS = 64;

template <int MT, int NT>
__global__ __launch_bounds__(64 * MOE_NARROW_WAVES) void moe_narrow_kernel(const MoeParams p, int slices) {
    constexpr int DEPTH = MT * NT <= 2 ? 6 : 4;
    __shared__ v4f red[MOE_NARROW_WAVES][NT][MT][64];
    const int pm = blockIdx.x / slices, n0 = (blockIdx.x % slices) * 16 * NT;
    const int ed = p.expt_data[pm];
    const int e = ed & 0xFFFF, b = ed >> 16;
    if (ed < 0 || e >= p.E) return;  // uniform over the workgroup (bit 31 set: -1 or malformed)
    const int m_e = p.hist[e], start = p.offs[e];
    const int rows = min(m_e - b * MOE_BM, 16 * MT);
    if (rows <= 0 || start < 0) return;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    // sorted row and token of the lane's row in each 16-row group (-1: none)
    int srow[MT], tok[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int rr = t * 16 + r, sr = start + b * MOE_BM + rr;
        int tk = -1;
        if (rr < rows && sr < p.g_len) {
            tk = p.gather ? div_recip(p.gather[sr], p.rtopk) : sr;
            if (tk < 0 || tk >= p.T) tk = -1;
        }
        srow[t] = sr;
        tok[t] = tk;
    }
    const int S = p.K / 128;
    const int s0 = wave * S / MOE_NARROW_WAVES, s1 = (wave + 1) * S / MOE_NARROW_WAVES;
    const int rows_b = min(16 * NT, p.N - n0);
    const auto rb = make_rsrc(p.W + (int64_t)e * p.swe + (int64_t)n0 * p.swn, (uint32_t)(rows_b * p.swn));
    const auto ra = make_rsrc(p.X, (uint32_t)((int64_t)p.T * p.sxm));
    uint32_t b_off[NT], a_off[MT];
#pragma unroll
    for (int i = 0; i < NT; ++i) b_off[i] = (uint32_t)((i * 16 + r) * p.swn + 16 * q);
#pragma unroll
    for (int t = 0; t < MT; ++t) a_off[t] = tok[t] < 0 ? OOB : (uint32_t)(tok[t] * p.sxm + 16 * q);

    struct Frag {
        v4i b0[NT], b1[NT], a0[MT], a1[MT];
    };
    // Steps at or past s1 read zeros: offsets with the OOB bit are past every
    // range. Offsets stay below 2^32: b_off, and a_off of a valid row, are below
    // 2^31, an invalid row's a_off is OOB itself, and kb < 2^31.
    auto load = [&](int s, Frag& f) {
        const uint32_t kb = (uint32_t)s * 128, kill = s < s1 ? 0u : OOB;
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const uint32_t o = (b_off[i] + kb) | kill;
            f.b0[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, o, 0, 0);
            f.b1[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, o + 64, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const uint32_t o = (a_off[t] + kb) | kill;
            f.a0[t] = __builtin_amdgcn_raw_buffer_load_b128(ra, o, 0, 0);
            f.a1[t] = __builtin_amdgcn_raw_buffer_load_b128(ra, o + 64, 0, 0);
        }
    };
    v4f acc[NT][MT];
#pragma unroll
    for (int i = 0; i < NT; ++i)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[i][t] = v4f{0.f, 0.f, 0.f, 0.f};
    auto mma = [&](const Frag& f) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const v8i bb = v8i{f.a0[t][0], f.a0[t][1], f.a0[t][2], f.a0[t][3], f.a1[t][0], f.a1[t][1], f.a1[t][2], f.a1[t][3]};
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                const v8i aa = v8i{f.b0[i][0], f.b0[i][1], f.b0[i][2], f.b0[i][3],
                                   f.b1[i][0], f.b1[i][1], f.b1[i][2], f.b1[i][3]};
                acc[i][t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(aa, bb, acc[i][t], 0, 0, 0, 127, 0, 127);
            }
        }
    };
    Frag f[DEPTH];
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
    const float* wsc = p.ws ? p.ws + (int64_t)e * p.ws_e : nullptr;
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int n = n0 + 16 * i + 4 * q;
        if (n >= p.N) break;  // N % 4 == 0: n .. n+3 all in or all out
        float4 cs = make_float4(1.f, 1.f, 1.f, 1.f), cb = make_float4(0.f, 0.f, 0.f, 0.f);
        if (wsc) {
            if (p.ws_vec) {
                cs = *reinterpret_cast<const float4*>(wsc + n);
            } else {
                const int gn = (int)p.ws_gn;
                cs = make_float4(wsc[(int64_t)(n / gn) * p.ws_n], wsc[(int64_t)((n + 1) / gn) * p.ws_n],
                                 wsc[(int64_t)((n + 2) / gn) * p.ws_n], wsc[(int64_t)((n + 3) / gn) * p.ws_n]);
            }
        }
        if (p.bias) {
            const float* bp = p.bias + (int64_t)e * p.bias_e + n;
            cb = p.bias_vec ? *reinterpret_cast<const float4*>(bp) : make_float4(bp[0], bp[1], bp[2], bp[3]);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t * 16 + r >= rows || srow[t] >= p.y_rows) continue;
            v4f v = red[0][i][t][lane];
#pragma unroll
            for (int w = 1; w < MOE_NARROW_WAVES; ++w) v += red[w][i][t][lane];
            const float a = !p.xs ? 1.0f : (tok[t] < 0 ? 0.0f : p.xs[(int64_t)tok[t] * p.xs_tok]);
            *reinterpret_cast<v2i*>(p.Y + (int64_t)srow[t] * p.sym + n) =
                v2i{(int)pk_bf16(v[0] * a * cs.x + cb.x, v[1] * a * cs.y + cb.y),
                    (int)pk_bf16(v[2] * a * cs.z + cb.z, v[3] * a * cs.w + cb.w)};
        }
    }
}

template <int MT, int NT>
static void launch_moe_narrow_nt(const MoeParams& p, hipStream_t stream) {
    const int slices = (p.N + 16 * NT - 1) / (16 * NT);
    moe_narrow_kernel<MT, NT><<<dim3((unsigned)((int64_t)p.grid_m * slices)), 64 * MOE_NARROW_WAVES, 0, stream>>>(p, slices);
}

// Narrow MoE launch: MT 16-row groups cover the routed rows (1, 2 or 4);
// 16 columns per workgroup, or 64 when N > 4096.
static int launch_moe_narrow(const MoeParams& p, int64_t routed_rows, hipStream_t stream) {
    if (p.grid_m == 0 || p.N == 0) return 0;
    const bool wide = p.N > 4096;
    if (routed_rows <= 16) {
        if (wide) launch_moe_narrow_nt<1, 4>(p, stream);
        else launch_moe_narrow_nt<1, 1>(p, stream);
    } else if (routed_rows <= 32) {
        if (wide) launch_moe_narrow_nt<2, 4>(p, stream);
        else launch_moe_narrow_nt<2, 1>(p, stream);
    } else {
        launch_moe_narrow_nt<4, 1>(p, stream);
    }
    return hkq_launch_status();
}

// ---------------------------------------------------------------------------
// Persistent A8W8 MoE kernel over the dense GEMMs' K-tile stream
// (gemm_stream.h), one workgroup per CU. The units whose two routing entries
// are consecutive blocks of one expert (256-row tiles) form one stream: the
// next tile's first K-tiles load during the current tile's last ones, its
// gather entries reach LDS while the current tile computes (the tiled kernel
// waits for them in each tile's prologue), and the epilogue stages C through
// LDS areas that take the place of the unit-building lists. The lone blocks run before or after the stream with the tiled
// kernel's block code (64-row blocks on a 3-stage ring: a 64 x 256 tile has
// little MFMA work to hide its loads behind).
// LEAN scale layouts only (no bias; column scales absent, per expert or per
// channel), 128-byte K-tiles, K % 1024 == 0.
constexpr int MS_MAXU = 64;  // units per workgroup (one per lane of wave 0; the host checks)
using MoeWhole = DenseCfg<MODE_A8W8, MOE_WM, MOE_WN, 4, MOE_TN, 128>;
constexpr int MS_SCL = 2 * MoeWhole::STAGE;   // 2 slots: 256 row scales, then 256 column scales
constexpr int MS_SLOT = 2 * 256 * 4;
constexpr int MS_TOK = MS_SCL + 2 * MS_SLOT;  // 2 slots of 256 gather entries
constexpr int MS_WL = MS_TOK + 2 * 1024;      // stream units: e, row0, n0, start, rows (8 ints each)
constexpr int MS_RL = MS_WL + MS_MAXU * 32;   // lone units: entry, n0 (4 ints each)
constexpr int MS_CNT = MS_RL + MS_MAXU * 16;  // unit counts
constexpr int MS_MAXE = 1024;                 // routing entries (the host checks)
constexpr int MS_WP = MS_CNT + 64;            // whole pairs: e, row0, start, rows (4 ints each)
constexpr int MS_RP = MS_WP + MS_MAXE / 2 * 16;  // lone blocks: the entry (1 int each)
// the epilogue's staging areas (one per wave) take the place of the whole-pair
// and lone-block lists, which are read only while the unit lists are built
constexpr int MS_STG = MS_WP;
constexpr int MS_LDS = MS_RP + MS_MAXE * 4 > MS_STG + MOE_WM * MOE_WN * STREAM_STG ? MS_RP + MS_MAXE * 4
                                                                                     : MS_STG + MOE_WM * MOE_WN * STREAM_STG;
static_assert(MS_LDS <= 160 * 1024, "LDS budget of a CDNA4 CU");
// Lone blocks run as 128-column pieces (256 with N-contiguous weights, whose
// K-tiles are 256 columns wide): twice as many pieces as 256-column tiles, so
// that they spread over more workgroups (measured on MI355X, Mixtral down: the
// workgroups with a lone tile after their two stream tiles ended ~85 us after
// the others).
constexpr int MS_LONE_BN = 128, MS_LONE_TN = MS_LONE_BN / (MOE_WN * 32);
constexpr int MS_LONE_NS1 = 5, MS_LONE_NS2 = 4;  // ring stages of 64- and 128-row pieces
static_assert(DenseCfg<MODE_A8W8, MOE_WM, MOE_WN, 2, MOE_TN, 128>::lds_bytes(2) <= MS_WL &&
                  DenseCfg<MODE_A8W8, MOE_WM, MOE_WN, 1, MOE_TN, 128>::lds_bytes(3) <= MS_WL &&
                  DenseCfg<MODE_A8W8, MOE_WM, MOE_WN, 2, MS_LONE_TN, 128>::lds_bytes(MS_LONE_NS2) <= MS_WL &&
                  DenseCfg<MODE_A8W8, MOE_WM, MOE_WN, 1, MS_LONE_TN, 128>::lds_bytes(MS_LONE_NS1) <= MS_WL,
              "the tiled blocks after the stream leave the unit lists alone");

struct MoeStreamSeq {
    static constexpr bool GATHER = true;
    const MoeParams* p;
    int tiles, KT;
    uint32_t lsa, lsb;
    uint32_t b_kstep;  // N-contiguous weights: bytes from one K-tile to the next
    const HKQ_LDS int* wl;
    HKQ_LDS int* tok;
    int lane, wave;
    struct Unit {
        int e, row0, n0, start, rows;
    };
    __device__ Unit unit(int k) const {
        const HKQ_LDS int* u = wl + 8 * k;
        return Unit{__builtin_amdgcn_readfirstlane(u[0]), __builtin_amdgcn_readfirstlane(u[1]),
                    __builtin_amdgcn_readfirstlane(u[2]), __builtin_amdgcn_readfirstlane(u[3]),
                    __builtin_amdgcn_readfirstlane(u[4])};
    }
    __device__ StreamSrc src(int k) const {
        const Unit u = unit(k);
        StreamSrc s;
        s.a = p->X;
        s.a_bytes = (uint32_t)min((int64_t)p->T * p->sxm, (int64_t)0x7FFFFFFF);
        if (p->wt) {
            s.b = p->W + (int64_t)u.e * p->swe + u.n0;
            s.b_bytes = (uint32_t)min((int64_t)(p->K - 1) * p->swk + min(p->N - u.n0, MOE_BN), (int64_t)0x7FFFFFFF);
        } else {
            s.b = p->W + (int64_t)u.e * p->swe + (int64_t)u.n0 * p->swn;
            s.b_bytes = (uint32_t)min((int64_t)min(p->N - u.n0, MOE_BN) * p->swn, (int64_t)0x7FFFFFFF);
        }
        s.as = s.bs = nullptr;
        s.as_bytes = s.bs_bytes = 0;
        return s;
    }
    // token of row r of tile k (-1: past the expert's rows, the gather index or T)
    __device__ int token(int k, const Unit& u, int r) const {
        const int s = u.start + u.row0 + r;
        if (r >= u.rows || s >= p->g_len) return -1;
        const int t = p->gather ? div_recip(tok[(k & 1) * 256 + r], p->rtopk) : s;
        return (t >= 0 && t < p->T) ? t : -1;
    }
    // gather entries of tile k's 256 rows into token slot k & 1: one 4-byte
    // LDS-direct load per lane and wave (zeros past the gather index, past the
    // last tile or without a gather, so that every wave issues the load)
    __device__ void load_tokens(int k) const {
        int s0 = 0;
        bool live = k < tiles && p->gather != nullptr;
        if (live) {
            const Unit u = unit(k);
            s0 = u.start + u.row0;
            live = s0 < p->g_len;
        }
        const uint32_t bytes = live ? (uint32_t)min(p->g_len - s0, 256) * 4u : 0u;
        lds_load4(live ? p->gather + s0 : p->gather, bytes,
                  reinterpret_cast<HKQ_LDS uint8_t*>(tok + (k & 1) * 256 + wave * 64), (uint32_t)(wave * 64 + lane) * 4u);
    }
    template <class AOff>
    __device__ void a_rows(int k, AOff& a) const {
        using KT = MoeWhole::KT;
        const Unit u = unit(k);
#pragma unroll
        for (int i = 0; i < MoeWhole::LA; ++i) {
            const int r = (i * MoeWhole::NW + wave) * MoeWhole::RPL + lane / KT::CHUNKS;
            const int t = token(k, u, r);
            a.v[i] = t < 0 ? OOB : (uint32_t)(t * p->sxm) + (uint32_t)(KT::load_chunk(lane, r) << 4);
        }
    }
};

// Epilogue of a stream tile: the dense stream's staged stores
// (stream_store_tile) into the tile's sorted rows, with the row scales
// (gathered per token) and the column scales fetched into LDS when the tile
// begins.
struct MoeStreamEpi {
    static constexpr int TM = 4, TN = MOE_TN;
    // per wave: the epilogue's C stores, then begin()'s row-scale, column-scale
    // and gather-entry loads
    static constexpr int VM_ISSUED = TN * TM * 2 + 3;
    const MoeStreamSeq* seq;
    const MoeParams* p;
    HKQ_LDS uint8_t* scl;
    HKQ_LDS uint8_t* stg;  // this wave's STREAM_STG bytes of staging
    int lane, wave;
    __device__ void begin(int k) {
        const MoeStreamSeq::Unit u = seq->unit(k);
        HKQ_LDS uint8_t* slot = scl + (k & 1) * MS_SLOT;
        const int t = seq->token(k, u, wave * 64 + lane);
        const uint32_t xs_bytes =
            p->xs && p->T > 0 ? (uint32_t)min(((int64_t)(p->T - 1) * p->xs_tok + 1) * 4, (int64_t)0x7FFFFFFF) : 0u;
        lds_load4(p->xs, xs_bytes, slot + wave * 256, t < 0 ? OOB : (uint32_t)t * (uint32_t)p->xs_tok * 4u);
        const int n = u.n0 + wave * 64 + lane;
        const float* w = p->ws ? p->ws + (int64_t)u.e * p->ws_e : nullptr;
        const uint32_t ws_bytes = p->ws ? (p->ws_n == 0 ? 4u : (uint32_t)p->N * 4u) : 0u;
        lds_load4(w, ws_bytes, slot + 1024 + wave * 256, n < p->N ? (p->ws_n == 0 ? 0u : (uint32_t)n * 4u) : OOB);
        seq->load_tokens(k + 1);
    }
    __device__ void end(int k, v16f (&acc)[TN][TM]) {
        const MoeStreamSeq::Unit u = seq->unit(k);
        const int wm = wave / MOE_WN, wn = wave % MOE_WN;
        const int khalf = lane >> 5, r = lane & 31;
        const HKQ_LDS float* sl = reinterpret_cast<const HKQ_LDS float*>(scl + (k & 1) * MS_SLOT);
        const int s0 = u.start + u.row0;
        const int mw0 = wm * TM * 32, nw0 = u.n0 + wn * TN * 32;
        float rs[TM];
#pragma unroll
        for (int j = 0; j < TM; ++j) rs[j] = p->xs ? sl[mw0 + j * 32 + r] : 1.0f;
        stream_store_tile<TM, TN>(
            acc, stg, p->Y + (int64_t)(s0 + mw0) * p->sym + nw0, p->sym, min(u.rows, p->y_rows - s0) - mw0,
            p->N - nw0, rs,
            [&](int i, int g) {
                return p->ws ? *reinterpret_cast<const HKQ_LDS v4f*>(sl + 256 + wn * TN * 32 + i * 32 + 8 * g + 4 * khalf)
                             : v4f{1.f, 1.f, 1.f, 1.f};
            },
            lane);
    }
};

template <bool BT>
__global__ __launch_bounds__(64 * MOE_WM * MOE_WN, 1) void moe_stream_kernel(const MoeParams p) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int b = blockIdx.x, G = gridDim.x;
    HKQ_LDS int* wl = reinterpret_cast<HKQ_LDS int*>(smem + MS_WL);
    HKQ_LDS int* rl = reinterpret_cast<HKQ_LDS int*>(smem + MS_RL);
    HKQ_LDS int* cnt = reinterpret_cast<HKQ_LDS int*>(smem + MS_CNT);
    // Work units in two global lists, each in pair_walk order over its own
    // entries: the whole pairs' tiles (the stream) and the lone blocks' tiles.
    // A whole pair is an entry (e, b) with b even followed by the entry
    // (e, b + 1), so that with the producers' layout every expert's blocks pair
    // up among themselves and only an odd count's last block (the expert's
    // fewest rows) is lone; any other valid entry is a lone block. Workgroup b
    // takes stream units b, b + G, ... and lone units G-1-b, 2G-1-b, ...: a
    // workgroup with one more stream tile than others gets the fewer of the
    // (cheaper) lone units. Wave 0 classifies the entries 64 at a time, then
    // lane k builds entry k of each of the workgroup's lists.
    HKQ_LDS int* wp = reinterpret_cast<HKQ_LDS int*>(smem + MS_WP);
    HKQ_LDS int* rp = reinterpret_cast<HKQ_LDS int*>(smem + MS_RP);
    if (wave == 0) {
        const uint64_t below = (1ull << lane) - 1ull;
        auto entry = [&](int m) {  // -1 past the list or for an invalid entry
            const int ed = m >= 0 && m < p.grid_m ? p.expt_data[m] : -1;
            return ed >= 0 && (ed & 0xFFFF) < p.E ? ed : -1;
        };
        auto leads = [](int ed, int next) {  // (e, b even) followed by (e, b + 1)
            return ed >= 0 && ((ed >> 16) & 1) == 0 && next == ed + (1 << 16);
        };
        int nwp = 0, nrp = 0;
        for (int m0 = 0; m0 < p.grid_m; m0 += 64) {
            const int m = m0 + lane;
            const int ed = entry(m), next = entry(m + 1), prev = entry(m - 1);
            const bool lead = leads(ed, next);
            const bool lone = ed >= 0 && !lead && !leads(prev, ed);
            bool whole = false;
            int e0 = 0, row0 = 0, start = 0, rows = 0;
            if (lead) {
                e0 = ed & 0xFFFF;
                row0 = (ed >> 16) * MOE_BM;
                start = p.offs[e0];
                rows = min(p.hist[e0] - row0, 2 * MOE_BM);
                whole = rows > 0 && start >= 0;  // else the pair has nothing to compute
            }
            const uint64_t bw = __ballot(whole), br = __ballot(lone);
            if (whole) {
                HKQ_LDS int* d = wp + 4 * (nwp + __popcll(bw & below));
                d[0] = e0;
                d[1] = row0;
                d[2] = start;
                d[3] = rows;
            }
            if (lone) rp[nrp + __popcll(br & below)] = ed;
            nwp += __popcll(bw);
            nrp += __popcll(br);
        }
        const int k = lane;
        const int w = b + k * G, r = (G - 1 - b) + k * G;
        const int tiles_l = BT ? p.tiles_n : (p.N + MS_LONE_BN - 1) / MS_LONE_BN;
        const bool wl_live = w < nwp * p.tiles_n, rl_live = r < nrp * tiles_l;
        if (wl_live) {
            int qi, tn;
            pair_walk(w, nwp, p.tiles_n, p.group_m, p.xcd_cols, qi, tn);
            const HKQ_LDS int* src = wp + 4 * qi;
            HKQ_LDS int* d = wl + 8 * k;
            d[0] = src[0];
            d[1] = src[1];
            d[2] = tn * MOE_BN;
            d[3] = src[2];
            d[4] = src[3];
        }
        if (rl_live) {
            int qi, tn;
            pair_walk(r, nrp, tiles_l, p.group_m, BT ? p.xcd_cols : (tiles_l >= 32 ? 1 : 0), qi, tn);
            HKQ_LDS int* d = rl + 4 * k;
            d[0] = rp[qi];
            d[1] = tn * (BT ? MOE_BN : MS_LONE_BN);
        }
        const uint64_t cw = __ballot(wl_live), cr = __ballot(rl_live);
        if (lane == 0) {
            cnt[0] = __popcll(cw);
            cnt[1] = __popcll(cr);
        }
    }
    __syncthreads();
    const int n_whole = __builtin_amdgcn_readfirstlane(cnt[0]), n_rest = __builtin_amdgcn_readfirstlane(cnt[1]);

    auto lone = [&]() {
        for (int i = 0; i < n_rest; ++i) {
            const int ed = __builtin_amdgcn_readfirstlane(rl[4 * i]), n0 = __builtin_amdgcn_readfirstlane(rl[4 * i + 1]);
            const int e = ed & 0xFFFF, bk = ed >> 16;
            __syncthreads();  // every wave is done with the LDS of what ran before
            if constexpr (BT) {
                if (p.hist[e] - bk * MOE_BM <= MOE_BM / 2)
                    moe_block<1, 128, 3, true, BT>(p, e, bk * MOE_BM, n0, smem);
                else
                    moe_block<2, 128, 2, true, BT>(p, e, bk * MOE_BM, n0, smem);
            } else {
                if (p.hist[e] - bk * MOE_BM <= MOE_BM / 2)
                    moe_block<1, 128, MS_LONE_NS1, true, false, MS_LONE_TN>(p, e, bk * MOE_BM, n0, smem);
                else
                    moe_block<2, 128, MS_LONE_NS2, true, false, MS_LONE_TN>(p, e, bk * MOE_BM, n0, smem);
            }
        }
    };
    // Odd workgroups run their lone units before the stream, even ones after
    // it: a lone block reads its expert's weight columns with few rows to
    // hide them (mostly from HBM: the whole pairs of its expert ran long
    // before or after), so half of them at each end halves the HBM demand.
    const bool first = b & 1;
    if (first) lone();
    if (n_whole > 0) {
        __syncthreads();  // every wave is done with the LDS of what ran before
        MoeStreamSeq seq{&p,   n_whole, p.K / 128, 0u, 0u, (uint32_t)(128 * p.swk), wl,
                         reinterpret_cast<HKQ_LDS int*>(smem + MS_TOK), lane, wave};
        seq.load_tokens(0);
        tile_barrier<0>();  // tile 0's gather entries visible to every wave
        TableOff<MoeWhole::LA> a_off;
        seq.a_rows(0, a_off);
        TableOff<MoeWhole::LB> b_off;
        if constexpr (BT) b_off = dense_offs_t<MoeWhole::NW, MoeWhole::LB>(wave, lane, p.swk);
        else b_off = dense_offs<MoeWhole::NW, 128, MoeWhole::LB>(wave, lane, p.swn);
        MoeStreamEpi epi{&seq, &p, smem + MS_SCL, smem + MS_STG + wave * STREAM_STG, lane, wave};
        v16f acc[MOE_TN][4];
        gemm_stream<MODE_A8W8, MOE_WM, MOE_WN, 4, MOE_TN, BT>(seq, a_off, b_off, smem, lane, wave, acc, epi);
    }
    if (!first) lone();
}

template <int KTB, int NS>
static int launch_moe(MoeParams& p, hipStream_t stream) {
    using Whole = DenseCfg<MODE_A8W8, MOE_WM, MOE_WN, 4, MOE_TN, KTB>;
    using Half = DenseCfg<MODE_A8W8, MOE_WM, MOE_WN, 2, MOE_TN, KTB>;
    constexpr int LDS = Whole::lds_bytes(NS) > Half::lds_bytes(NS) ? Whole::lds_bytes(NS) : Half::lds_bytes(NS);
    static_assert(LDS <= 160 * 1024, "LDS budget of a CDNA4 CU");
    const bool lean = !p.bias && (!p.ws || p.ws_vec || p.ws_n == 0);
    // N-contiguous weights (wt) need 128-byte K-tiles (the entry point checks)
    auto kern = lean ? moe_gemm_kernel<KTB, NS, true> : moe_gemm_kernel<KTB, NS, false>;
    if constexpr (KTB == 128)
        if (p.wt) kern = lean ? moe_gemm_kernel<KTB, NS, true, true> : moe_gemm_kernel<KTB, NS, false, true>;
    const int variant = (lean ? 1 : 0) + (p.wt ? 2 : 0);
    static bool attr_set[4] = {false, false, false, false};
    if (!attr_set[variant]) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
        if (e != hipSuccess) {
            set_error("hipFuncSetAttribute(MaxDynamicSharedMemorySize=%d) failed: %s", LDS, hipGetErrorString(e));
            return (int)e;
        }
        attr_set[variant] = true;
    }
    p.tiles_n = (p.N + MOE_BN - 1) / MOE_BN;
    const bool group_default = p.group_m <= 0;
    if (group_default) p.group_m = 2;
    p.xcd_cols = moe_xcd_cols(p.tiles_n);
    const int64_t nblk = (int64_t)((p.grid_m + 1) / 2) * p.tiles_n;
    if (nblk == 0) return 0;
    if constexpr (KTB == 128) {
        // the persistent stream (HKQ_MOE_STREAM=0 keeps the tiled kernel): at
        // least two units per CU (measured on MI355X, Mixtral A8W8: gate/up,
        // 15.75 units per CU, 0.946 -> 0.878 ms; down, 2.25 per CU, 0.491 ->
        // 0.475 ms), at most MS_MAXU units per CU and MS_MAXE entries, 16-byte
        // aligned Y rows, and 32-bit offsets for the gathered row scales
        const char* se = std::getenv("HKQ_MOE_STREAM");
        const int64_t ncu = cu_count();
        if (!(se && se[0] == '0') && lean && ncu > 0 && (p.K / 128) % 8 == 0 && nblk >= 2 * ncu &&
            ((int64_t)p.grid_m * (p.wt ? p.tiles_n : (p.N + MS_LONE_BN - 1) / MS_LONE_BN) + ncu - 1) / ncu <= MS_MAXU &&
            p.grid_m <= MS_MAXE && p.sym % 8 == 0 &&
            reinterpret_cast<uintptr_t>(p.Y) % 16 == 0 &&
            (int64_t)p.T * p.xs_tok * 4 < (1ll << 31) && 256 * p.sym * 2 < (1ll << 31)) {
            auto skern = p.wt ? moe_stream_kernel<true> : moe_stream_kernel<false>;
            static bool sattr[2] = {false, false};
            if (!sattr[p.wt]) {
                hipError_t e =
                    hipFuncSetAttribute((const void*)skern, hipFuncAttributeMaxDynamicSharedMemorySize, MS_LDS);
                if (e != hipSuccess) {
                    set_error("hipFuncSetAttribute(MaxDynamicSharedMemorySize=%d) failed: %s", MS_LDS,
                              hipGetErrorString(e));
                    return (int)e;
                }
                sattr[p.wt] = true;
            }
            // walk groups of four pairs with the XCD-aligned walk (Mixtral
            // gate/up, 112 column tiles: 0.920 -> 0.912 ms against two; one
            // took 0.918 against 0.899), one pair where the columns are too
            // few for it (down, 16 column tiles: 0.477 -> 0.464 ms against two)
            if (group_default) p.group_m = p.xcd_cols ? 4 : 1;
            skern<<<dim3((unsigned)ncu), 64 * MOE_WM * MOE_WN, MS_LDS, stream>>>(p);
            return hkq_launch_status();
        }
    }
    kern<<<dim3((unsigned)nblk), 64 * MOE_WM * MOE_WN, LDS, stream>>>(p);
    return hkq_launch_status();
}

// ---------------------------------------------------------------------------
// MXFP4 MoE GEMM over the block-sorted routing of moe_align_block_size
// (moe-gemm/moe_op_mxfp4/kernel.cpp:90-237): tile row r of 128-row block pm
// is gate id = sorted_token_ids[pm*128 + r] (valid when < num_valid_tokens),
// its A row is id / top_k, its expert expert_ids[pm] (-1: the block's valid
// rows are written as zeros), and
//   C[id, n] = bf16((sum_k A[id/topk, k] B[e, n, k]) * a_scale[0] * b_scale[e]
//                   * (mul_routed_weight ? topk_weights[id] : 1))
// with A, B E2M1 pairs and e8m0 scales per 32 K values on both. Output rows
// are written at the gate id (the reference's C[token_id]).
// ---------------------------------------------------------------------------
struct MoeFp4Params {
    const uint8_t* A;       // [tokens, sam] bytes, K/2 used
    const uint8_t* As;      // [tokens, sas] e8m0, K/32 used
    const uint8_t* B;       // expert e at B + e*sbe, row n at + n*sbn (K/2 bytes); wt: row kk of
                            // K/2 at + kk*sbn (N bytes)
    const uint8_t* Bs;      // expert e at Bs + e*sbse, row n at + n*sbsn (K/32 bytes); wt: row of 32
                            // values of K at + (k/32)*sbsn (N bytes)
    uint16_t* C;            // row id at C + id*scm
    const float* a_scale;   // nullptr: 1
    const float* b_scale;   // nullptr: 1
    const float* topk_w;    // nullptr: no routed weight
    const int32_t* sorted;  // [grid_m * 128]
    const int32_t* expert;  // [grid_m]
    int tokens, E, N, K, topk, num_valid, grid_m, tiles_n, group_m, c16;
    double rtopk;  // 1.0 / topk (div_recip)
    int split;     // tiles of the last round cut into their two blocks (pair_unit)
    int xcd_cols;  // pair_walk's column order
    int64_t sam, sas, sbe, sbn, sbse, sbsn, scm;
    int wt;  // B and Bs N-contiguous ([K/2, N] and [K/32, N] per expert)
};

constexpr uint32_t FP4_OOB = 0x7FFF0000u;  // a row offset past every operand's bounds

// Rows [pm*128, pm*128 + TM*64) of the sorted routing (one block, or two
// consecutive blocks of expert e) times columns [n0, n0 + 256), expert e >= 0.
template <int TM, int KTB, int NS, bool BT = false>
__device__ __forceinline__ void moe_fp4_block(const MoeFp4Params& p, int pm, int e, int n0, HKQ_LDS uint8_t* smem) {
    constexpr int TN = MOE_TN;
    using Cfg = DenseCfg<MODE_MXFP4, MOE_WM, MOE_WN, TM, TN, KTB>;
    constexpr int NW = Cfg::NW, BM = Cfg::BM, BN = Cfg::BN, LA = Cfg::LA, LB = Cfg::LB;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / MOE_WN, wn = wave % MOE_WN;
    const int nw = n0 + wn * TN * 32;
    const int32_t* ids = p.sorted + (int64_t)pm * MOE_BM;
    // gate id of tile row r, or -1 when it is padding
    auto gate_of = [&](int r) {
        const int id = ids[r];
        return (id >= 0 && id < p.num_valid) ? id : -1;
    };
    // A row of tile row r, or -1 (padding, or a row past the activations)
    auto arow_of = [&](int r) {
        const int id = gate_of(r);
        const int t = id < 0 ? -1 : div_recip(id, p.rtopk);
        return t < p.tokens ? t : -1;
    };

    const int rows_b = min(p.N - n0, BN);
    LoopSrc src;
    src.a = p.A;
    src.a_bytes = min((int64_t)p.tokens * p.sam, (int64_t)FP4_OOB);
    src.as = p.As;
    src.as_bytes = min((int64_t)p.tokens * p.sas, (int64_t)FP4_OOB);
    if constexpr (BT) {
        // N-contiguous weights and scales: the tile's columns of every row
        // (columns past N read the next row's bytes, which only reach output
        // columns that are never stored)
        src.b = p.B + (int64_t)e * p.sbe + n0;
        src.b_bytes = min((int64_t)(p.K / 2 - 1) * p.sbn + rows_b, (int64_t)FP4_OOB);
        src.b_kstep = (int64_t)KTB * p.sbn;
        src.bs = p.Bs + (int64_t)e * p.sbse + n0;
        src.bs_bytes = min((int64_t)(p.K / 32 - 1) * p.sbsn + rows_b, (int64_t)FP4_OOB);
    } else {
        src.b = p.B + (int64_t)e * p.sbe + (int64_t)n0 * p.sbn;
        src.b_bytes = min((int64_t)rows_b * p.sbn, (int64_t)FP4_OOB);
        src.bs = p.Bs + (int64_t)e * p.sbse + (int64_t)n0 * p.sbsn;
        src.bs_bytes = min((int64_t)rows_b * p.sbsn, (int64_t)FP4_OOB);
    }
    src.lsa = p.sas;
    src.lsb = p.sbsn;
    src.KT = (p.K / 2) / KTB;
    // the A scale rows this lane loads (the main loop's slot order): 128-byte
    // K-tiles: row g*32 + lane/2 of group g = (k*NW + wave) % SB_GROUPS for
    // slot k; 64-byte K-tiles: row g*64 + lane of group g = (k*NW + wave) % GA
    src.sa_gathered = true;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        int r;
        if constexpr (Cfg::SBLK) {
            const int g = (k * NW + wave) % Cfg::SB_GROUPS;
            r = g * 32 < BM ? g * 32 + (lane >> 1) : -1;
        } else {
            r = k < Cfg::LSA ? ((k * NW + wave) % Cfg::GA) * 64 + lane : -1;
        }
        const int t = r < 0 ? -1 : arow_of(r);
        src.sa_row[k] = t < 0 ? FP4_OOB : (uint32_t)(t * p.sas);
    }
    TableOff<LA> a_off;
#pragma unroll
    for (int i = 0; i < LA; ++i) {
        const int r = (i * NW + wave) * Cfg::RPL + lane / Cfg::KT::CHUNKS;
        const int t = arow_of(r);
        a_off.v[i] = t < 0 ? FP4_OOB : (uint32_t)(t * p.sam) + (uint32_t)(Cfg::KT::load_chunk(lane, r) << 4);
    }
    TableOff<LB> b_off;
    if constexpr (BT) b_off = dense_offs_t<NW, LB>(wave, lane, p.sbn);
    else b_off = dense_offs<NW, KTB, LB>(wave, lane, p.sbn);

    // the epilogue's row scales (routed weights), fetched before the K loop
    const float gs = (p.a_scale ? p.a_scale[0] : 1.0f) * (p.b_scale ? p.b_scale[e] : 1.0f);
    float rs[TM];
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int id = gate_of(wm * TM * 32 + j * 32 + (lane & 31));
        rs[j] = (p.topk_w && id >= 0) ? gs * p.topk_w[id] : gs;
    }

    v16f acc[TN][TM];
    gemm_mainloop<MODE_MXFP4, MOE_WM, MOE_WN, TM, TN, KTB, NS, BT>(src, a_off, b_off, smem, lane, wave, acc);

    // The output rows (gate ids) of the wave's TM*32 rows, loaded before the
    // staging so that the store loop takes them from registers: a global load
    // per pass of rows there held every pass up (measured on MI355X, Mixtral
    // gate/up: 9.7 us per 256-row tile's epilogue).
    int rid[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) rid[h] = h * 64 < TM * 32 ? gate_of(wm * TM * 32 + h * 64 + lane) : -1;
    store_tile_bf16_rows<TM, TN>(
        acc, smem, wave, lane, p.C, p.scm, p.N, nw, p.c16 != 0,
        [&](int r) { return (int64_t)__shfl(r < 64 ? rid[0] : rid[1], r & 63); }, [&](int j) { return rs[j]; },
        [&](int, int) { return make_float4(1.f, 1.f, 1.f, 1.f); }, NoBias{});
}

// The valid rows of block pm, whose expert id is -1, are written as zeros (as
// the reference does); columns [n0, n0 + 256).
__device__ __forceinline__ void moe_fp4_zero_block(const MoeFp4Params& p, int pm, int n0) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int32_t* ids = p.sorted + (int64_t)pm * MOE_BM;
    for (int r = wave; r < MOE_BM; r += 4) {
        const int id = ids[r];
        if (id < 0 || id >= p.num_valid) continue;
        for (int n = n0 + lane * 4; n < min(p.N, n0 + MOE_BN); n += 256)
            *reinterpret_cast<v2i*>(p.C + (int64_t)id * p.scm + n) = v2i{0, 0};
    }
}

// Workgroup: routing blocks (2q, 2q + 1) x column tile tn; two blocks of one
// expert form one 256-row tile, otherwise each block is its own 128-row tile
// (64 rows when its upper half is padding; with expert -1, zeros). Tile
// order: pair_walk, one pair at a time.
template <int KTB, int NS, bool BT = false>
__global__ __launch_bounds__(64 * MOE_WM * MOE_WN, 1) void moe_mxfp4_kernel(const MoeFp4Params p) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;
    int q, tn, half;
    if (!pair_unit(blockIdx.x, (p.grid_m + 1) / 2, p.tiles_n, p.group_m, p.xcd_cols, p.split, q, tn, half)) return;
    const int n0 = tn * MOE_BN;
    const int pm0 = 2 * q, pm1 = 2 * q + 1;
    const int e0 = p.expert[pm0], e1 = pm1 < p.grid_m ? p.expert[pm1] : -2;
    if (half < 0 && e0 >= 0 && e0 < p.E && e1 == e0) {
        moe_fp4_block<4, KTB, NS, BT>(p, pm0, e0, n0, smem);
        return;
    }
    // the pair's blocks one at a time (both, or the one this unit was given);
    // expert -1: zeros; an expert id past E: nothing to compute or write
    const int h0 = half < 0 ? 0 : half, h1 = half < 0 ? 1 : half;
#pragma unroll 1
    for (int h = h0; h <= h1; ++h) {
        const int pm = pm0 + h;
        if (pm >= p.grid_m) break;
        const int e = p.expert[pm];
        if (e == -1) {
            moe_fp4_zero_block(p, pm, n0);
        } else if (e >= 0 && e < p.E) {
            __syncthreads();  // every wave is done with an earlier block's epilogue staging
            // entries 64..127 all padding (an expert's last block): a 64-row
            // tile (every wave reads the same 64 entries: a uniform choice)
            const int id = p.sorted[(int64_t)pm * MOE_BM + MOE_BM / 2 + (threadIdx.x & 63)];
            if (__ballot(id >= 0 && id < p.num_valid) == 0)
                moe_fp4_block<1, KTB, NS, BT>(p, pm, e, n0, smem);
            else
                moe_fp4_block<2, KTB, NS, BT>(p, pm, e, n0, smem);
        }
    }
}

// ---------------------------------------------------------------------------
// Decode-size MXFP4 MoE (at most 32 valid gate ids): the streaming layout of
// the narrow GEMM. Workgroup u takes block u / slices and the 16*NT columns of
// slice u % slices; for every 16-entry group of the block that holds a valid
// gate id (with the sorted layout that is the first one or two groups) its 4
// waves stream K through the 16x16x128 MFMA with per-lane e8m0 scales (lane l:
// entry l % 16 of the group, bytes [16q, 16q+16) of a 64-byte K-step and the
// scale byte q of the step's 4 blocks, q = l/16). Blocks of expert -1 write
// zeros to their valid rows, as the tiled kernel does.
constexpr int MOE_FP4_NARROW_MAX_VALID = 32;

template <int NT>
__global__ __launch_bounds__(64 * MOE_NARROW_WAVES) void moe_fp4_narrow_kernel(const MoeFp4Params p, int slices) {
    constexpr int DEPTH = NT >= 4 ? 4 : 8;
    __shared__ v4f red[MOE_NARROW_WAVES][NT][64];
    const int pm = blockIdx.x / slices, n0 = (blockIdx.x % slices) * 16 * NT;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int32_t* ids = p.sorted + (int64_t)pm * MOE_BM;
    const int e = p.expert[pm];
    if (e < 0 || e >= p.E) {
        if (e < 0) {  // valid rows of an unassigned block are zeros
            for (int rr = threadIdx.x; rr < MOE_BM; rr += 64 * MOE_NARROW_WAVES) {
                const int id = ids[rr];
                if (id < 0 || id >= p.num_valid) continue;
                for (int n = n0; n < min(p.N, n0 + 16 * NT); n += 4)
                    *reinterpret_cast<v2i*>(p.C + (int64_t)id * p.scm + n) = v2i{0, 0};
            }
        }
        return;
    }
    const int S = p.K / 128;  // 64-byte K-steps
    const int s0 = wave * S / MOE_NARROW_WAVES, s1 = (wave + 1) * S / MOE_NARROW_WAVES;
    const int rows_b = min(16 * NT, p.N - n0);
    const auto rb = make_rsrc(p.B + (int64_t)e * p.sbe + (int64_t)n0 * p.sbn, (uint32_t)(rows_b * p.sbn));
    const auto rbs = make_rsrc(p.Bs + (int64_t)e * p.sbse + (int64_t)n0 * p.sbsn, (uint32_t)(rows_b * p.sbsn));
    const auto ra = make_rsrc(p.A, (uint32_t)((int64_t)p.tokens * p.sam));
    const auto ras = make_rsrc(p.As, (uint32_t)((int64_t)p.tokens * p.sas));
    uint32_t b_off[NT], bs_off[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        b_off[i] = (uint32_t)((i * 16 + r) * p.sbn + 16 * q);
        bs_off[i] = (uint32_t)((i * 16 + r) * p.sbsn);
    }
    const float gs = (p.a_scale ? p.a_scale[0] : 1.0f) * (p.b_scale ? p.b_scale[e] : 1.0f);

    for (int g = 0; g < MOE_BM / 16; ++g) {
        const int id0 = ids[g * 16 + r];
        const int id = (id0 >= 0 && id0 < p.num_valid) ? id0 : -1;
        if (__builtin_amdgcn_ballot_w64(id >= 0) == 0) continue;  // uniform: no valid entry in the group
        const int tk = id < 0 ? -1 : div_recip(id, p.rtopk);
        const bool live = tk >= 0 && tk < p.tokens;
        // Offsets stay below 2^32: valid ones are below 2^31, an invalid row's
        // is OOB itself, and the K part is below 2^31.
        const uint32_t a_off = live ? (uint32_t)(tk * p.sam + 16 * q) : OOB;
        const uint32_t as_off = live ? (uint32_t)(tk * p.sas) : OOB;
        struct Frag {
            v4i b[NT], a;
            uint32_t sb[NT], sa;
        };
        auto load = [&](int s, Frag& f) {
            const uint32_t kb = (uint32_t)s * 64, ks = (uint32_t)s * 4, kill = s < s1 ? 0u : OOB;
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                f.b[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, (b_off[i] + kb) | kill, 0, 0);
                f.sb[i] = __builtin_amdgcn_raw_buffer_load_b32(rbs, (bs_off[i] + ks) | kill, 0, 0);
            }
            f.a = __builtin_amdgcn_raw_buffer_load_b128(ra, (a_off + kb) | kill, 0, 0);
            f.sa = __builtin_amdgcn_raw_buffer_load_b32(ras, (as_off + ks) | kill, 0, 0);
        };
        v4f acc[NT];
#pragma unroll
        for (int i = 0; i < NT; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
        auto mma = [&](const Frag& f) {
            const v8i bb = v8i{f.a[0], f.a[1], f.a[2], f.a[3], 0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                const v8i aa = v8i{f.b[i][0], f.b[i][1], f.b[i][2], f.b[i][3], 0, 0, 0, 0};
                acc[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(aa, bb, acc[i], 4, 4, 0, (int)(f.sb[i] >> (8 * q)),
                                                                          0, (int)(f.sa >> (8 * q)));
            }
        };
        Frag f[DEPTH];
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) load(s0 + d, f[d]);
        for (int s = s0; s < s1; s += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                mma(f[d]);
                load(s + d + DEPTH, f[d]);
            }
        }
        __syncthreads();  // the previous group's sums have been read
#pragma unroll
        for (int i = 0; i < NT; ++i) red[wave][i][lane] = acc[i];
        __syncthreads();
        if (wave == 0 && id >= 0) {
            const float rs = p.topk_w ? gs * p.topk_w[id] : gs;
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                const int n = n0 + 16 * i + 4 * q;
                if (n >= p.N) break;  // N % 4 == 0: n .. n+3 all in or all out
                v4f v = red[0][i][lane];
#pragma unroll
                for (int w = 1; w < MOE_NARROW_WAVES; ++w) v += red[w][i][lane];
                *reinterpret_cast<v2i*>(p.C + (int64_t)id * p.scm + n) =
                    v2i{(int)pk_bf16(v[0] * rs, v[1] * rs), (int)pk_bf16(v[2] * rs, v[3] * rs)};
            }
        }
    }
}

static int launch_moe_fp4_narrow(const MoeFp4Params& p, hipStream_t stream) {
    if (p.grid_m == 0 || p.N == 0) return 0;
    const int threads = 64 * MOE_NARROW_WAVES;
    if (p.N > 4096) {
        const int slices = (p.N + 63) / 64;
        moe_fp4_narrow_kernel<4><<<dim3((unsigned)((int64_t)p.grid_m * slices)), threads, 0, stream>>>(p, slices);
    } else {
        const int slices = (p.N + 15) / 16;
        moe_fp4_narrow_kernel<1><<<dim3((unsigned)((int64_t)p.grid_m * slices)), threads, 0, stream>>>(p, slices);
    }
    return hkq_launch_status();
}

template <int KTB, int NS>
static int launch_moe_fp4(MoeFp4Params& p, hipStream_t stream) {
    using Whole = DenseCfg<MODE_MXFP4, MOE_WM, MOE_WN, 4, MOE_TN, KTB>;
    using Half = DenseCfg<MODE_MXFP4, MOE_WM, MOE_WN, 2, MOE_TN, KTB>;
    constexpr int LDS = Whole::lds_bytes(NS) > Half::lds_bytes(NS) ? Whole::lds_bytes(NS) : Half::lds_bytes(NS);
    static_assert(LDS <= 160 * 1024, "LDS budget of a CDNA4 CU");
    // N-contiguous weights (wt) need 128-byte K-tiles (the entry point checks)
    auto kern = moe_mxfp4_kernel<KTB, NS>;
    if constexpr (KTB == 128)
        if (p.wt) kern = moe_mxfp4_kernel<KTB, NS, true>;
    static bool attr_set[2] = {false, false};
    if (!attr_set[p.wt]) {
        hipError_t err = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
        if (err != hipSuccess) {
            set_error("hipFuncSetAttribute(MaxDynamicSharedMemorySize=%d) failed: %s", LDS, hipGetErrorString(err));
            return (int)err;
        }
        attr_set[p.wt] = true;
    }
    p.tiles_n = (p.N + MOE_BN - 1) / MOE_BN;
    if (p.group_m <= 0) p.group_m = 1;
    p.xcd_cols = moe_xcd_cols(p.tiles_n);
    const int64_t tiles = (int64_t)((p.grid_m + 1) / 2) * p.tiles_n;
    if (tiles == 0) return 0;
    p.split = (int)moe_tail_split(tiles);
    const int64_t nblk = tiles + p.split;
    kern<<<dim3((unsigned)nblk), 64 * MOE_WM * MOE_WN, LDS, stream>>>(p);
    return hkq_launch_status();
}

}  // namespace hkq

using namespace hkq;

// wt == 0: W[e] is [N, K] with row stride stride_w (K contiguous); wt == 1:
// W[e] is [K, N] with row stride stride_w (N contiguous, the reference's layout).
static int moe_a8w8_impl(const void* X, const void* W, void* Y, const float* x_scale, int64_t xs_stride_tok,
                         const float* w_scale, int64_t ws_stride_e, int64_t ws_stride_n, int64_t ws_group_n,
                         const float* bias, int64_t bias_stride_e, const int32_t* gather, const int32_t* hist,
                         const int32_t* offs, const int32_t* expt_data, int64_t T, int64_t E, int64_t N, int64_t K,
                         int64_t grid_m, int64_t topk, int64_t stride_xm, int64_t stride_we, int64_t stride_w, int wt,
                         int64_t stride_ym, int64_t y_rows, int64_t gather_len, hipStream_t stream) {
    HKQ_CHECK_ARG(T >= 0 && E > 0 && E <= 0xFFFF && N >= 0 && K > 0 && grid_m >= 0 && topk > 0 && topk <= 0xFFFF,
                  "T, grid_m >= 0; 0 < E <= 65535; K > 0; 0 < topk <= 65535");
    HKQ_CHECK_ARG(T < (1 << 30) && N < (1 << 30) && K < (1 << 30) && grid_m < (1 << 30), "dimensions must be < 2^30");
    HKQ_CHECK_ARG(K % 64 == 0, "K must be a multiple of 64");
    HKQ_CHECK_ARG(N % 4 == 0, "N must be a multiple of 4");
    HKQ_CHECK_ARG(stride_xm >= K && stride_xm % 16 == 0, "stride_xm must be >= K and a multiple of 16");
    // the kernels address gathered X rows with 32-bit buffer offsets
    HKQ_CHECK_ARG(T * stride_xm < (1ll << 31), "X must span less than 2^31 bytes (T * stride_xm)");
    if (wt) {
        HKQ_CHECK_ARG(K % 128 == 0, "N-contiguous weights need K to be a multiple of 128");
        HKQ_CHECK_ARG(stride_w >= N && stride_w % 16 == 0, "stride_wk must be >= N and a multiple of 16 (W[e] is [K, N])");
        HKQ_CHECK_ARG(K * stride_w < (1ll << 31), "one expert's weights must span less than 2^31 bytes (K * stride_wk)");
    } else {
        HKQ_CHECK_ARG(stride_w >= K && stride_w % 16 == 0, "stride_wn must be >= K and a multiple of 16 (W[e] is [N, K])");
    }
    HKQ_CHECK_ARG(stride_we >= 0 && stride_we % 16 == 0, "stride_we must be a non-negative multiple of 16");
    HKQ_CHECK_ARG(stride_ym >= N && stride_ym % 4 == 0, "stride_ym must be >= N and a multiple of 4");
    HKQ_CHECK_ARG(ws_group_n >= 1, "ws_group_n must be >= 1");
    HKQ_CHECK_ARG(xs_stride_tok >= 0, "xs_stride_tok must be >= 0");
    HKQ_CHECK_ARG(y_rows >= 0 && gather_len >= 0, "y_rows and gather_len must be >= 0");
    HKQ_CHECK_ARG(hist && offs && expt_data, "routing metadata pointers must not be null");
    HKQ_CHECK_ALIGN(X, 16);
    HKQ_CHECK_ALIGN(W, 16);
    HKQ_CHECK_ALIGN(Y, 8);
    MoeParams p{};
    p.X = static_cast<const uint8_t*>(X);
    p.W = static_cast<const uint8_t*>(W);
    p.Y = static_cast<uint16_t*>(Y);
    p.xs = x_scale;
    p.ws = w_scale;
    p.bias = bias;
    p.gather = gather;
    p.hist = hist;
    p.offs = offs;
    p.expt_data = expt_data;
    p.T = (int)T; p.E = (int)E; p.N = (int)N; p.K = (int)K; p.topk = (int)topk; p.rtopk = 1.0 / (double)topk; p.grid_m = (int)grid_m;
    p.y_rows = (int)y_rows;
    p.g_len = gather ? (int)gather_len : (int)y_rows;
    p.sxm = stride_xm; p.swe = stride_we; p.sym = stride_ym;
    p.wt = wt;
    p.swn = wt ? 1 : stride_w;
    p.swk = wt ? stride_w : 1;
    p.xs_tok = xs_stride_tok; p.ws_e = ws_stride_e; p.ws_n = ws_stride_n; p.bias_e = bias_stride_e;
    p.ws_gn = std::min<int64_t>(ws_group_n, std::max<int64_t>(N, 1));  // same quotients for n < N, 32-bit
    p.ws_vec = w_scale && ws_stride_n == 1 && ws_group_n == 1 && ws_stride_e % 4 == 0 &&
               reinterpret_cast<uintptr_t>(w_scale) % 16 == 0;
    p.bias_vec = bias && bias_stride_e % 4 == 0 && reinterpret_cast<uintptr_t>(bias) % 16 == 0;
    p.c16 = (stride_ym % 8 == 0) && (reinterpret_cast<uintptr_t>(Y) % 16 == 0);
    // Decode sizes take the streaming path: at most 32 routed rows, or 64 with
    // N <= 4096 (measured: with 64 rows and N = 28672 the tiled kernel is 8%
    // faster, at N = 4096 the streaming one 1.9x). The routed rows are the
    // gathered (token, choice) pairs, T * topk, or the T sorted rows without
    // a gather; every block then holds at most that many rows.
    const int64_t routed = gather ? T * topk : T;
    const bool decode = routed <= 32 || (routed <= MOE_NARROW_MAX_ROWS && N <= 4096);
    if (decode && !wt && K % 128 == 0 && 64 * stride_w < (1ll << 31))
        return launch_moe_narrow(p, routed, stream);
    // 128-byte K-tiles (2-stage ring) when every row has whole ones: a partial
    // last K-tile would read the next row's bytes instead of zeros
    return K % 128 == 0 ? launch_moe<128, 2>(p, stream) : launch_moe<64, 4>(p, stream);
}

extern "C" int hkq_moe_a8w8(const void* X, const void* W, void* Y, const float* x_scale, int64_t xs_stride_tok,
                            const float* w_scale, int64_t ws_stride_e, int64_t ws_stride_n, int64_t ws_group_n,
                            const float* bias, int64_t bias_stride_e, const int32_t* gather, const int32_t* hist,
                            const int32_t* offs, const int32_t* expt_data, int64_t T, int64_t E, int64_t N,
                            int64_t K, int64_t grid_m, int64_t topk, int64_t stride_xm, int64_t stride_we,
                            int64_t stride_wn, int64_t stride_ym, int64_t y_rows, int64_t gather_len,
                            hipStream_t stream) {
    return moe_a8w8_impl(X, W, Y, x_scale, xs_stride_tok, w_scale, ws_stride_e, ws_stride_n, ws_group_n, bias,
                         bias_stride_e, gather, hist, offs, expt_data, T, E, N, K, grid_m, topk, stride_xm, stride_we,
                         stride_wn, 0, stride_ym, y_rows, gather_len, stream);
}

extern "C" int hkq_moe_a8w8_kn(const void* X, const void* W, void* Y, const float* x_scale, int64_t xs_stride_tok,
                               const float* w_scale, int64_t ws_stride_e, int64_t ws_stride_n, int64_t ws_group_n,
                               const float* bias, int64_t bias_stride_e, const int32_t* gather, const int32_t* hist,
                               const int32_t* offs, const int32_t* expt_data, int64_t T, int64_t E, int64_t N,
                               int64_t K, int64_t grid_m, int64_t topk, int64_t stride_xm, int64_t stride_we,
                               int64_t stride_wk, int64_t stride_ym, int64_t y_rows, int64_t gather_len,
                               hipStream_t stream) {
    return moe_a8w8_impl(X, W, Y, x_scale, xs_stride_tok, w_scale, ws_stride_e, ws_stride_n, ws_group_n, bias,
                         bias_stride_e, gather, hist, offs, expt_data, T, E, N, K, grid_m, topk, stride_xm, stride_we,
                         stride_wk, 1, stride_ym, y_rows, gather_len, stream);
}

// wt == 0: B[e] [N, K/2] (row stride stride_b) and B_mx_scale[e] [N, K/32]
// (row stride stride_bmx), K contiguous; wt == 1: B[e] [K/2, N] and
// B_mx_scale[e] [K/32, N], N contiguous (the reference's layout).
static int moe_mxfp4_impl(const void* A, const void* B, void* C, const void* A_mx_scale, const void* B_mx_scale,
                          const float* A_scale, const float* B_scale, const float* topk_weights,
                          const int32_t* sorted_token_ids, const int32_t* expert_ids, int64_t N, int64_t K,
                          int64_t num_valid_tokens, int64_t top_k, int mul_routed_weight, int64_t stride_am,
                          int64_t stride_be, int64_t stride_bn, int64_t stride_cm, int64_t stride_amxm,
                          int64_t stride_bmxe, int64_t stride_bmxn, int64_t num_tokens, int64_t num_experts,
                          int64_t grid_m, int wt, hipStream_t stream) {
    HKQ_CHECK_ARG(N >= 0 && K > 0 && num_valid_tokens >= 0 && top_k > 0 && top_k <= 0xFFFF && num_tokens >= 0 &&
                      num_experts > 0 && grid_m >= 0,
                  "N, num_valid_tokens, num_tokens, grid_m >= 0; K, num_experts > 0; 0 < top_k <= 65535");
    HKQ_CHECK_ARG(N < (1 << 30) && K < (1 << 30) && grid_m < (1 << 22) && num_tokens < (1 << 30) &&
                      num_valid_tokens < (1 << 30),
                  "dimensions out of range");
    HKQ_CHECK_ARG(K % 128 == 0, "K must be a multiple of 128 (64 bytes of E2M1 pairs)");
    HKQ_CHECK_ARG(N % 4 == 0, "N must be a multiple of 4");
    HKQ_CHECK_ARG(stride_am >= K / 2 && stride_am % 16 == 0, "stride_am must be >= K/2 bytes and a multiple of 16");
    if (wt) {
        HKQ_CHECK_ARG(K % 256 == 0, "N-contiguous weights need K to be a multiple of 256");
        HKQ_CHECK_ARG(stride_bn >= N && stride_bn % 16 == 0,
                      "stride_bk must be >= N and a multiple of 16 (B[e] is [K/2, N], N contiguous)");
        HKQ_CHECK_ARG(stride_bmxn >= N && stride_bmxn % 16 == 0,
                      "stride_bmxk must be >= N and a multiple of 16 (B_mx_scale[e] is [K/32, N])");
        HKQ_CHECK_ARG((K / 2) * stride_bn < (int64_t)FP4_OOB && (K / 32) * stride_bmxn < (int64_t)FP4_OOB,
                      "one expert's weights and scales must span less than 2^31 - 2^16 bytes");
        HKQ_CHECK_ARG(stride_bmxe % 16 == 0 && reinterpret_cast<uintptr_t>(B_mx_scale) % 16 == 0,
                      "N-contiguous weight scales: B_mx_scale 16-byte aligned, stride_bmxe a multiple of 16");
    } else {
        HKQ_CHECK_ARG(stride_bn >= K / 2 && stride_bn % 16 == 0,
                      "stride_bn must be >= K/2 bytes and a multiple of 16 (B[e] is [N, K/2], K contiguous)");
    }
    HKQ_CHECK_ARG(stride_be >= 0 && stride_be % 16 == 0, "stride_be must be a non-negative multiple of 16");
    HKQ_CHECK_ARG(stride_amxm >= K / 32 && (wt || stride_bmxn >= K / 32) && stride_bmxe >= 0,
                  "scale strides must cover K/32 bytes per row (scales [rows, K/32], K contiguous)");
    HKQ_CHECK_ARG((K / 2) % 128 == 0 || (stride_amxm % 4 == 0 && stride_bmxn % 4 == 0),
                  "with K % 256 != 0 the scale row strides must be multiples of 4");
    HKQ_CHECK_ARG((int64_t)num_tokens * stride_am < (int64_t)FP4_OOB &&
                      (int64_t)num_tokens * stride_amxm < (int64_t)FP4_OOB,
                  "the activations must span less than 2^31 - 2^16 bytes");
    HKQ_CHECK_ARG(stride_cm >= N && stride_cm % 4 == 0, "stride_cm must be >= N and a multiple of 4");
    HKQ_CHECK_ARG(grid_m == 0 || (sorted_token_ids && expert_ids), "sorted_token_ids and expert_ids are required");
    HKQ_CHECK_ARG(!mul_routed_weight || topk_weights, "topk_weights is required with mul_routed_weight");
    HKQ_CHECK_ALIGN(A, 16);
    HKQ_CHECK_ALIGN(B, 16);
    HKQ_CHECK_ALIGN(A_mx_scale, 4);
    HKQ_CHECK_ALIGN(B_mx_scale, 4);
    HKQ_CHECK_ALIGN(C, 8);
    MoeFp4Params p{};
    p.A = static_cast<const uint8_t*>(A);
    p.As = static_cast<const uint8_t*>(A_mx_scale);
    p.B = static_cast<const uint8_t*>(B);
    p.Bs = static_cast<const uint8_t*>(B_mx_scale);
    p.C = static_cast<uint16_t*>(C);
    p.a_scale = A_scale;
    p.b_scale = B_scale;
    p.topk_w = mul_routed_weight ? topk_weights : nullptr;
    p.sorted = sorted_token_ids;
    p.expert = expert_ids;
    p.tokens = (int)num_tokens; p.E = (int)num_experts; p.N = (int)N; p.K = (int)K; p.topk = (int)top_k; p.rtopk = 1.0 / (double)top_k;
    p.num_valid = (int)num_valid_tokens; p.grid_m = (int)grid_m;
    p.sam = stride_am; p.sas = stride_amxm; p.sbe = stride_be; p.sbn = stride_bn; p.sbse = stride_bmxe;
    p.sbsn = stride_bmxn; p.scm = stride_cm;
    p.wt = wt;
    p.c16 = (stride_cm % 8 == 0) && (reinterpret_cast<uintptr_t>(C) % 16 == 0);
    // The streaming path when the tiled grid would give fewer than a quarter
    // of the CUs work and there are at most 32 valid gate ids (measured: one
    // token's down projection, N = 4096, 56 -> 22 us; with N = 28672 or eight
    // tokens the tiled kernel is faster). Its scale loads are dwords, and 64
    // weight rows must span less than 2 GiB.
    const int64_t ncu = cu_count() > 0 ? cu_count() : 256;
    const bool few_tiles = ((grid_m + 1) / 2) * ((N + MOE_BN - 1) / MOE_BN) * 4 < ncu;
    if (!wt && few_tiles && num_valid_tokens <= MOE_FP4_NARROW_MAX_VALID && stride_amxm % 4 == 0 && stride_bmxn % 4 == 0 &&
        stride_bmxe % 4 == 0 && reinterpret_cast<uintptr_t>(A_mx_scale) % 4 == 0 &&
        reinterpret_cast<uintptr_t>(B_mx_scale) % 4 == 0 && 64 * stride_bn < (1ll << 31) && 64 * stride_bmxn < (1ll << 31))
        return launch_moe_fp4_narrow(p, stream);
    // 128-byte K-tiles when rows have whole ones (K % 256 == 0), else 64-byte ones
    return (K / 2) % 128 == 0 ? launch_moe_fp4<128, 2>(p, stream) : launch_moe_fp4<64, 4>(p, stream);
}

extern "C" int hkq_moe_mxfp4(const void* A, const void* B, void* C, const void* A_mx_scale, const void* B_mx_scale,
                             const float* A_scale, const float* B_scale, const float* topk_weights,
                             const int32_t* sorted_token_ids, const int32_t* expert_ids, int64_t N, int64_t K,
                             int64_t num_valid_tokens, int64_t top_k, int mul_routed_weight, int64_t stride_am,
                             int64_t stride_be, int64_t stride_bn, int64_t stride_cm, int64_t stride_amxm,
                             int64_t stride_bmxe, int64_t stride_bmxn, int64_t num_tokens, int64_t num_experts,
                             int64_t grid_m, hipStream_t stream) {
    return moe_mxfp4_impl(A, B, C, A_mx_scale, B_mx_scale, A_scale, B_scale, topk_weights, sorted_token_ids,
                          expert_ids, N, K, num_valid_tokens, top_k, mul_routed_weight, stride_am, stride_be, stride_bn,
                          stride_cm, stride_amxm, stride_bmxe, stride_bmxn, num_tokens, num_experts, grid_m, 0, stream);
}

extern "C" int hkq_moe_mxfp4_kn(const void* A, const void* B, void* C, const void* A_mx_scale,
                                const void* B_mx_scale, const float* A_scale, const float* B_scale,
                                const float* topk_weights, const int32_t* sorted_token_ids,
                                const int32_t* expert_ids, int64_t N, int64_t K, int64_t num_valid_tokens,
                                int64_t top_k, int mul_routed_weight, int64_t stride_am, int64_t stride_be,
                                int64_t stride_bk, int64_t stride_cm, int64_t stride_amxm, int64_t stride_bmxe,
                                int64_t stride_bmxk, int64_t num_tokens, int64_t num_experts, int64_t grid_m,
                                hipStream_t stream) {
    return moe_mxfp4_impl(A, B, C, A_mx_scale, B_mx_scale, A_scale, B_scale, topk_weights, sorted_token_ids,
                          expert_ids, N, K, num_valid_tokens, top_k, mul_routed_weight, stride_am, stride_be, stride_bk,
                          stride_cm, stride_amxm, stride_bmxe, stride_bmxk, num_tokens, num_experts, grid_m, 1, stream);
}
