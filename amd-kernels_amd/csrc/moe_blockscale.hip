// moe_blockscale.hip -- the block-scale A8W8 MoE grouped GEMM and the weight
// prepack that lets every MoE GEMM take the reference's weight layout.
//
// hkq_moe_a8w8_blockscale restates moe-gemm/moe_op_gemm_a8w8_blockscale/
// kernel.cpp:54-167 (per 64-deep K step: acc += isum * X_scale[tok, k/gk] *
// W_scale[e, k/gk, n/gn], :114-145) on E4M3FN codes:
//
//   Y[s, n] = bf16( sum_g (sum_{k in g} X[tok, k] W[e, n, k]) * xs[tok, g]
//                   * ws[e, g, n / group_n] + bias[e, n] ),   g = k / group_k
//
// for the OGS routing tiles ExptData[pm] = e | (b << 16), sorted row
// s = offs[e] + b*128 + r (r < hist[e] - b*128), tok = gather[s] / topk.
// group_k is a multiple of 64 (the reference's kernel is exact only then: it
// indexes the group once per 64-deep tile); group_n >= 1.
//
// fp32 group scales cannot ride in the MFMA's e8m0 operands, so every K-tile
// of one scale group is promoted on the VALU: acc += P * xs * ws, P the
// tile's partial of a 32x32 sub-tile. Two kernels:
//  - group_k = 128 * 2^j and K % 128 == 0: the 8-wave K loop of
//    blockscale_core.h (128-wide K-tiles, two MFMAs per partial) over
//    256 x 256 tiles that take two routing blocks of an expert at once;
//  - any other group_k (a multiple of 64): a workgroup computes one routing
//    block (128 rows) by 256 columns with 4 waves of 64 x 128; K-tiles are 64
//    bytes (one K-step, hence one scale group) in a 3-stage LDS ring, each
//    stage carrying the step's 128 row scales and 256 column scales next to
//    the operand rows. The ring (76.5 KB) lets two workgroups share a CU, so
//    one's VALU promotion runs beside the other's MFMAs.
// Both gather the A rows per lane through the routing index (rows of other
// tokens never enter LDS) and fill LDS with buffer_load ... lds.
//
// hkq_moe_pack_kmajor transposes [E, R, N] byte planes (N contiguous: the
// reference's MoE weights [E, K, N], MXFP4 weights [E, K/2, N] and e8m0 weight
// scales [E, K/32, N], tests/test_moe.py:723-729, 808-815, 909-925) into the
// K-contiguous [E, N, R] rows the MoE kernels stream into LDS.
#include "blockscale_core.h"
#include "hkq_host.h"

#include <cstdlib>

namespace hkq {

// ---------------------------------------------------------------------------
// Prepack: dst[e][n][r] = src[e][r][n] over 64 x 64 byte tiles staged in LDS.
// ---------------------------------------------------------------------------
constexpr int PK_T = 64, PK_PITCH = PK_T + 4;

__global__ __launch_bounds__(256) void pack_kmajor_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                          int R, int N, int64_t sse, int64_t ssr, int64_t dse,
                                                          int64_t dsn, int vec) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[PK_T * PK_PITCH];
    const int64_t e = blockIdx.z;
    const int r0 = blockIdx.y * PK_T, n0 = blockIdx.x * PK_T;
    const int t = threadIdx.x;
    {
        // thread t reads 16 bytes of source row r0 + t/4 at column n0 + (t%4)*16
        const int rl = t >> 2, cl = (t & 3) * 16;
        const int r = r0 + rl, c = n0 + cl;
        const uint8_t* s = src + e * sse + (int64_t)r * ssr + c;
        uint32_t w[4] = {0u, 0u, 0u, 0u};
        if (r < R) {
            if (vec && c + 16 <= N) {
                const uint4 v = *reinterpret_cast<const uint4*>(s);
                w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
            } else {
#pragma unroll
                for (int b = 0; b < 16; ++b)
                    if (c + b < N) w[b >> 2] |= (uint32_t)s[b] << (8 * (b & 3));
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) *reinterpret_cast<uint32_t*>(tile + rl * PK_PITCH + cl + 4 * q) = w[q];
    }
    __syncthreads();
    {
        // thread t writes 16 bytes of destination row n0 + t/4 at column r0 + (t%4)*16
        const int nl = t >> 2, rc = (t & 3) * 16;
        const int n = n0 + nl, r = r0 + rc;
        if (n >= N) return;
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t x = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) x |= (uint32_t)tile[(rc + 4 * q + b) * PK_PITCH + nl] << (8 * b);
            w[q] = x;
        }
        uint8_t* d = dst + e * dse + (int64_t)n * dsn + r;
        if (vec && r + 16 <= R) {
            *reinterpret_cast<uint4*>(d) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
#pragma unroll
            for (int b = 0; b < 16; ++b)
                if (r + b < R) d[b] = (uint8_t)(w[b >> 2] >> (8 * (b & 3)));
        }
    }
}

// ---------------------------------------------------------------------------
// Block-scale MoE GEMM
// ---------------------------------------------------------------------------
struct MoeBsParams {
    const uint8_t* X;       // [T, sxm] E4M3FN, K contiguous
    const uint8_t* W;       // expert e at W + e*swe; wt == 0: row n at + n*swn, K contiguous;
                            // wt == 1 (N-contiguous [K, N]): row k at + k*swk
    uint16_t* Y;            // sorted row s at Y + s*sym
    const float* xs;        // X_scale (t, g) at t*xsm + g*xsk
    const float* ws;        // W_scale (e, g, c) at e*wse + g*wsk + c*wsn, c = n / gn
    const float* bias;      // nullptr: 0; else bias[e * bias_e + n]
    const int32_t* gather;  // nullptr: token = s
    const int32_t* hist;
    const int32_t* offs;
    const int32_t* expt_data;
    int T, E, N, K, topk, grid_m, y_rows, g_len, gk, gn, tiles_n, c16;
    double rtopk;  // 1.0 / topk (div_recip)
    int64_t sxm, swe, swn, sym, xsm, xsk, wse, wsk, wsn, bias_e;
    int64_t xs_elems, ws_elems;  // reads of the scale tensors stay below these extents
    int64_t swk;
    int wt;
    int ncu;  // CUs of the device (0: no tail split)
};

// Word index from which ExptData entries compute their own 128-row block
// instead of pairing with the next: when the grid's 256-row tiles (one per
// block pair or lone block, per column tile) come to fewer than 4 rounds and
// leave a last round that fills at most half of the CUs, that round's tiles
// are cut in two (measured on MI355X, Mixtral down, 592 tiles: 0.701 ->
// 0.671 ms; with 16 rounds, gate/up, the cut made it slower). Counted per
// workgroup from the expert histogram (the valid entries are the first
// sum(ceil(hist / 128)), in expert order); it moves work between workgroups,
// never changes which rows are computed.
__device__ __forceinline__ int bs_tail_from(const MoeBsParams& p) {
    if (p.ncu <= 0) return p.grid_m;
    const int lane = threadIdx.x & 63;
    int nb = 0, un = 0;
    for (int x = lane; x < p.E; x += 64) {
        const int h = p.hist[x];
        const int b = h > 0 ? (h + 127) / 128 : 0;
        nb += b;
        un += (b + 1) / 2;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        nb += __shfl_xor(nb, o);
        un += __shfl_xor(un, o);
    }
    const int last = (un * p.tiles_n) % p.ncu;
    if (un * p.tiles_n >= 4 * p.ncu || last == 0 || 2 * last > p.ncu) return p.grid_m;
    return max(0, min(nb, p.grid_m) - 2 * ((last + p.tiles_n - 1) / p.tiles_n));
}

// Word index of the li-th word that computes a tile, in word order (-1 past
// the last): a valid word (e < E) that is not the second word of a pair, the
// second word (e | (b+1) << 16, b even) following its pair's first one before
// tail_from. Every wave of the workgroup finds the same word, 512 words per
// step (8 consecutive words per lane, their loads issued together); the
// caller loads the first step's words (bs_words), ahead of the histogram
// loads that tail_from waits on.
constexpr int BS_LW = 8;
__device__ __forceinline__ void bs_words(const MoeBsParams& p, int m0, int (&ed)[BS_LW]) {
    const int mw = m0 + (int)(threadIdx.x & 63) * BS_LW;
#pragma unroll
    for (int k = 0; k < BS_LW; ++k) ed[k] = mw + k < p.grid_m ? p.expt_data[mw + k] : -1;
}
__device__ __forceinline__ int bs_leader(const MoeBsParams& p, int li, int tail_from, const int (&ed0)[BS_LW]) {
    constexpr int W = BS_LW;
    const int lane = threadIdx.x & 63;
    int base = 0, carry = -1;  // expt_data[m0 - 1]
    for (int m0 = 0; m0 < p.grid_m; m0 += 64 * W) {
        const int mw = m0 + lane * W;
        int ed[W];
        if (m0 == 0) {
#pragma unroll
            for (int k = 0; k < W; ++k) ed[k] = ed0[k];
        } else {
            bs_words(p, m0, ed);
        }
        const int up = __shfl(ed[W - 1], (lane + 63) & 63);
        uint32_t lead = 0;
#pragma unroll
        for (int k = 0; k < W; ++k) {
            const int prev = k > 0 ? ed[k - 1] : (lane == 0 ? carry : up);
            const bool valid = ed[k] >= 0 && (ed[k] & 0xFFFF) < p.E;
            const bool second = valid && ((ed[k] >> 16) & 1) && mw + k > 0 && mw + k < tail_from && prev == ed[k] - 0x10000;
            lead |= (valid && !second) ? 1u << k : 0u;
        }
        const int c = __popc(lead);
        int incl = c;  // inclusive prefix of the lanes' counts
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o);
            if (lane >= o) incl += v;
        }
        const int total = __shfl(incl, 63);
        if (li < base + total) {  // uniform
            const int excl = base + incl - c;
            const bool here = li >= excl && li < excl + c;
            int pos = -1;
            if (here) {
                uint32_t mk = lead;
                for (int q = 0; q < li - excl; ++q) mk &= mk - 1;
                pos = mw + __builtin_ctz(mk);
            }
            return __shfl(pos, __builtin_ctzll(__ballot(here)));
        }
        base += total;
        carry = __shfl(ed[W - 1], 63);
    }
    return -1;
}

// The expert's weight source of a tile at column n0: base, extent (bytes from
// the base; N-contiguous columns past N read the next row's bytes, which only
// reach output columns that are never stored) and the bytes from one K-tile of
// KTB values to the next.
struct MoeBsB {
    const uint8_t* base;
    int64_t bytes, kstep;
};
template <bool BT, int KTB>
__device__ __forceinline__ MoeBsB moe_bs_b(const MoeBsParams& p, int e, int n0, int rows_b) {
    if constexpr (BT)
        return MoeBsB{p.W + (int64_t)e * p.swe + n0, min((int64_t)(p.K - 1) * p.swk + rows_b, (int64_t)0x7FFFFFFF),
                      (int64_t)KTB * p.swk};
    else
        return MoeBsB{p.W + (int64_t)e * p.swe + (int64_t)n0 * p.swn, min((int64_t)rows_b * p.swn, (int64_t)0x7FFFFFFF),
                      (int64_t)KTB};
}
// Load offset of a wave's B load i (NW waves, KTB-byte K-tiles): K-major rows
// of KTB bytes, or (BT) 4 rows of K x 256 columns per load in KTileT order.
template <bool BT, int NW, int KTB>
__device__ __forceinline__ uint32_t moe_bs_b_off(const MoeBsParams& p, int i, int wave, int lane) {
    if constexpr (BT) {
        const int r = (i * NW + wave) * KTileT::ROWS_PER_LOAD + lane / 16;
        return (uint32_t)(r * p.swk) + (uint32_t)(KTileT::phys(r, lane % 16) << 4);
    } else {
        return dense_row_off<NW, KTB>(i, wave, lane, p.swn);
    }
}

constexpr int MBS_WM = 2, MBS_WN = 2, MBS_TM = 2, MBS_TN = 4, MBS_NW = 4;
constexpr int MBS_BM = MBS_WM * MBS_TM * 32, MBS_BN = MBS_WN * MBS_TN * 32;  // 128 x 256
constexpr int MBS_KTB = 64, MBS_NS = 3;
constexpr int MBS_LA = MBS_BM * MBS_KTB / 1024 / MBS_NW, MBS_LB = MBS_BN * MBS_KTB / 1024 / MBS_NW;  // 2, 4
constexpr int MBS_NLD = MBS_LA + MBS_LB + 2;  // + one row-scale and one column-scale load per wave
constexpr int MBS_SA = (MBS_BM + MBS_BN) * MBS_KTB, MBS_SB = MBS_SA + MBS_BM * 4;
constexpr int MBS_STAGE = MBS_SB + MBS_BN * 4;
constexpr int MBS_EPI = MBS_NW * MBS_TM * 32 * (MBS_TN * 32 * 2 + 16);
constexpr int MBS_LDS = MBS_NS * MBS_STAGE > MBS_EPI ? MBS_NS * MBS_STAGE : MBS_EPI;
static_assert(2 * MBS_LDS <= 160 * 1024, "two workgroups per CU");

// GNW: group_n is a multiple of 32, so the 32 columns of a sub-tile share one
// weight scale; otherwise every column has its own.
template <bool GNW, bool BT = false>
__global__ __launch_bounds__(64 * MBS_NW, 2) void moe_blockscale_kernel(const MoeBsParams p) {
    using KT = KTile<MBS_KTB>;
    constexpr int TM = MBS_TM, TN = MBS_TN, NW = MBS_NW;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / MBS_WN, wn = wave % MBS_WN;
    const int khalf = lane >> 5;

    const int pm = blockIdx.x / p.tiles_n, tn = blockIdx.x % p.tiles_n;
    const int ed = p.expt_data[pm];
    const int e = ed & 0xFFFF, b = ed >> 16;
    if (ed < 0 || e >= p.E) return;  // uniform: -1 or a malformed entry
    const int m_e = p.hist[e], start = p.offs[e];
    const int row0 = b * 128;
    const int rows = min(m_e - row0, MBS_BM);
    if (rows <= 0 || start < 0) return;
    const int n0 = tn * MBS_BN;
    const int rows_b = min(p.N - n0, MBS_BN);

    auto token_of = [&](int r) {
        const int s = start + row0 + r;
        if (r >= rows || s >= p.g_len) return -1;
        const int t = p.gather ? div_recip(p.gather[s], p.rtopk) : s;
        return (t >= 0 && t < p.T) ? t : -1;
    };

    // operand rows: A gathered per lane (rows of other tokens never enter LDS),
    // B the expert's rows n0 .. n0 + 255
    uint32_t a_off[MBS_LA], b_off[MBS_LB];
#pragma unroll
    for (int i = 0; i < MBS_LA; ++i) {
        const int r = (i * NW + wave) * KT::ROWS_PER_LOAD + lane / KT::CHUNKS;
        const int t = token_of(r);
        a_off[i] = t < 0 ? OOB : (uint32_t)(t * p.sxm) + (uint32_t)(KT::load_chunk(lane, r) << 4);
    }
#pragma unroll
    for (int i = 0; i < MBS_LB; ++i) b_off[i] = moe_bs_b_off<BT, NW, MBS_KTB>(p, i, wave, lane);
    const MoeBsB bsrc = moe_bs_b<BT, MBS_KTB>(p, e, n0, rows_b);
    const uint8_t* wb = bsrc.base;
    const int64_t a_bytes = min((int64_t)p.T * p.sxm, (int64_t)0x7FFFFFFF);
    const int64_t b_bytes = bsrc.bytes;
    // scales: row r = (wave & 1) * 64 + lane (waves 2, 3 load the same rows as
    // 0, 1, so that every wave issues the same number of loads), column
    // n0 + wave * 64 + lane; the group part is added per K-tile
    const int t_sa = token_of((wave & 1) * 64 + lane);
    const uint32_t sa_off = t_sa < 0 ? OOB : (uint32_t)(t_sa * p.xsm * 4);
    const int nc = n0 + wave * 64 + lane;
    const uint32_t sb_off = nc < p.N ? (uint32_t)((nc / p.gn) * p.wsn * 4) : OOB;
    const float* wsb = p.ws + (int64_t)e * p.wse;
    const uint32_t xs_bytes = (uint32_t)min(p.xs_elems * 4, (int64_t)0x7FFFFFFF);
    const uint32_t ws_bytes = (uint32_t)min(max(p.ws_elems - (int64_t)e * p.wse, (int64_t)0) * 4, (int64_t)0x7FFFFFFF);
    const int KTN = p.K / MBS_KTB;

    auto issue = [&](int kt) {
        const bool live = kt < KTN;
        const int kb = kt * MBS_KTB;
        const int g = live ? kb / p.gk : 0;
        HKQ_LDS uint8_t* st = smem + (kt % MBS_NS) * MBS_STAGE;
#pragma unroll
        for (int i = 0; i < MBS_LA; ++i)
            lds_load16(p.X + kb, live && a_bytes > kb ? (uint32_t)(a_bytes - kb) : 0u, st + (i * NW + wave) * 1024,
                       a_off[i]);
        const int64_t kbb = (int64_t)kt * bsrc.kstep;
#pragma unroll
        for (int i = 0; i < MBS_LB; ++i)
            lds_load16(wb + kbb, live && b_bytes > kbb ? (uint32_t)(b_bytes - kbb) : 0u,
                       st + MBS_BM * MBS_KTB + (i * NW + wave) * 1024, b_off[i]);
        lds_load4(p.xs, live ? xs_bytes : 0u, st + MBS_SA + (wave & 1) * 256, sa_off + (uint32_t)(g * p.xsk * 4));
        lds_load4(wsb, live ? ws_bytes : 0u, st + MBS_SB + wave * 256, sb_off + (uint32_t)(g * p.wsk * 4));
    };

    v16f acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = v16f{};

    const int arow = wm * TM * 32 + (lane & 31), brow = wn * TN * 32 + (lane & 31);
    auto frag = [&](const HKQ_LDS uint8_t* tile, int r) {
        const v4i lo = lds_read16(tile + KT::swz(r, 2 * khalf));
        const v4i hi = lds_read16(tile + KT::swz(r, 2 * khalf + 1));
        return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    // BT: n-tile i's operand from the transposed K-tile (64 rows of K x 256
    // columns): rows 32 * khalf + 8q + (j >> 1) of the lane's column, q = 0..3
    const int tj = lane & 15, tg = (lane >> 4) & 1, trow = 32 * khalf + (tj >> 1);
    auto frag_t = [&](const HKQ_LDS uint8_t* tile, int i) {
        const HKQ_LDS uint8_t* b =
            tile + trow * KTileT::ROW + (KTileT::phys(trow, (wn * TN * 32 + i * 32) / 16 + tg) << 4) + 8 * (tj & 1);
        v2i q[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) q[r] = lds_read_tr8(b + 8 * r * KTileT::ROW);
        return v8i{q[0][0], q[0][1], q[1][0], q[1][1], q[2][0], q[2][1], q[3][0], q[3][1]};
    };

    issue(0);
    issue(1);
    for (int kt = 0; kt < KTN; ++kt) {
        // K-tile kt resident (only kt+1's loads may still be in flight) and
        // every wave is done with kt-1's stage, which takes kt+2
        tile_barrier<MBS_NLD>();
        issue(kt + 2);
        const HKQ_LDS uint8_t* st = smem + (kt % MBS_NS) * MBS_STAGE;
        v8i fa[TM], fb[TN];
#pragma unroll
        for (int j = 0; j < TM; ++j) fa[j] = frag(st, arow + j * 32);
#pragma unroll
        for (int i = 0; i < TN; ++i) {
            if constexpr (BT) fb[i] = frag_t(st + MBS_BM * MBS_KTB, i);
            else fb[i] = frag(st + MBS_BM * MBS_KTB, brow + i * 32);
        }
        const HKQ_LDS float* sas = reinterpret_cast<const HKQ_LDS float*>(st + MBS_SA);
        const HKQ_LDS float* sbs = reinterpret_cast<const HKQ_LDS float*>(st + MBS_SB);
        float sa[TM];
#pragma unroll
        for (int j = 0; j < TM; ++j) sa[j] = sas[arow + j * 32];
        // sub-tile s = i*TM + j: its MFMA makes the step partial P, promoted
        // after the next sub-tile's MFMA is issued
        v16f P[2];
        v4f sbv[2][4];
        float sbw[2];
        auto load_sb = [&](int i, int slot) {
            const int c = wn * TN * 32 + i * 32;
            if constexpr (GNW) {
                sbw[slot] = sbs[c];
            } else {
#pragma unroll
                for (int g = 0; g < 4; ++g) sbv[slot][g] = *reinterpret_cast<const HKQ_LDS v4f*>(sbs + c + 8 * g + 4 * khalf);
            }
        };
        auto promote = [&](int s) {
            const int i = s / TM, j = s % TM;
            const v16f& Ps = P[s & 1];
            if constexpr (GNW) {
                const float sc = sa[j] * sbw[i & 1];
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = __builtin_fmaf(Ps[r], sc, acc[i][j][r]);
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    acc[i][j][r] = __builtin_fmaf(Ps[r], sa[j] * sbv[i & 1][r >> 2][r & 3], acc[i][j][r]);
            }
        };
        // column scales of n-tile i sit in slot i & 1; those of i + 1 are read
        // once the last promotion that needs slot (i + 1) & 1 (n-tile i - 1's) is done
        load_sb(0, 0);
#pragma unroll
        for (int s = 0; s < TN * TM; ++s) {
            const int i = s / TM, j = s % TM;
            P[s & 1] = mfma_sel<false, 0, 0>(fb[i], fa[j], v16f{}, 127, 127);
            if (s > 0) promote(s - 1);
            if (j == TM - 1 && i + 1 < TN) load_sb(i + 1, (i + 1) & 1);
        }
        promote(TN * TM - 1);
    }
    mfma_drain();
    tile_barrier<0>();  // no load in flight, every wave past its reads: the stages take the epilogue

    const int s0 = start + row0;
    const int nw = n0 + wn * TN * 32;
    const int out_rows = min(rows, p.y_rows - s0);
    auto one = [](int) { return 1.0f; };
    auto ones = [](int, int) { return make_float4(1.f, 1.f, 1.f, 1.f); };
    uint16_t* Y = p.Y + (int64_t)s0 * p.sym;
    if (p.bias)
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, Y, p.sym, out_rows, p.N, wm * TM * 32, nw, p.c16 != 0, one, ones,
                                [&](int i, int g) {
                                    const int n = nw + i * 32 + 8 * g + 4 * khalf;
                                    if (n >= p.N) return make_float4(0.f, 0.f, 0.f, 0.f);
                                    const float* bp = p.bias + (int64_t)e * p.bias_e + n;
                                    return make_float4(bp[0], bp[1], bp[2], bp[3]);
                                });
    else
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, Y, p.sym, out_rows, p.N, wm * TM * 32, nw, p.c16 != 0, one, ones,
                                NoBias{});
}

// ---------------------------------------------------------------------------
// group_k a multiple of 128 (and K too): the 8-wave K loop of
// blockscale_core.h, 128-wide K-tiles of one scale group each, over tiles of
// 256 rows x 256 columns. A tile takes a pair of routing blocks of one expert
// when the pair sits in consecutive ExptData words (e | b << 16 with b even,
// then e | (b+1) << 16): the first word's workgroup computes both, and the
// second word gets no workgroup (bs_leader). Any other word computes its own
// 128 rows (the tile's other half reads zero). Every listed block is computed
// once, as the reference's grid does.
// ---------------------------------------------------------------------------
template <int SBM, bool BT = false>
__global__ __launch_bounds__(64 * BS_NW, 1) void moe_blockscale8_kernel(const MoeBsParams p) {
    constexpr int TM = BS_TM, TN = BS_TN, NW = BS_NW;
    using KT = KTile<BS_KT>;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / BS_WN, wn = wave % BS_WN;
    const int khalf = lane >> 5;

    // Workgroup li * tiles_n + tn takes the li-th computing word: the words
    // that a pair's first word covers get no workgroup of their own, and the
    // spare workgroups (as many as such words) come last and return (with one
    // workgroup per word, every transition between workgroups on a CU left it
    // idle ~4.5 us; measured on MI355X, Mixtral gate/up: 134 us per CU of gaps).
    const int li = blockIdx.x / p.tiles_n, tn = blockIdx.x % p.tiles_n;
    int ed0[BS_LW];
    bs_words(p, 0, ed0);
    const int tail_from = __builtin_amdgcn_readfirstlane(bs_tail_from(p));
    const int pm = __builtin_amdgcn_readfirstlane(bs_leader(p, li, tail_from, ed0));
    if (pm < 0) return;  // uniform: a spare workgroup
    const int ed = p.expt_data[pm];
    const int e = ed & 0xFFFF, b = ed >> 16;
    // the pair's first word computes it (unless this word is in the tail)
    const bool pair = !(b & 1) && pm + 1 < tail_from && pm + 1 < p.grid_m && p.expt_data[pm + 1] == ed + 0x10000;
    const int m_e = p.hist[e], start = p.offs[e];
    const int row0 = b * 128;
    const int rows = min(m_e - row0, pair ? BS_BM : 128);
    if (rows <= 0 || start < 0) return;
    const int n0 = tn * BS_BN;
    const int rows_b = min(p.N - n0, BS_BN);

    auto token_of = [&](int r) {
        const int s = start + row0 + r;
        if (r >= rows || s >= p.g_len) return -1;
        const int t = p.gather ? div_recip(p.gather[s], p.rtopk) : s;
        return (t >= 0 && t < p.T) ? t : -1;
    };

    // operand rows: A gathered per lane (rows of other tokens never enter LDS),
    // B the expert's rows n0 .. n0 + 255; load i of a wave fills rows
    // (i*NW + wave)*8 .. +7 of its operand tile
    uint32_t a_off[BS_LA], b_off[BS_LB];
#pragma unroll
    for (int i = 0; i < BS_LA; ++i) {
        const int r = (i * NW + wave) * KT::ROWS_PER_LOAD + lane / KT::CHUNKS;
        const int t = token_of(r);
        a_off[i] = t < 0 ? OOB : (uint32_t)t * (uint32_t)p.sxm + (uint32_t)(KT::load_chunk(lane, r) << 4);
        asm volatile("" : "+v"(a_off[i]));  // kept as the 32-bit offset, not re-derived in the loop
    }
#pragma unroll
    for (int i = 0; i < BS_LB; ++i) b_off[i] = moe_bs_b_off<BT, NW, BS_KT>(p, i, wave, lane);
    const MoeBsB bsrc = moe_bs_b<BT, BS_KT>(p, e, n0, rows_b);
    const uint8_t* wb = bsrc.base;
    const int64_t a_bytes = min((int64_t)p.T * p.sxm, (int64_t)0x7FFFFFFF);
    const int64_t b_bytes = bsrc.bytes;
    // scales: row (wave & 3) * 64 + lane, column n0 + (wave & 3) * 64 + lane
    // (waves 4-7 repeat the loads of 0-3, so that every wave issues the same
    // loads); the group moves the base
    const int t_sa = token_of((wave & 3) * 64 + lane);
    uint32_t sa_off = t_sa < 0 ? OOB : (uint32_t)t_sa * (uint32_t)p.xsm * 4u;
    const int nc = n0 + (wave & 3) * 64 + lane;
    uint32_t sb_off = nc < p.N ? (uint32_t)(nc / p.gn) * (uint32_t)p.wsn * 4u : OOB;
    asm volatile("" : "+v"(sa_off));
    asm volatile("" : "+v"(sb_off));
    const float* wsb = p.ws + (int64_t)e * p.wse;
    const int64_t xs_bytes = min(p.xs_elems * 4, (int64_t)0x7FFFFFFF);
    const int64_t ws_bytes = min(max(p.ws_elems - (int64_t)e * p.wse, (int64_t)0) * 4, (int64_t)0x7FFFFFFF);
    // K-tile kt lies in scale group kt >> kpg_log2 (group_k / 128 is a power
    // of 2: a division here is VALU work that costs the K loop its registers)
    const int kpg_log2 = 31 - __builtin_clz(p.gk / BS_KT);
    const uint32_t lds_base = (uint32_t)(uintptr_t)smem;
    const int KTN = p.K / BS_KT;

    // load q (0 .. BS_NLD-1) of K-tile kt: A, B, then the row and column scales
    auto issue = [&](int kt, int q) {
        const bool live = kt < KTN;
        const int64_t kb = (int64_t)kt * BS_KT;
        const int st = kt & 1;
        if (q < BS_LA + BS_LB) {
            HKQ_LDS uint8_t* dst = reinterpret_cast<HKQ_LDS uint8_t*>((uintptr_t)(lds_base + bs_load_dst(st, q, wave)));
            const int64_t kbb = BT ? (int64_t)kt * bsrc.kstep : kb;
            if (q < BS_LA)
                lds_load16(p.X + kb, live && a_bytes > kb ? (uint32_t)(a_bytes - kb) : 0u, dst, a_off[q]);
            else
                lds_load16(wb + kbb, live && b_bytes > kbb ? (uint32_t)(b_bytes - kbb) : 0u, dst, b_off[q - BS_LA]);
        } else {
            HKQ_LDS uint8_t* slot = smem + BS_SC + st * BS_SLOT;
            const int g = live ? kt >> kpg_log2 : 0;
            if (q == BS_LA + BS_LB) {
                const int64_t gb = (int64_t)g * p.xsk * 4;
                lds_load4(p.xs + (int64_t)g * p.xsk, live && xs_bytes > gb ? (uint32_t)(xs_bytes - gb) : 0u,
                          slot + (wave & 3) * 256, sa_off);
            } else {
                const int64_t gb = (int64_t)g * p.wsk * 4;
                lds_load4(wsb + (int64_t)g * p.wsk, live && ws_bytes > gb ? (uint32_t)(ws_bytes - gb) : 0u,
                          slot + 1024 + (wave & 3) * 256, sb_off);
            }
        }
    };

    // waves whose 64 rows lie past the tile's (every wave with wm >= 2 in a
    // lone block) only load: one computing wave per SIMD instead of two
    v16f acc[TN][TM];
    if (wm * TM * 32 < rows)
        bs8_kloop<SBM, BS_TN, true, BT>(smem, lane, wm, wn * BS_TN * 32, KTN, issue, acc);
    else
        bs8_kloop<SBM, BS_TN, false, BT>(smem, lane, wm, wn * BS_TN * 32, KTN, issue, acc);

    const int s0 = start + row0;
    const int nw = n0 + wn * TN * 32;
    const int out_rows = min(rows, p.y_rows - s0);
    auto one = [](int) { return 1.0f; };
    auto ones = [](int, int) { return make_float4(1.f, 1.f, 1.f, 1.f); };
    uint16_t* Y = p.Y + (int64_t)s0 * p.sym;
    if (p.bias)
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, Y, p.sym, out_rows, p.N, wm * TM * 32, nw, p.c16 != 0, one, ones,
                                [&](int i, int g) {
                                    const int n = nw + i * 32 + 8 * g + 4 * khalf;
                                    if (n >= p.N) return make_float4(0.f, 0.f, 0.f, 0.f);
                                    const float* bp = p.bias + (int64_t)e * p.bias_e + n;
                                    return make_float4(bp[0], bp[1], bp[2], bp[3]);
                                });
    else
        store_tile_bf16<TM, TN>(acc, smem, wave, lane, Y, p.sym, out_rows, p.N, wm * TM * 32, nw, p.c16 != 0, one, ones,
                                NoBias{});
}

}  // namespace hkq

using namespace hkq;

extern "C" int hkq_moe_pack_kmajor(const void* src, void* dst, int64_t E, int64_t R, int64_t N,
                                   int64_t src_stride_e, int64_t src_stride_r, int64_t dst_stride_e,
                                   int64_t dst_stride_n, hkq_stream_t stream) {
    HKQ_CHECK_ARG(E >= 0 && R >= 0 && N >= 0, "E, R, N must be >= 0");
    HKQ_CHECK_ARG(E <= 65535 && R < (1 << 30) && N < (1 << 30), "E must be <= 65535 and R, N < 2^30");
    HKQ_CHECK_ARG(src_stride_r >= N && src_stride_e >= 0 && dst_stride_n >= R && dst_stride_e >= 0,
                  "strides must cover the rows (src_stride_r >= N, dst_stride_n >= R)");
    HKQ_CHECK_ARG(E <= 1 || (src_stride_e >= R * src_stride_r && dst_stride_e >= N * dst_stride_n),
                  "expert strides must not overlap the experts' planes");
    if (E == 0 || R == 0 || N == 0) return 0;
    HKQ_CHECK_ARG(src && dst, "src and dst must not be null");
    const int vec = (reinterpret_cast<uintptr_t>(src) % 16 == 0) && (reinterpret_cast<uintptr_t>(dst) % 16 == 0) &&
                    src_stride_r % 16 == 0 && dst_stride_n % 16 == 0 && src_stride_e % 16 == 0 &&
                    dst_stride_e % 16 == 0;
    const dim3 grid((unsigned)((N + PK_T - 1) / PK_T), (unsigned)((R + PK_T - 1) / PK_T), (unsigned)E);
    pack_kmajor_kernel<<<grid, 256, 0, stream>>>(static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), (int)R,
                                                 (int)N, src_stride_e, src_stride_r, dst_stride_e, dst_stride_n, vec);
    return hkq_launch_status();
}

// wt == 0: W[e] is [N, K] with row stride stride_w (K contiguous); wt == 1:
// W[e] is [K, N] with row stride stride_w (N contiguous, the reference's layout).
static int moe_blockscale_impl(const void* X, const void* W, void* Y, const float* x_scale, int64_t xs_stride_m,
                               int64_t xs_stride_k, const float* w_scale, int64_t ws_stride_e, int64_t ws_stride_k,
                               int64_t ws_stride_n, int64_t group_k, int64_t group_n, const float* bias,
                               int64_t bias_stride_e, const int32_t* gather, const int32_t* hist, const int32_t* offs,
                               const int32_t* expt_data, int64_t T, int64_t E, int64_t N, int64_t K, int64_t grid_m,
                               int64_t topk, int64_t stride_xm, int64_t stride_we, int64_t stride_w, int wt,
                               int64_t stride_ym, int64_t y_rows, int64_t gather_len, hkq_stream_t stream) {
    HKQ_CHECK_ARG(T >= 0 && E > 0 && E <= 0xFFFF && N >= 0 && K > 0 && grid_m >= 0 && topk > 0 && topk <= 0xFFFF,
                  "T, grid_m >= 0; 0 < E <= 65535; K > 0; 0 < topk <= 65535");
    HKQ_CHECK_ARG(T < (1 << 30) && N < (1 << 30) && K < (1 << 30) && grid_m < (1 << 30), "dimensions must be < 2^30");
    HKQ_CHECK_ARG(K % 64 == 0, "K must be a multiple of 64");
    HKQ_CHECK_ARG(N % 4 == 0, "N must be a multiple of 4");
    HKQ_CHECK_ARG(group_k >= 64 && group_k % 64 == 0, "group_k must be a positive multiple of 64");
    HKQ_CHECK_ARG(group_n >= 1, "group_n must be >= 1");
    HKQ_CHECK_ARG(x_scale && w_scale, "X_scale and W_scale are required");
    HKQ_CHECK_ARG(xs_stride_m >= 0 && xs_stride_k >= 0 && ws_stride_e >= 0 && ws_stride_k >= 0 && ws_stride_n >= 0,
                  "scale strides must be >= 0");
    HKQ_CHECK_ARG(stride_xm >= K && stride_xm % 16 == 0, "stride_xm must be >= K and a multiple of 16");
    HKQ_CHECK_ARG(T * stride_xm < (1ll << 31), "X must span less than 2^31 bytes (T * stride_xm)");
    if (wt) {
        HKQ_CHECK_ARG(stride_w >= N && stride_w % 16 == 0, "stride_wk must be >= N and a multiple of 16 (W[e] is [K, N])");
        HKQ_CHECK_ARG(K * stride_w < (1ll << 31), "one expert's weights must span less than 2^31 bytes (K * stride_wk)");
    } else {
        HKQ_CHECK_ARG(stride_w >= K && stride_w % 16 == 0, "stride_wn must be >= K and a multiple of 16 (W[e] is [N, K])");
        HKQ_CHECK_ARG(256 * stride_w < (1ll << 31), "256 weight rows must span less than 2^31 bytes");
    }
    HKQ_CHECK_ARG(stride_we >= 0 && stride_we % 16 == 0, "stride_we must be a non-negative multiple of 16");
    HKQ_CHECK_ARG(stride_ym >= N && stride_ym % 4 == 0, "stride_ym must be >= N and a multiple of 4");
    HKQ_CHECK_ARG(y_rows >= 0 && gather_len >= 0, "y_rows and gather_len must be >= 0");
    HKQ_CHECK_ARG(hist && offs && expt_data, "routing metadata pointers must not be null");
    HKQ_CHECK_ALIGN(X, 16);
    HKQ_CHECK_ALIGN(W, 16);
    HKQ_CHECK_ALIGN(Y, 8);
    HKQ_CHECK_ALIGN(x_scale, 4);
    HKQ_CHECK_ALIGN(w_scale, 4);
    const int64_t G = (K + group_k - 1) / group_k, C = (N + group_n - 1) / group_n;
    // extents of the scale tensors as the strides describe them
    const int64_t xs_elems = (T > 0 ? (T - 1) * xs_stride_m : 0) + (G - 1) * xs_stride_k + 1;
    const int64_t ws_elems = (E - 1) * ws_stride_e + (G - 1) * ws_stride_k + (C - 1) * ws_stride_n + 1;
    HKQ_CHECK_ARG(xs_elems < (1ll << 29) && (G - 1) * ws_stride_k + (C - 1) * ws_stride_n < (1ll << 29),
                  "scale tensors must span less than 2^31 bytes");
    MoeBsParams p{};
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
    p.gk = (int)group_k; p.gn = (int)group_n;
    p.sxm = stride_xm; p.swe = stride_we; p.sym = stride_ym;
    p.wt = wt;
    p.swn = wt ? 1 : stride_w;
    p.swk = wt ? stride_w : 1;
    p.xsm = xs_stride_m; p.xsk = xs_stride_k; p.wse = ws_stride_e; p.wsk = ws_stride_k; p.wsn = ws_stride_n;
    p.bias_e = bias_stride_e;
    p.xs_elems = xs_elems; p.ws_elems = ws_elems;
    p.c16 = (stride_ym % 8 == 0) && (reinterpret_cast<uintptr_t>(Y) % 16 == 0);
    // group_k = 128 * 2^j (and K % 128 == 0): the 8-wave kernel, 128-wide
    // K-tiles of one scale group each; HKQ_MOE_BLOCKSCALE8=0 selects the
    // 64-wide kernel for every group_k
    static const bool bs8_on = [] {
        const char* v = std::getenv("HKQ_MOE_BLOCKSCALE8");
        return !(v && v[0] == '0');
    }();
    const int64_t kpg = group_k / BS_KT;  // K-tiles per scale group
    if (bs8_on && K % BS_KT == 0 && group_k % BS_KT == 0 && (kpg & (kpg - 1)) == 0) {
        p.tiles_n = (int)((N + BS_BN - 1) / BS_BN);
        p.ncu = cu_count();
        const int64_t nblk = grid_m * p.tiles_n;
        if (nblk == 0) return 0;
        const bool ntile = group_n % 32 == 0;
        auto kern = ntile ? (wt ? moe_blockscale8_kernel<BS_SB_NTILE, true> : moe_blockscale8_kernel<BS_SB_NTILE>)
                          : (wt ? moe_blockscale8_kernel<BS_SB_COL, true> : moe_blockscale8_kernel<BS_SB_COL>);
        const int v8 = (ntile ? 1 : 0) + (wt ? 2 : 0);
        static bool attr8_set[4] = {false, false, false, false};
        if (!attr8_set[v8]) {
            hipError_t err = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, BS_LDS);
            if (err != hipSuccess) {
                set_error("hipFuncSetAttribute(MaxDynamicSharedMemorySize=%d) failed: %s", BS_LDS, hipGetErrorString(err));
                return (int)err;
            }
            attr8_set[v8] = true;
        }
        kern<<<dim3((unsigned)nblk), 64 * BS_NW, BS_LDS, stream>>>(p);
        return hkq_launch_status();
    }
    p.tiles_n = (int)((N + MBS_BN - 1) / MBS_BN);
    const int64_t nblk = grid_m * p.tiles_n;
    if (nblk == 0) return 0;
    const bool gnw = group_n % 32 == 0;
    auto kern = gnw ? (wt ? moe_blockscale_kernel<true, true> : moe_blockscale_kernel<true>)
                    : (wt ? moe_blockscale_kernel<false, true> : moe_blockscale_kernel<false>);
    const int v = (gnw ? 1 : 0) + (wt ? 2 : 0);
    static bool attr_set[4] = {false, false, false, false};
    if (!attr_set[v]) {
        hipError_t err = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, MBS_LDS);
        if (err != hipSuccess) {
            set_error("hipFuncSetAttribute(MaxDynamicSharedMemorySize=%d) failed: %s", MBS_LDS, hipGetErrorString(err));
            return (int)err;
        }
        attr_set[v] = true;
    }
    kern<<<dim3((unsigned)nblk), 64 * MBS_NW, MBS_LDS, stream>>>(p);
    return hkq_launch_status();
}

extern "C" int hkq_moe_a8w8_blockscale(const void* X, const void* W, void* Y, const float* x_scale,
                                       int64_t xs_stride_m, int64_t xs_stride_k, const float* w_scale,
                                       int64_t ws_stride_e, int64_t ws_stride_k, int64_t ws_stride_n,
                                       int64_t group_k, int64_t group_n, const float* bias, int64_t bias_stride_e,
                                       const int32_t* gather, const int32_t* hist, const int32_t* offs,
                                       const int32_t* expt_data, int64_t T, int64_t E, int64_t N, int64_t K,
                                       int64_t grid_m, int64_t topk, int64_t stride_xm, int64_t stride_we,
                                       int64_t stride_wn, int64_t stride_ym, int64_t y_rows, int64_t gather_len,
                                       hkq_stream_t stream) {
    return moe_blockscale_impl(X, W, Y, x_scale, xs_stride_m, xs_stride_k, w_scale, ws_stride_e, ws_stride_k,
                               ws_stride_n, group_k, group_n, bias, bias_stride_e, gather, hist, offs, expt_data, T, E,
                               N, K, grid_m, topk, stride_xm, stride_we, stride_wn, 0, stride_ym, y_rows, gather_len,
                               stream);
}

extern "C" int hkq_moe_a8w8_blockscale_kn(const void* X, const void* W, void* Y, const float* x_scale,
                                          int64_t xs_stride_m, int64_t xs_stride_k, const float* w_scale,
                                          int64_t ws_stride_e, int64_t ws_stride_k, int64_t ws_stride_n,
                                          int64_t group_k, int64_t group_n, const float* bias, int64_t bias_stride_e,
                                          const int32_t* gather, const int32_t* hist, const int32_t* offs,
                                          const int32_t* expt_data, int64_t T, int64_t E, int64_t N, int64_t K,
                                          int64_t grid_m, int64_t topk, int64_t stride_xm, int64_t stride_we,
                                          int64_t stride_wk, int64_t stride_ym, int64_t y_rows, int64_t gather_len,
                                          hkq_stream_t stream) {
    return moe_blockscale_impl(X, W, Y, x_scale, xs_stride_m, xs_stride_k, w_scale, ws_stride_e, ws_stride_k,
                               ws_stride_n, group_k, group_n, bias, bias_stride_e, gather, hist, offs, expt_data, T, E,
                               N, K, grid_m, topk, stride_xm, stride_we, stride_wk, 1, stride_ym, y_rows, gather_len,
                               stream);
}
