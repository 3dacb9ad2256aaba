// routing.hip -- MoE routing metadata producers (kernels/moe-routing/* of the
// reference): top-k expert selection with the expert bitmatrix, column sums of
// the bitmatrix with per-128-row exclusive partials, the OGS expert/tile
// metadata, the gather/scatter indices of the expert-sorted gate order, and
// the block-padded sorted order of moe_align_block_size.
//
// Every index output is deterministic. Gates of one expert keep their input
// order (a stable counting sort: per-wave LDS counters plus a wave-level match
// of equal experts built from one ballot per expert-id bit), which is the order
// the reference's test formulas define (tests/test_moe.py:97-128,229-256);
// the reference kernels place them with global atomics. No kernel needs a
// memset: every output element is written by exactly one lane.
#include <float.h>

#include <algorithm>

#include "hkq_device.h"
#include "hkq_host.h"

namespace hkq {

// Experts addressable by the counting-sort kernels (compute_indx receives no
// expert count, so its LDS tables are sized for this many).
constexpr int RT_MAX_EXPTS = 1024;
constexpr int RT_EBITS = 10;

// Lanes below this one in mask m.
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// dst[i] = src[i] for i < n by the whole workgroup (NT threads), eight
// independent loads in flight per thread before the LDS stores.
template <int NT>
__device__ __forceinline__ void copy_to_lds(int* dst, const int32_t* src, int n) {
    for (int i0 = 0; i0 < n; i0 += NT * 8) {
        int v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = i0 + j * NT + (int)threadIdx.x;
            v[j] = i < n ? src[i] : 0;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = i0 + j * NT + (int)threadIdx.x;
            if (i < n) dst[i] = v[j];
        }
    }
}

// Mask of the lanes of this wave whose key equals this lane's key (lanes with
// ok == false match nothing and are matched by nothing). Keys are < 2^nbits.
// Called with all 64 lanes active.
__device__ __forceinline__ uint64_t match_key(uint32_t key, bool ok, int nbits) {
    uint64_t m = __ballot(ok);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (key >> b) & 1u;
        const uint64_t s = __ballot(bit);
        m &= bit ? s : ~s;
    }
    return ok ? m : 0ull;
}

// ---------------------------------------------------------------------------
// moe_topk (moe-routing/moe_topk/kernel.cpp:70-205): per row the K largest of
// n_expts bf16 logits, ordered by value (descending) then expert index
// (ascending), -0 == +0, NaN and -inf never selected; slots left empty (fewer
// than K eligible logits) hold index -1 and value -FLT_MAX. With softmax the
// values become expf(v_k - v_0) * (1 / sum_k expf(v_k - v_0)), summed in k
// order. Values are written as bf16; one bitmatrix word per 32 experts.
// ---------------------------------------------------------------------------
struct TopkParams {
    const uint16_t* X;
    int64_t sxm;
    uint16_t* Yv;
    int32_t* Yi;
    int64_t sym;
    uint32_t* bits;  // nullptr: no bitmatrix
    int64_t sbm, sbn;
    int rows, E, K, softmax, nwords;
};

// Order-preserving map of bf16 bits onto 16 bits (-0 folded onto +0).
__device__ __forceinline__ uint32_t order16(uint32_t h) {
    h = (h == 0x8000u) ? 0u : h;
    return (h & 0x8000u) ? (~h & 0xFFFFu) : (h | 0x8000u);
}
__device__ __forceinline__ uint32_t unorder16(uint32_t k) { return (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu); }

// Maximum over aligned groups of L lanes (L a power of two <= 64), the result
// in every lane of the group. Within a row of 16 lanes the exchanges are DPP
// moves (quad_perm xor 1 / xor 2, half-row mirror, row mirror: each pairs the
// two halves of the current group); wider groups use ds_swizzle / bpermute.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int L>
__device__ __forceinline__ uint32_t group_max_u32(uint32_t m) {
    if constexpr (L >= 2) m = max(m, dpp_u32<0xB1>(m));   // quad_perm [1,0,3,2]
    if constexpr (L >= 4) m = max(m, dpp_u32<0x4E>(m));   // quad_perm [2,3,0,1]
    if constexpr (L >= 8) m = max(m, dpp_u32<0x141>(m));  // row_half_mirror
    if constexpr (L >= 16) m = max(m, dpp_u32<0x140>(m)); // row_mirror
    if constexpr (L >= 32) m = max(m, (uint32_t)__builtin_amdgcn_ds_swizzle((int)m, 0x401F));  // xor 16
    if constexpr (L >= 64) m = max(m, (uint32_t)__shfl_xor((int)m, 32, 64));
    return m;
}

// L lanes per row, V logits per lane (lane j holds experts j, j + L, ...),
// KMAX >= K winners kept in registers. A logit and its expert pack into one
// 32-bit key, order16(bf16) << 16 | (0xFFFF - expert): the largest key is the
// largest logit, ties going to the lower expert; 0 = not eligible (NaN, -inf,
// padding).
template <int L, int V, int KMAX>
__global__ __launch_bounds__(256) void topk_kernel(const TopkParams p) {
    constexpr int RPB = 256 / L;
    const int j = threadIdx.x % L;
    const int row = blockIdx.x * RPB + threadIdx.x / L;
    const bool live = row < p.rows;
    const uint16_t* x = p.X + (int64_t)(live ? row : 0) * p.sxm;

    uint32_t key[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int e = j + v * L;
        const uint32_t h = (live && e < p.E) ? (uint32_t)x[e] : 0xFF80u;
        const bool ok = (h & 0x7FFFu) <= 0x7F80u && h != 0xFF80u;
        key[v] = ok ? (order16(h) << 16) | (0xFFFFu - (uint32_t)e) : 0u;
    }

    uint32_t win[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
        win[k] = 0;
        if (k < p.K) {
            uint32_t m = key[0];
#pragma unroll
            for (int v = 1; v < V; ++v) m = max(m, key[v]);
            m = group_max_u32<L>(m);
            win[k] = m;
#pragma unroll
            for (int v = 0; v < V; ++v) key[v] = key[v] == m ? 0u : key[v];
        }
    }
    if (!live) return;

    float val[KMAX];
    if (p.softmax) {
        // expf(v_k - v_0) summed in k order, then scaled by 1 / sum; empty
        // slots take -FLT_MAX
#pragma unroll
        for (int k = 0; k < KMAX; ++k) val[k] = win[k] ? bf16_to_f32(unorder16(win[k] >> 16)) : -FLT_MAX;
        const float mx = val[0];
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
            if (k < p.K) {
                val[k] = expf(val[k] - mx);
                sum += val[k];
            }
        }
        const float inv = 1.0f / sum;
#pragma unroll
        for (int k = 0; k < KMAX; ++k) val[k] *= inv;
    }

    const int64_t yo = (int64_t)row * p.sym;
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
        if (k < p.K && (k % L) == j) {
            const int idx = win[k] ? (int)(0xFFFFu - (win[k] & 0xFFFFu)) : -1;
            uint32_t h;
            if (p.softmax) h = f32_to_bf16(val[k]);
            else h = idx >= 0 ? (uint32_t)x[idx] : 0xFF80u;  // the logit's own bits; bf16(-FLT_MAX) = -inf
            p.Yv[yo + k] = (uint16_t)h;
            p.Yi[yo + k] = idx;
        }
    }
    if (p.bits) {
        for (int w = j; w < p.nwords; w += L) {
            uint32_t word = 0;
#pragma unroll
            for (int k = 0; k < KMAX; ++k) {
                const uint32_t e = 0xFFFFu - (win[k] & 0xFFFFu);
                if (k < p.K && win[k] && (int)(e >> 5) == w) word |= 1u << (e & 31);
            }
            p.bits[(int64_t)row * p.sbm + (int64_t)w * p.sbn] = word;
        }
    }
}

// ---------------------------------------------------------------------------
// sum_bitmatrix_rows (moe-routing/moe_bitmatrix/kernel.cpp:84-160,168-204):
// ret[e] = rows with bit e set; partials[t, e] = the same count over the rows
// of the 128-row tiles before tile t (an exclusive prefix over tiles).
// One workgroup per 32-expert column word; tiles are counted with one ballot
// per bit, 256 tiles at a time, then scanned with a carry.
// ---------------------------------------------------------------------------
struct BitsumParams {
    const uint32_t* B;
    int64_t sbm, sbn;
    uint32_t* ret;
    uint32_t* partials;  // nullptr: totals only
    int64_t spm, spn;
    int rows, nwords, pcols;  // partial columns written: e < pcols
};

constexpr int BS_TILE = 128;
constexpr int BS_CHUNK = 256;  // tiles per LDS pass
constexpr int BS_TPT = BS_CHUNK / 32;  // tiles per scanning thread

__device__ __forceinline__ uint32_t tile_bit_count(const uint32_t* col, int64_t sbm, int rows, int r0, int lane) {
    const int ra = r0 + lane, rb = ra + 64;
    const uint32_t w0 = ra < rows ? col[(int64_t)ra * sbm] : 0u;
    const uint32_t w1 = rb < rows ? col[(int64_t)rb * sbm] : 0u;
    uint32_t mine = 0;
#pragma unroll
    for (int bit = 0; bit < 32; ++bit) {
        const uint32_t c = (uint32_t)__popcll(__ballot((w0 >> bit) & 1u)) + (uint32_t)__popcll(__ballot((w1 >> bit) & 1u));
        mine = lane == bit ? c : mine;
    }
    return mine;  // lane b < 32: rows of the tile with bit b set
}

__global__ __launch_bounds__(1024) void bitsum_kernel(const BitsumParams p) {
    __shared__ uint32_t cnt[BS_CHUNK][32];
    __shared__ uint32_t gsum[32][33];
    __shared__ uint32_t carry[32];
    const int word = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = threadIdx.x & 31, g = threadIdx.x >> 5;  // scan roles
    const int ntiles = (p.rows + BS_TILE - 1) / BS_TILE;
    const uint32_t* col = p.B + (int64_t)word * p.sbn;
    if (threadIdx.x < 32) carry[threadIdx.x] = 0;

    for (int c0 = 0; c0 < ntiles; c0 += BS_CHUNK) {
        const int nt = min(BS_CHUNK, ntiles - c0);
        for (int t = wave; t < nt; t += 16) {
            const uint32_t c = tile_bit_count(col, p.sbm, p.rows, (c0 + t) * BS_TILE, lane);
            if (lane < 32) cnt[t][lane] = c;
        }
        __syncthreads();
        // thread (g, b): tiles [g*BS_TPT, (g+1)*BS_TPT) of bit b
        uint32_t loc[BS_TPT], s = 0;
#pragma unroll
        for (int i = 0; i < BS_TPT; ++i) {
            const int t = g * BS_TPT + i;
            loc[i] = s;
            s += t < nt ? cnt[t][b] : 0u;
        }
        gsum[g][b] = s;
        __syncthreads();
        uint32_t pre = carry[b], tot = 0;
        for (int q = 0; q < 32; ++q) {
            const uint32_t v = gsum[q][b];
            pre += q < g ? v : 0u;
            tot += v;
        }
        if (p.partials) {
            const int64_t e = (int64_t)word * 32 + b;
#pragma unroll
            for (int i = 0; i < BS_TPT; ++i) {
                const int t = g * BS_TPT + i;
                if (t < nt && e < p.pcols) p.partials[(int64_t)(c0 + t) * p.spm + e * p.spn] = pre + loc[i];
            }
        }
        __syncthreads();
        if (g == 0) carry[b] += tot;
        __syncthreads();
    }
    if (threadIdx.x < 32) p.ret[word * 32 + threadIdx.x] = carry[threadIdx.x];
}

// Wide form of the same sums when every expert column has a partials column:
// bitcount_kernel counts one 128-row tile per wave (16 tiles per workgroup,
// grid over tiles x words) into partials; bitscan_kernel then turns each
// expert's column of tile counts into its exclusive prefix, in place, and
// writes ret.
__global__ __launch_bounds__(1024) void bitcount_kernel(const BitsumParams p) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int word = blockIdx.y;
    const int t = blockIdx.x * 16 + wave;
    const int ntiles = (p.rows + BS_TILE - 1) / BS_TILE;
    if (t >= ntiles) return;  // wave-uniform
    const uint32_t c = tile_bit_count(p.B + (int64_t)word * p.sbn, p.sbm, p.rows, t * BS_TILE, lane);
    if (lane < 32) p.partials[(int64_t)t * p.spm + ((int64_t)word * 32 + lane) * p.spn] = c;
}

__global__ __launch_bounds__(1024) void bitscan_kernel(const BitsumParams p) {
    __shared__ uint32_t gsum[32][33];
    __shared__ uint32_t carry[32];
    const int word = blockIdx.x;
    const int b = threadIdx.x & 31, g = threadIdx.x >> 5;
    const int ntiles = (p.rows + BS_TILE - 1) / BS_TILE;
    uint32_t* colp = p.partials + ((int64_t)word * 32 + b) * p.spn;
    if (threadIdx.x < 32) carry[threadIdx.x] = 0;
    for (int c0 = 0; c0 < ntiles; c0 += BS_CHUNK) {
        const int nt = min(BS_CHUNK, ntiles - c0);
        uint32_t v[BS_TPT], loc[BS_TPT], s = 0;
#pragma unroll
        for (int i = 0; i < BS_TPT; ++i) {
            const int t = g * BS_TPT + i;
            v[i] = t < nt ? colp[(int64_t)(c0 + t) * p.spm] : 0u;
        }
#pragma unroll
        for (int i = 0; i < BS_TPT; ++i) {
            loc[i] = s;
            s += v[i];
        }
        gsum[g][b] = s;
        __syncthreads();
        uint32_t pre = carry[b], tot = 0;
        for (int q = 0; q < 32; ++q) {
            const uint32_t x = gsum[q][b];
            pre += q < g ? x : 0u;
            tot += x;
        }
#pragma unroll
        for (int i = 0; i < BS_TPT; ++i) {
            const int t = g * BS_TPT + i;
            if (t < nt) colp[(int64_t)(c0 + t) * p.spm] = pre + loc[i];
        }
        __syncthreads();
        if (g == 0) carry[b] += tot;
        __syncthreads();
    }
    if (threadIdx.x < 32) p.ret[word * 32 + threadIdx.x] = carry[threadIdx.x];
}

// ---------------------------------------------------------------------------
// expt_data (moe-routing/moe_expt_data/kernel.cpp:25-106):
//   token_start[e] = sum_{e' < e} hist[e'], token_start[E] = n_gates;
//   tile_start[e]  = sum_{e' < e} ceil(hist[e'] / 2^log2), tile_start[E] = total tiles;
//   md[t] = e | (i << 16) for the i-th tile of expert e, 0xFFFFFFFF for t >= total.
// Every workgroup scans hist itself (E <= ED_MAX_EXPTS) and fills its own
// range of md (tile owner by binary search over the tile starts).
// ---------------------------------------------------------------------------
struct ExptDataParams {
    const int32_t* hist;
    int32_t* token_start;
    int32_t* tile_start;
    uint32_t* md;
    int E, max_tiles, n_gates, log2;
    int starts;   // write token_start / tile_start (workgroup 0)
    int tiles;    // 1: every md entry; 0: only the sentinel tail (stage 1)
};

constexpr int ED_MAX_EXPTS = 4096;
constexpr int ED_TILES_PER_BLOCK = 512;

// Exclusive block-wide scan of one value per thread (NW waves); returns the
// prefix and stores the total in *total. wsum holds NW ints.
template <int NW>
__device__ __forceinline__ int block_scan(int v, int* wsum, int* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o, 64);
        incl += lane >= o ? t : 0;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int pre = 0, tot = 0;
#pragma unroll
    for (int q = 0; q < NW; ++q) {
        pre += q < wave ? wsum[q] : 0;
        tot += wsum[q];
    }
    __syncthreads();
    *total = tot;
    return pre + incl - v;
}

__global__ __launch_bounds__(256) void expt_data_kernel(const ExptDataParams p) {
    __shared__ int tstart[ED_MAX_EXPTS + 1];
    __shared__ int hist[ED_MAX_EXPTS];
    __shared__ int wsum[4];
    copy_to_lds<256>(hist, p.hist, p.E);
    __syncthreads();
    const int per = (p.E + 255) / 256;
    const int e0 = threadIdx.x * per, e1 = min(p.E, e0 + per);
    int ntok = 0, ntile = 0;
    for (int e = e0; e < e1; ++e) {
        const int h = hist[e];
        ntok += h;
        ntile += (h + (1 << p.log2) - 1) >> p.log2;
    }
    int tok_total, tile_total;
    int tok = block_scan<4>(ntok, wsum, &tok_total);
    int tile = block_scan<4>(ntile, wsum, &tile_total);
    const bool lead = blockIdx.x == 0 && p.starts;
    for (int e = e0; e < e1; ++e) {
        const int h = hist[e];
        tstart[e] = tile;
        if (lead) {
            p.token_start[e] = tok;
            p.tile_start[e] = tile;
        }
        tok += h;
        tile += (h + (1 << p.log2) - 1) >> p.log2;
    }
    if (threadIdx.x == 0) {
        tstart[p.E] = tile_total;
        if (lead) {
            p.token_start[p.E] = p.n_gates;
            p.tile_start[p.E] = tile_total;
        }
    }
    __syncthreads();
    const int t0 = blockIdx.x * ED_TILES_PER_BLOCK;
    const int t1 = min(p.max_tiles, t0 + ED_TILES_PER_BLOCK);
    for (int t = t0 + threadIdx.x; t < t1; t += 256) {
        if (t >= tile_total) {
            p.md[t] = 0xFFFFFFFFu;
        } else if (p.tiles) {
            // last expert whose first tile is <= t (experts without tiles share
            // their start with the next one and are skipped by "last")
            int lo = 0, hi = p.E - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (tstart[mid] <= t) lo = mid;
                else hi = mid - 1;
            }
            p.md[t] = (uint32_t)lo | ((uint32_t)(t - tstart[lo]) << 16);
        }
    }
}

// Stage 2 on its own (moe_expt_data/kernel.cpp:69-89): the tiles of expert
// blockIdx.x from the caller's tile_start; fused = only the first tile, with
// the bare expert id (:93-106). Entries at or past `limit` are not written.
__global__ __launch_bounds__(256) void expt_data_stage2_kernel(const int32_t* hist, const int32_t* tile_start,
                                                               uint32_t* md, int log2, int fused, int limit) {
    const int e = blockIdx.x;
    const int h = hist[e];
    if (h <= 0) return;
    const int n = fused ? 1 : (h + (1 << log2) - 1) >> log2;
    const int off = tile_start[e];
    for (int i = threadIdx.x; i < n; i += 256)
        if (off + i < limit) md[off + i] = (uint32_t)e | ((uint32_t)i << 16);
}

// ---------------------------------------------------------------------------
// routing_compute_indx (moe-routing/moe_routing/kernel.cpp:78-205): the gates
// (flattened [tokens, K] expert ids) of each 128-token block are ranked among
// the gates of the same expert in the block (input order), and
//   pos = tokens_start[e] + partial_offs[block, e] + rank,
//   scatter[g] = pos, gather[pos] = g, gate_scal[pos] = expt_scal[g].
// Gates whose expert id is outside [0, RT_MAX_EXPTS) (e.g. -1, dropped) get
// scatter[g] = -1 and no slot. Without partial_offs (the fused variant) one
// workgroup walks the blocks in order and carries the per-expert counts.
// ---------------------------------------------------------------------------
struct IndxParams {
    int32_t* gather;
    int32_t* scatter;
    uint16_t* gate_scal;        // nullptr: not written
    const uint16_t* expt_scal;  // nullptr with gate_scal
    const int32_t* expt_indx;
    const int32_t* partial_offs;  // nullptr: carried in LDS (single workgroup)
    int64_t spm, spn;
    const int32_t* tokens_start;
    int n_gates, K, nblocks;
};

constexpr int CI_TOKENS = 128;  // tokens per block (moe_routing/kernel.cpp:222)

// CH chunks of 64 gates per wave (4 * CH * 64 >= 128 * K); NB blocks in
// flight per workgroup (4 waves each). With partial_offs the grid has one
// workgroup per block (NB = 1); without, one workgroup walks all blocks NB at
// a time and carries the per-expert counts.
template <int CH, int NB>
__global__ __launch_bounds__(256 * NB) void compute_indx_kernel(const IndxParams p) {
    __shared__ int cnt[NB][4][RT_MAX_EXPTS];
    __shared__ int run[RT_MAX_EXPTS];
    const int lane = threadIdx.x & 63, wave = (threadIdx.x >> 6) & 3, slot = threadIdx.x >> 8;
    const int G = CI_TOKENS * p.K;
    const bool carry = p.partial_offs == nullptr;
    if (carry)
        for (int e = threadIdx.x; e < RT_MAX_EXPTS; e += 256 * NB) run[e] = 0;

    const int b0 = carry ? 0 : blockIdx.x, b1 = carry ? p.nblocks : blockIdx.x + 1;
    for (int it = b0; it < b1; it += NB) {
        const int blk = it + slot;  // may be >= b1: then every gate is out of range
        for (int i = threadIdx.x; i < NB * 4 * RT_MAX_EXPTS; i += 256 * NB) (&cnt[0][0][0])[i] = 0;
        __syncthreads();
        int ex[CH], rk[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int gl = (wave * CH + c) * 64 + lane;
            const int64_t g = (int64_t)blk * G + gl;
            const bool in = blk < b1 && gl < G && g < p.n_gates;
            const int e = in ? p.expt_indx[g] : -1;
            const bool ok = (uint32_t)e < (uint32_t)RT_MAX_EXPTS;
            const uint64_t m = match_key((uint32_t)e, ok, RT_EBITS);
            const int r = (int)lanes_below(m), n = __popcll(m);
            const int base = ok ? cnt[slot][wave][e] : 0;
            if (ok && r == n - 1) cnt[slot][wave][e] = base + n;
            ex[c] = ok ? e : (in ? -2 : -1);
            rk[c] = base + r;
        }
        __syncthreads();
        // exclusive prefix over (block in flight, wave), starting from the carry
        for (int e = threadIdx.x; e < RT_MAX_EXPTS; e += 256 * NB) {
            int s = carry ? run[e] : 0;
#pragma unroll
            for (int j = 0; j < NB; ++j)
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const int v = cnt[j][w][e];
                    cnt[j][w][e] = s;
                    s += v;
                }
            if (carry) run[e] = s;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int gl = (wave * CH + c) * 64 + lane;
            const int64_t g = (int64_t)blk * G + gl;
            const int e = ex[c];
            if (e >= 0) {
                int pos = p.tokens_start[e] + cnt[slot][wave][e] + rk[c];
                if (!carry) pos += p.partial_offs[(int64_t)blk * p.spm + (int64_t)e * p.spn];
                p.scatter[g] = pos;
                p.gather[pos] = (int32_t)g;
                if (p.gate_scal) p.gate_scal[pos] = p.expt_scal[g];
            } else if (e == -2) {
                p.scatter[g] = -1;
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// moe_align_block_size (moe-routing/moe_align_block_size/kernel.cpp:22-127,
// formula tests/test_moe.py:229-256): counts c[e] of topk_ids, padded counts
// a[e] = ceil(c[e] / bs) * bs, cumsum[e] = sum_{e' < e} a[e'], total = cumsum[E];
// sorted[cumsum[e] + i] = the i-th index (input order) with expert e, padded
// slots = numel; expert_ids[blk] = e for the blocks of expert e.
// Two launches: per-segment counts into the caller's workspace, then every
// segment ranks and scatters its own ids (the cumsum is recomputed per
// workgroup from the counts). Ids outside [0, E) are skipped.
// ---------------------------------------------------------------------------
constexpr int AL_MAX_COUNTS = 16384;  // segments x experts staged in LDS

struct AlignParams {
    const int32_t* ids;
    int32_t* sorted;
    int32_t* expert_ids;
    int32_t* counts;  // workspace [nseg, E]
    int32_t* cumsum;  // [E + 1]
    int32_t* total;   // [1]
    int E, bs, numel, seg, nseg, ebits;
};

constexpr int AL_NW = 16;  // waves per workgroup

__global__ __launch_bounds__(64 * AL_NW) void align_count_kernel(const AlignParams p) {
    __shared__ int cnt[RT_MAX_EXPTS];
    for (int e = threadIdx.x; e < p.E; e += 64 * AL_NW) cnt[e] = 0;
    __syncthreads();
    const int i0 = blockIdx.x * p.seg, i1 = min(p.numel, i0 + p.seg);
    for (int b = i0; b < i1; b += 4 * 64 * AL_NW) {
        int e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = b + j * 64 * AL_NW + (int)threadIdx.x;
            e[j] = i < i1 ? p.ids[i] : -1;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if ((uint32_t)e[j] < (uint32_t)p.E) atomicAdd(&cnt[e[j]], 1);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < p.E; e += 64 * AL_NW) p.counts[(int64_t)blockIdx.x * p.E + e] = cnt[e];
}

// Dynamic LDS: tot[E], pre[E], cum[E + 1], segc[nseg * E], wcnt[AL_NW][E].
__global__ __launch_bounds__(64 * AL_NW) void align_scatter_kernel(const AlignParams p) {
    extern __shared__ int lds[];
    int* tot = lds;
    int* pre = tot + p.E;
    int* cum = pre + p.E;
    int* segc = cum + p.E + 1;
    int* wcnt = segc + p.nseg * p.E;  // [AL_NW][E]
    __shared__ int wsum[AL_NW];
    constexpr int NT = 64 * AL_NW;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int seg = blockIdx.x;

    // per expert: the total count and the count in the segments before this one
    copy_to_lds<NT>(segc, p.counts, p.nseg * p.E);
    for (int i = threadIdx.x; i < AL_NW * p.E; i += NT) wcnt[i] = 0;
    __syncthreads();
    for (int e = threadIdx.x; e < p.E; e += NT) {
        int t = 0, before = 0;
        for (int s = 0; s < p.nseg; ++s) {
            const int c = segc[s * p.E + e];
            before += s < seg ? c : 0;
            t += c;
        }
        tot[e] = t;
        pre[e] = before;
    }
    __syncthreads();
    // padded exclusive cumsum over experts (thread-contiguous expert ranges)
    const int per = (p.E + NT - 1) / NT;
    const int e0 = threadIdx.x * per, e1 = min(p.E, e0 + per);
    int acc = 0;
    for (int e = e0; e < e1; ++e) acc += (tot[e] + p.bs - 1) / p.bs * p.bs;
    int all;
    int run = block_scan<AL_NW>(acc, wsum, &all);
    for (int e = e0; e < e1; ++e) {
        cum[e] = run;
        run += (tot[e] + p.bs - 1) / p.bs * p.bs;
    }
    if (threadIdx.x == 0) cum[p.E] = all;

    // per-wave counts of this segment (wave w takes a contiguous share, a
    // multiple of 64 ids)
    const int i0 = seg * p.seg, i1 = min(p.numel, i0 + p.seg);
    const int q = (p.seg / AL_NW + 63) / 64 * 64;
    const int w0 = min(i1, i0 + wave * q), w1 = min(i1, w0 + q);
    int* mine = wcnt + wave * p.E;
    for (int b = w0; b < w1; b += 4 * 64) {
        int e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = b + j * 64 + lane;
            e[j] = i < w1 ? p.ids[i] : -1;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if ((uint32_t)e[j] < (uint32_t)p.E) atomicAdd(&mine[e[j]], 1);
    }
    __syncthreads();
    // base of (wave, expert) = cum[e] + earlier segments + earlier waves
    for (int e = threadIdx.x; e < p.E; e += NT) {
        int s = cum[e] + pre[e];
        for (int w = 0; w < AL_NW; ++w) {
            const int v = wcnt[w * p.E + e];
            wcnt[w * p.E + e] = s;
            s += v;
        }
    }
    __syncthreads();
    // chunks of 64 ids, four loads in flight: each id takes base + its rank
    // among the chunk's ids of the same expert, and the last of them
    // advances the base
    for (int b = w0; b < w1; b += 4 * 64) {
        int e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = b + j * 64 + lane;
            e[j] = i < w1 ? p.ids[i] : -1;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = b + j * 64 + lane;
            const bool ok = (uint32_t)e[j] < (uint32_t)p.E;
            const uint64_t m = match_key((uint32_t)e[j], ok, p.ebits);
            const int r = (int)lanes_below(m), n = __popcll(m);
            const int base = ok ? mine[e[j]] : 0;
            if (ok && r == n - 1) mine[e[j]] = base + n;
            if (ok) p.sorted[base + r] = i;
        }
    }

    // padding, expert ids of the blocks, cumsum and total: experts e == seg (mod nseg)
    for (int e = seg; e < p.E; e += p.nseg) {
        const int pad0 = cum[e] + tot[e], end = cum[e + 1];
        for (int x = pad0 + threadIdx.x; x < end; x += NT) p.sorted[x] = p.numel;
        for (int blk = cum[e] / p.bs + threadIdx.x; blk < end / p.bs; blk += NT) p.expert_ids[blk] = e;
    }
    if (seg == 0) {
        for (int e = threadIdx.x; e <= p.E; e += NT) p.cumsum[e] = cum[e];
        if (threadIdx.x == 0) *p.total = all;
    }
}

}  // namespace hkq

// ============================================================================
// Host launchers (C ABI)
// ============================================================================
namespace {
using namespace hkq;

template <int L, int V>
int launch_topk(const TopkParams& p, int kmax, hipStream_t s) {
    const dim3 grid((p.rows + 256 / L - 1) / (256 / L));
    switch (kmax) {
        case 2: topk_kernel<L, V, 2><<<grid, 256, 0, s>>>(p); break;
        case 4: topk_kernel<L, V, 4><<<grid, 256, 0, s>>>(p); break;
        case 8: topk_kernel<L, V, 8><<<grid, 256, 0, s>>>(p); break;
        default: topk_kernel<L, V, 16><<<grid, 256, 0, s>>>(p); break;
    }
    return hkq_launch_status();
}

template <int CH>
int launch_indx(const IndxParams& p, hipStream_t s) {
    if (p.partial_offs) compute_indx_kernel<CH, 1><<<p.nblocks, 256, 0, s>>>(p);
    else compute_indx_kernel<CH, 4><<<1, 1024, 0, s>>>(p);
    return hkq_launch_status();
}

int indx(int32_t* gather, int32_t* scatter, void* gate_scal, const void* expt_scal, const int32_t* expt_indx,
         const int32_t* partial_offs, int64_t spm, int64_t spn, const int32_t* tokens_start, int64_t n_gates, int K,
         hipStream_t stream) {
    HKQ_CHECK_ARG(K >= 1 && K <= 16, "n_expts_act must be in [1, 16]");
    HKQ_CHECK_ARG(n_gates >= 0 && n_gates <= INT32_MAX, "n_gates must be in [0, 2^31)");
    if (n_gates == 0) return 0;
    HKQ_CHECK_ARG(gather && scatter && expt_indx && tokens_start, "GatherIndx, ScatterIndx, ExptIndx and TokensStart are required");
    HKQ_CHECK_ARG((gate_scal == nullptr) == (expt_scal == nullptr), "GateScal and ExptScal must both be given or both be null");
    HKQ_CHECK_ALIGN(gather, 4);
    HKQ_CHECK_ALIGN(scatter, 4);
    HKQ_CHECK_ALIGN(expt_indx, 4);
    HKQ_CHECK_ALIGN(tokens_start, 4);
    HKQ_CHECK_ALIGN(gate_scal, 2);
    HKQ_CHECK_ALIGN(expt_scal, 2);
    HKQ_CHECK_ARG(partial_offs == nullptr || (spm >= 0 && spn >= 0), "PartialOffs strides must be non-negative");
    HKQ_CHECK_ALIGN(partial_offs, 4);
    IndxParams p{};
    p.gather = gather;
    p.scatter = scatter;
    p.gate_scal = (uint16_t*)gate_scal;
    p.expt_scal = (const uint16_t*)expt_scal;
    p.expt_indx = expt_indx;
    p.partial_offs = partial_offs;
    p.spm = spm;
    p.spn = spn;
    p.tokens_start = tokens_start;
    p.n_gates = (int)n_gates;
    p.K = K;
    const int64_t G = (int64_t)CI_TOKENS * K;
    p.nblocks = (int)((n_gates + G - 1) / G);
    if (K <= 2) return launch_indx<1>(p, stream);
    if (K <= 4) return launch_indx<2>(p, stream);
    if (K <= 8) return launch_indx<4>(p, stream);
    return launch_indx<8>(p, stream);
}

int expt_data(const int32_t* hist, int32_t* token_start, int32_t* tile_start, uint32_t* md, int64_t E,
              int64_t max_tiles, int64_t n_gates, int log2, int tiles, hipStream_t stream) {
    HKQ_CHECK_ARG(E >= 1 && E <= ED_MAX_EXPTS, "n_expts_tot must be in [1, 4096]");
    HKQ_CHECK_ARG(max_tiles >= 0 && max_tiles <= INT32_MAX, "max_num_tiles must be in [0, 2^31)");
    HKQ_CHECK_ARG(log2 >= 0 && log2 <= 16, "tile_dim_log2 must be in [0, 16]");
    HKQ_CHECK_ARG(hist && token_start && tile_start && (md || max_tiles == 0), "Hist, TokenStart, TileStart and MDTileInfo are required");
    HKQ_CHECK_ALIGN(hist, 4);
    HKQ_CHECK_ALIGN(token_start, 4);
    HKQ_CHECK_ALIGN(tile_start, 4);
    HKQ_CHECK_ALIGN(md, 4);
    ExptDataParams p{};
    p.hist = hist;
    p.token_start = token_start;
    p.tile_start = tile_start;
    p.md = md;
    p.E = (int)E;
    p.max_tiles = (int)max_tiles;
    p.n_gates = (int)n_gates;
    p.log2 = log2;
    p.starts = 1;
    p.tiles = tiles;
    const int grid = (int)std::max<int64_t>(1, (max_tiles + ED_TILES_PER_BLOCK - 1) / ED_TILES_PER_BLOCK);
    expt_data_kernel<<<grid, 256, 0, stream>>>(p);
    return hkq_launch_status();
}

int stage2(const int32_t* hist, const int32_t* tile_start, uint32_t* md, int64_t E, int log2, int fused, int limit,
           hipStream_t stream) {
    HKQ_CHECK_ARG(E >= 1 && E <= INT32_MAX, "n_expts_tot must be >= 1");
    HKQ_CHECK_ARG(log2 >= 0 && log2 <= 16, "tile_dim_log2 must be in [0, 16]");
    HKQ_CHECK_ARG(hist && tile_start && md, "Hist, TileStart and TileInfo are required");
    HKQ_CHECK_ALIGN(hist, 4);
    HKQ_CHECK_ALIGN(tile_start, 4);
    HKQ_CHECK_ALIGN(md, 4);
    expt_data_stage2_kernel<<<(unsigned)E, 256, 0, stream>>>(hist, tile_start, md, log2, fused, limit);
    return hkq_launch_status();
}

int bitsum(const uint32_t* B, int64_t rows, int64_t sbm, int64_t sbn, uint32_t* ret, uint32_t* partials, int64_t spm,
           int64_t spn, int64_t pcols, int64_t nwords, hipStream_t stream) {
    HKQ_CHECK_ARG(rows >= 0 && rows <= INT32_MAX, "shape_bm must be in [0, 2^31)");
    HKQ_CHECK_ARG(nwords >= 1 && nwords <= 65535, "the bitmatrix must have 1 to 65535 column words");
    HKQ_CHECK_ARG(sbm >= 0 && sbn >= 0 && spm >= 0 && spn >= 0, "strides must be non-negative");
    HKQ_CHECK_ARG(ret && (B || rows == 0), "B and Ret are required");
    HKQ_CHECK_ALIGN(B, 4);
    HKQ_CHECK_ALIGN(ret, 4);
    HKQ_CHECK_ALIGN(partials, 4);
    BitsumParams p{};
    p.B = B;
    p.sbm = sbm;
    p.sbn = sbn;
    p.ret = ret;
    p.partials = partials;
    p.spm = spm;
    p.spn = spn;
    p.rows = (int)rows;
    p.nwords = (int)nwords;
    p.pcols = (int)std::min<int64_t>(pcols, INT32_MAX);
    const int64_t ntiles = (rows + BS_TILE - 1) / BS_TILE;
    if (partials && pcols >= 32 * nwords && ntiles > 16) {
        // every expert has a partials column to hold its tile counts
        bitcount_kernel<<<dim3((unsigned)((ntiles + 15) / 16), (unsigned)nwords), 1024, 0, stream>>>(p);
        const int rc = hkq_launch_status();
        if (rc) return rc;
        bitscan_kernel<<<(unsigned)nwords, 1024, 0, stream>>>(p);
        return hkq_launch_status();
    }
    bitsum_kernel<<<(unsigned)nwords, 1024, 0, stream>>>(p);
    return hkq_launch_status();
}

}  // namespace

extern "C" int hkq_moe_topk(const void* X, int64_t stride_xm, void* Yv, int32_t* Yi, int64_t stride_ym,
                            uint32_t* Bits, int64_t stride_bm, int64_t stride_bn, int64_t n_rows, int64_t n_expts_tot,
                            int K, int apply_softmax, hkq_stream_t stream) {
    HKQ_CHECK_ARG(n_rows >= 0 && n_rows <= INT32_MAX, "n_rows must be in [0, 2^31)");
    HKQ_CHECK_ARG(n_expts_tot >= 1 && n_expts_tot <= RT_MAX_EXPTS, "n_expts_tot must be in [1, 1024]");
    HKQ_CHECK_ARG(K >= 1 && K <= 16, "K must be in [1, 16]");
    HKQ_CHECK_ARG(stride_xm >= n_expts_tot || n_rows <= 1, "stride_xm must be >= n_expts_tot");
    HKQ_CHECK_ARG(stride_ym >= K || n_rows <= 1, "stride_ym must be >= K");
    HKQ_CHECK_ARG(Bits == nullptr || (stride_bm >= 0 && stride_bn >= 0), "bitmatrix strides must be non-negative");
    if (n_rows == 0) return 0;
    HKQ_CHECK_ARG(X && Yv && Yi, "X, Yv and Yi are required");
    HKQ_CHECK_ALIGN(X, 2);
    HKQ_CHECK_ALIGN(Yv, 2);
    HKQ_CHECK_ALIGN(Yi, 4);
    HKQ_CHECK_ALIGN(Bits, 4);
    TopkParams p{};
    p.X = (const uint16_t*)X;
    p.sxm = stride_xm;
    p.Yv = (uint16_t*)Yv;
    p.Yi = Yi;
    p.sym = stride_ym;
    p.bits = Bits;
    p.sbm = stride_bm;
    p.sbn = stride_bn;
    p.rows = (int)n_rows;
    p.E = (int)n_expts_tot;
    p.K = K;
    p.softmax = apply_softmax ? 1 : 0;
    p.nwords = (int)((n_expts_tot + 31) / 32);
    const int kmax = K <= 2 ? 2 : K <= 4 ? 4 : K <= 8 ? 8 : 16;
    const hipStream_t s = (hipStream_t)stream;
    // lanes per row: enough for at most 8 (E <= 32) or 16 logits per lane
    if (n_expts_tot <= 8) return launch_topk<1, 8>(p, kmax, s);
    if (n_expts_tot <= 16) return launch_topk<2, 8>(p, kmax, s);
    if (n_expts_tot <= 32) return launch_topk<4, 8>(p, kmax, s);
    if (n_expts_tot <= 64) return launch_topk<4, 16>(p, kmax, s);
    if (n_expts_tot <= 128) return launch_topk<8, 16>(p, kmax, s);
    if (n_expts_tot <= 256) return launch_topk<16, 16>(p, kmax, s);
    if (n_expts_tot <= 512) return launch_topk<32, 16>(p, kmax, s);
    return launch_topk<64, 16>(p, kmax, s);
}

extern "C" int hkq_sum_bitmatrix_rows(const uint32_t* B, int64_t shape_bm, int64_t stride_bm, int64_t stride_bn,
                                      uint32_t* Ret, uint32_t* Partials, int64_t stride_pm, int64_t stride_pn,
                                      int64_t shape_pn, int64_t shape_bn, hkq_stream_t stream) {
    HKQ_CHECK_ARG(Partials != nullptr || shape_bm == 0, "Partials is required (use hkq_sum_bitmatrix_rows_fused for totals only)");
    HKQ_CHECK_ARG(shape_pn >= 0, "shape_pn must be non-negative");
    return bitsum(B, shape_bm, stride_bm, stride_bn, Ret, Partials, stride_pm, stride_pn, shape_pn, shape_bn,
                  (hipStream_t)stream);
}

extern "C" int hkq_sum_bitmatrix_rows_fused(const uint32_t* B, int64_t shape_bm, int64_t stride_bm, int64_t stride_bn,
                                            uint32_t* Ret, int64_t n_blks_bitmatrix, hkq_stream_t stream) {
    return bitsum(B, shape_bm, stride_bm, stride_bn, Ret, nullptr, 0, 0, 0, n_blks_bitmatrix, (hipStream_t)stream);
}

extern "C" int hkq_expt_data_stage1(const int32_t* Hist, int32_t* TokenStart, int32_t* TileStart, uint32_t* MDTileInfo,
                                    int64_t n_expts_tot, int64_t max_num_tiles, int64_t n_gates, int tile_dim_log2,
                                    hkq_stream_t stream) {
    return expt_data(Hist, TokenStart, TileStart, MDTileInfo, n_expts_tot, max_num_tiles, n_gates, tile_dim_log2, 0,
                     (hipStream_t)stream);
}

extern "C" int hkq_expt_data_stage2(const int32_t* Hist, const int32_t* TileStart, uint32_t* TileInfo,
                                    int64_t n_expts_tot, int tile_dim_log2, hkq_stream_t stream) {
    return stage2(Hist, TileStart, TileInfo, n_expts_tot, tile_dim_log2, 0, INT32_MAX, (hipStream_t)stream);
}

extern "C" int hkq_expt_data_stage2_fused(const int32_t* Hist, const int32_t* TileStart, uint32_t* TileInfo,
                                          int64_t n_expts_tot, hkq_stream_t stream) {
    return stage2(Hist, TileStart, TileInfo, n_expts_tot, 0, 1, INT32_MAX, (hipStream_t)stream);
}

extern "C" int hkq_expt_data_compute(const int32_t* Hist, int32_t* TokenStart, int32_t* TileStart,
                                     uint32_t* MDTileInfo, int64_t n_expts_tot, int64_t max_num_tiles, int64_t n_gates,
                                     int tile_dim_log2, int use_fused_stage2, hkq_stream_t stream) {
    const hipStream_t s = (hipStream_t)stream;
    if (!use_fused_stage2)
        return expt_data(Hist, TokenStart, TileStart, MDTileInfo, n_expts_tot, max_num_tiles, n_gates, tile_dim_log2,
                         1, s);
    int rc = expt_data(Hist, TokenStart, TileStart, MDTileInfo, n_expts_tot, max_num_tiles, n_gates, tile_dim_log2, 0, s);
    return rc ? rc : stage2(Hist, TileStart, MDTileInfo, n_expts_tot, 0, 1, (int)max_num_tiles, s);
}

extern "C" int hkq_routing_compute_indx(int32_t* GatherIndx, int32_t* ScatterIndx, void* GateScal, const void* ExptScal,
                                        const int32_t* ExptIndx, const int32_t* PartialOffs, int64_t stride_pm,
                                        int64_t stride_pn, const int32_t* TokensStart, int64_t n_gates,
                                        int n_expts_act, hkq_stream_t stream) {
    HKQ_CHECK_ARG(PartialOffs != nullptr, "PartialOffs is required (use hkq_routing_compute_indx_fused without it)");
    return indx(GatherIndx, ScatterIndx, GateScal, ExptScal, ExptIndx, PartialOffs, stride_pm, stride_pn, TokensStart,
                n_gates, n_expts_act, (hipStream_t)stream);
}

extern "C" int hkq_routing_compute_indx_fused(int32_t* GatherIndx, int32_t* ScatterIndx, void* GateScal,
                                              const void* ExptScal, const int32_t* ExptIndx,
                                              const int32_t* TokensStart, int64_t n_gates, int n_expts_act,
                                              hkq_stream_t stream) {
    return indx(GatherIndx, ScatterIndx, GateScal, ExptScal, ExptIndx, nullptr, 0, 0, TokensStart, n_gates,
                n_expts_act, (hipStream_t)stream);
}

extern "C" int hkq_moe_align_block_size(const int32_t* topk_ids, int32_t* sorted_token_ids, int32_t* expert_ids,
                                        int32_t* tokens_cnts_buffer, int32_t* cumsum_buffer,
                                        int32_t* total_tokens_post_pad, int64_t num_experts, int64_t block_size,
                                        int64_t numel, hkq_stream_t stream) {
    HKQ_CHECK_ARG(num_experts >= 1 && num_experts <= RT_MAX_EXPTS, "num_experts must be in [1, 1024]");
    HKQ_CHECK_ARG(block_size >= 1 && block_size <= (1 << 20), "block_size must be in [1, 2^20]");
    HKQ_CHECK_ARG(numel >= 0 && numel <= INT32_MAX / 2, "numel must be in [0, 2^30)");
    HKQ_CHECK_ARG(tokens_cnts_buffer && cumsum_buffer && total_tokens_post_pad && (numel == 0 || (topk_ids && sorted_token_ids && expert_ids)),
                  "topk_ids, sorted_token_ids, expert_ids and the buffers are required");
    HKQ_CHECK_ALIGN(topk_ids, 4);
    HKQ_CHECK_ALIGN(sorted_token_ids, 4);
    HKQ_CHECK_ALIGN(expert_ids, 4);
    HKQ_CHECK_ALIGN(tokens_cnts_buffer, 4);
    HKQ_CHECK_ALIGN(cumsum_buffer, 4);
    HKQ_CHECK_ALIGN(total_tokens_post_pad, 4);
    const int64_t E = num_experts;
    // segments of a multiple of 256 ids; at most min(64, E + 1, 16384 / E) of
    // them, so the per-segment counts fit the reference's (E + 1) * E
    // workspace and the scatter kernel's LDS copy of them
    const int64_t maxseg = std::max<int64_t>(1, std::min<int64_t>({64, E + 1, AL_MAX_COUNTS / E}));
    int64_t seg = std::max<int64_t>(1024, (numel + maxseg - 1) / maxseg);
    seg = (seg + 255) / 256 * 256;
    const int64_t nseg = std::max<int64_t>(1, (numel + seg - 1) / seg);
    AlignParams p{};
    p.ids = topk_ids;
    p.sorted = sorted_token_ids;
    p.expert_ids = expert_ids;
    p.counts = tokens_cnts_buffer;
    p.cumsum = cumsum_buffer;
    p.total = total_tokens_post_pad;
    p.E = (int)E;
    p.bs = (int)block_size;
    p.numel = (int)numel;
    p.seg = (int)seg;
    p.nseg = (int)nseg;
    p.ebits = 0;
    while ((1ll << p.ebits) < E) ++p.ebits;
    const hipStream_t s = (hipStream_t)stream;
    const size_t lds = sizeof(int) * (size_t)(3 * E + 1 + nseg * E + AL_NW * E);
    static bool lds_set = false;  // the largest size any call can need, set once
    if (!lds_set) {
        const int most = (int)sizeof(int) * (3 * RT_MAX_EXPTS + 1 + AL_MAX_COUNTS + AL_NW * RT_MAX_EXPTS);
        const hipError_t e = hipFuncSetAttribute((const void*)align_scatter_kernel,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, most);
        if (e != hipSuccess) {
            ::hkq::set_error("hipFuncSetAttribute(align_scatter_kernel) failed: %s", hipGetErrorString(e));
            return (int)e;
        }
        lds_set = true;
    }
    align_count_kernel<<<(unsigned)nseg, 64 * AL_NW, 0, s>>>(p);
    int rc = hkq_launch_status();
    if (rc) return rc;
    align_scatter_kernel<<<(unsigned)nseg, 64 * AL_NW, lds, s>>>(p);
    return hkq_launch_status();
}
