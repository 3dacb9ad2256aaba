// gemm_core.h -- building blocks of the CDNA4 scaled-MFMA GEMMs (dense A8W8,
// block-scale, MXFP4 and the MoE grouped GEMM).
//
// C[m, n] = sum_k A[m, k] * B[n, k]   (both operands K-contiguous, "NT")
//
// Shared design
//   * one workgroup per BM x BN tile of C; waves own (TM*32) x (TN*32) sub-tiles
//     held in TM*TN 32x32 fp32 accumulators of v_mfma_scale_f32_32x32x64_f8f6f4;
//   * K is consumed in K-tiles of KTB = 64 or 128 bytes per row (FP8: 64 or
//     128 values, FP4: twice that), staged HBM -> LDS with buffer_load_dwordx4
//     ... lds (no VGPR staging) into NS ring stages, so a tile is requested
//     NS-1 K-tiles before it is needed;
//   * the MFMA "A" operand is the B tile (rows n) and the MFMA "B" operand is
//     the A tile (rows m): a lane's accumulator registers then hold four
//     consecutive n of one m.
//
// LDS K-tile layout (KTB = 64 or 128 bytes of K per row, KTB/16 chunks of 16
// bytes): logical chunk c of row r lives at physical chunk c ^ f(r) with
// f(r) = (r >> 2) & 3 (KTB 64) or (r >> 1) & 7 (KTB 128). A fragment read has
// 16 lanes on 16 consecutive rows with one logical chunk; their 16-byte slots
// modulo 256 bytes are then all distinct, so the read is free of bank
// conflicts on the 64 x 4-byte LDS banks. A wave-wide LDS-direct load writes
// 1 KB = 1024/KTB rows contiguously: lane l carries row l / (KTB/16) of the
// load and physical chunk l % (KTB/16).
//
// Operand fragment layout of the 32x32x64 MFMA (verified on gfx950): lane l
// supplies row (l % 32) and the 32 K-values [32*(l/32), 32*(l/32)+32) of the
// instruction's 64-deep K slice; FP8 uses all 32 bytes (8 VGPRs), FP4 uses 16
// bytes (4 VGPRs). Output: lane l, register i holds D[8*(i/4) + 4*(l/32) + i%4][l%32].
// The e8m0 scale operand applies per lane (its row and its 32-value K block)
// with value 2^(code - 127); opsel picks the byte of the 32-bit scale VGPR.
#pragma once
#include "hkq_device.h"

namespace hkq {

constexpr uint32_t OOB = 0x80000000u;  // buffer offset that always reads zero (num_records <= 2^31 - 1)

enum GemmMode { MODE_A8W8 = 0, MODE_BLOCKSCALE = 1, MODE_MXFP4 = 2, MODE_BF16 = 3 };

template <int KTB>
struct KTile {
    static_assert(KTB == 64 || KTB == 128, "K-tile rows of 64 or 128 bytes");
    static constexpr int CHUNKS = KTB / 16;
    static constexpr int ROWS_PER_LOAD = 1024 / KTB;  // rows written by one wave-wide 16-byte LDS-direct load
    __device__ static __forceinline__ int phys(int r, int c) {
        return KTB == 64 ? (c ^ ((r >> 2) & 3)) : (c ^ ((r >> 1) & 7));
    }
    // LDS byte offset of logical chunk c of row r
    __device__ static __forceinline__ int swz(int r, int c) { return r * KTB + (phys(r, c) << 4); }
    // Logical chunk carried by `lane` of a load whose lane writes row r of the tile.
    __device__ static __forceinline__ int load_chunk(int lane, int r) { return phys(r, lane % CHUNKS); }
};

// One LDS-direct load of `size` (4 or 16) bytes per lane from [base, base + bytes)
// at byte offset `off` to `dst` + lane * size (buffer_load ... lds: M0 holds
// the wave-uniform LDS destination).
//
// Issued as inline assembly on purpose: the compiler's wait-count pass treats a
// builtin LDS-direct load as a pending LDS write that any later ds_read might
// alias and strengthens the pipeline's vmcnt(N) waits to vmcnt(0), which would
// serialize the K-tile ring. The kernels order these loads themselves: every
// read of a stage is preceded by tile_barrier<N>, whose vmcnt(N) covers the
// loads that filled it, and a vmcnt(0) barrier precedes any other use of the
// LDS or of the vector-memory counter after the main loop.
__device__ __forceinline__ v4i buffer_desc(const void* base, uint32_t bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    return v4i{(int)(uint32_t)b, (int)((uint32_t)(b >> 32) & 0xFFFFu), (int)bytes, 0x00020000};
}
__device__ __forceinline__ void lds_load16(const void* base, uint32_t bytes, HKQ_LDS void* dst, uint32_t off) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(m0), "v"(off), "s"(buffer_desc(base, bytes))
                 : "memory", "m0");
}
// lds_load16 with a prepared buffer descriptor (one per operand tile, built
// once outside the K loop; the K position then rides in the lane offset, so a
// load costs one VALU add instead of a descriptor's worth of scalar work).
__device__ __forceinline__ void lds_load16_d(const v4i& desc, HKQ_LDS void* dst, uint32_t off) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(m0), "v"(off), "s"(desc)
                 : "memory", "m0");
}
// lds_load16 whose buffer descriptor is made wave-uniform explicitly: for
// sources the compiler cannot prove uniform (a source switched inside a loop),
// which would otherwise land in VGPRs and fail the instruction's SGPR operand.
__device__ __forceinline__ void lds_load16_u(const void* base, uint32_t bytes, HKQ_LDS void* dst, uint32_t off) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint32_t n = __builtin_amdgcn_readfirstlane(bytes);
    lds_load16(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo), n, dst, off);
}
__device__ __forceinline__ void lds_load4(const void* base, uint32_t bytes, HKQ_LDS void* dst, uint32_t off) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(m0), "v"(off), "s"(buffer_desc(base, bytes))
                 : "memory", "m0");
}

__device__ __forceinline__ v4i lds_read16(const HKQ_LDS uint8_t* p) { return *reinterpret_cast<const HKQ_LDS v4i*>(p); }

// N-contiguous ("transposed") B tiles: the weights of a K-tile stored as they
// lie in memory, 128 rows of K, each holding the tile's 256 output columns
// (256 bytes). Logical 16-byte chunk c of row r lives at physical chunk
// c ^ (2 * (r & 7)): the transposed reads below touch 8 consecutive rows at
// two adjacent logical chunks per 32 lanes, which then fall on 16 distinct
// chunk slots (all 64 banks).
struct KTileT {
    static constexpr int ROW = 256, ROWS = 128;
    static constexpr int ROWS_PER_LOAD = 1024 / ROW;  // rows written by one wave-wide 16-byte LDS-direct load
    __device__ static __forceinline__ int phys(int r, int c) { return c ^ (2 * (r & 7)); }
};

// ds_read_b64_tr_b8 (measured on gfx950): in each group of 16 lanes, lane j
// receives byte (j & 7) of the 8-byte pieces addressed by lanes 2i + (j >> 3),
// i = 0..7, as its bytes i. With lanes 2i and 2i + 1 addressing the two halves
// of row i's 16 bytes, lane j receives column j of 8 consecutive rows.
__device__ __forceinline__ v2i lds_read_tr8(const HKQ_LDS uint8_t* p) {
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32(reinterpret_cast<HKQ_LDS v2i*>(const_cast<HKQ_LDS uint8_t*>(p)));
}

template <bool FP4, int OPA, int OPB>
__device__ __forceinline__ v16f mfma_sel(const v8i& a, const v8i& b, const v16f& c, int sa, int sb) {
    if (FP4) return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 4, 4, OPA, sa, OPB, sb);
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, OPA, sa, OPB, sb);
}

// bf16 operands: 8 values (16 bytes) per lane, one 16-deep MFMA.
typedef __bf16 v8bf16 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ v16f mfma_bf16(const v4i& a, const v4i& b, const v16f& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf16, a), __builtin_bit_cast(v8bf16, b), c, 0, 0,
                                                  0);
}

// s_waitcnt immediate (gfx9 encoding): vmcnt in [3:0] and [15:14], expcnt in
// [6:4], lgkmcnt in [11:8].
constexpr int waitcnt_imm(int vm, int lgkm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | ((lgkm & 15) << 8); }

// Workgroup barrier that first waits until at most VM of this wave's vector
// memory operations are outstanding and all its LDS operations are done.
// __syncthreads' workgroup-scope fence does not cover buffer_load ... lds, so
// the explicit vmcnt wait is what makes another wave's K-tile visible.
template <int VM>
__device__ __forceinline__ void tile_barrier() {
    static_assert(VM >= 0 && VM <= 63, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(VM, 0));
    __syncthreads();
}

// Workgroup barrier after this wave's LDS operations are done; vector memory
// operations (e.g. stores still draining) are not waited for.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
    __syncthreads();
}

// Wait states after the last MFMA before its accumulators are read by VALU or
// memory instructions when the reads sit in another basic block (the compiler
// under-counts the 16-pass FP8 form across block boundaries).
__device__ __forceinline__ void mfma_drain() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 15");
    asm volatile("s_nop 15");
    __builtin_amdgcn_sched_barrier(0);
}

// Map a 1-D workgroup id to a (tile_m, tile_n) pair: first undo the round-robin
// dispatch over the 8 XCDs so each XCD gets a contiguous range of ids, then walk
// that range in column groups of GROUP_M tile rows so that concurrently resident
// workgroups of one XCD share A rows and B columns in that XCD's L2.
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
    const int nblk = tiles_m * tiles_n;
    const int q = nblk >> 3, rem = nblk & 7;
    const int xcd = bid & 7, idx = bid >> 3;
    bid = xcd < rem ? xcd * (q + 1) + idx : rem * (q + 1) + (xcd - rem) * q + idx;
    const int per_group = group_m * tiles_n;
    const int g = bid / per_group;
    const int first_m = g * group_m;
    const int gsize = min(tiles_m - first_m, group_m);
    const int in_g = bid - g * per_group;
    tm = first_m + in_g % gsize;
    tn = in_g / gsize;
}

// Epilogue shared by the GEMMs: scale in registers, stage each wave's bf16
// (TM*32) x (TN*32) sub-tile in LDS (row m, col n, row pitch TN*64 + 16 bytes),
// then store whole row segments of C (TN*64 bytes: 128 or 256; 16-byte stores
// when C's rows are 16-byte aligned, else two 8-byte stores; N % 4 == 0). The caller has retired
// every LDS use of the main loop (a vmcnt(0) barrier) before calling.
//   acc[i][j]: accumulator of n-tile i, m-tile j, D[n][m] layout
//   (lane: m = lane & 31; register r: n = 8*(r/4) + 4*(lane/32) + r%4);
//   row_scale(j) -> scale of the lane's m in m-tile j; col_scale4(i, g) -> the
//   4 scales of n = i*32 + 8g + 4*(lane/32) + 0..3 (both relative to the wave);
//   col_bias4(i, g) -> the 4 values added after scaling (zero when unused).
// Element-wise step after scaling: elem(j, i, g, v) maps the lane's 4 values v
// of m-tile j, n-tile i, register group g; the default leaves them unchanged.
// Bias of an epilogue without one: -0 is the additive identity for every
// value (x + -0 == x, also for x = -0), so the compiler drops the add.
struct NoBias {
    __device__ float4 operator()(int, int) const { return make_float4(-0.f, -0.f, -0.f, -0.f); }
};

// Element-wise hook of the epilogue: prefetch(i) runs before the values of
// n-tile i are formed (so a hook that reads memory can issue all of that
// tile's loads at once), then operator()(j, i, g, v) maps the scaled fp32
// values v of m-tile j, column group g before the bf16 conversion.
struct NoElem {
    __device__ void prefetch(int) {}
    __device__ float4 operator()(int, int, int, float4 v) const { return v; }
};

// Scale, convert and stage the wave's (TM*32) x (TN*32) sub-tile in LDS as bf16
// rows of PITCH bytes (returns the wave's staging area).
template <int TM, int TN, typename RowScale, typename ColScale4, typename ColBias4, typename Elem = NoElem>
__device__ __forceinline__ HKQ_LDS uint8_t* stage_tile_bf16(v16f (&acc)[TN][TM], HKQ_LDS uint8_t* smem, int wave,
                                                            int lane, RowScale row_scale, ColScale4 col_scale4,
                                                            ColBias4 col_bias4, Elem elem = Elem{}) {
    constexpr int PITCH = TN * 32 * 2 + 16;
    static_assert((TN * 32 * 2) % 128 == 0, "rows are whole 128-byte segments");
    HKQ_LDS uint8_t* ep = smem + wave * (TM * 32) * PITCH;
    const int khalf = lane >> 5;
    float rs[TM];
#pragma unroll
    for (int j = 0; j < TM; ++j) rs[j] = row_scale(j);
#pragma unroll
    for (int i = 0; i < TN; ++i) {
        elem.prefetch(i);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int nl = i * 32 + 8 * g + 4 * khalf;
            const float4 cs = col_scale4(i, g);
            const float4 cb = col_bias4(i, g);
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const float a = rs[j];
                const float4 v = elem(j, i, g,
                                      make_float4(acc[i][j][4 * g + 0] * a * cs.x + cb.x, acc[i][j][4 * g + 1] * a * cs.y + cb.y,
                                                  acc[i][j][4 * g + 2] * a * cs.z + cb.z, acc[i][j][4 * g + 3] * a * cs.w + cb.w));
                const uint32_t lo = pk_bf16(v.x, v.y);
                const uint32_t hi = pk_bf16(v.z, v.w);
                *reinterpret_cast<HKQ_LDS v2i*>(ep + (j * 32 + (lane & 31)) * PITCH + nl * 2) = v2i{(int)lo, (int)hi};
            }
        }
    }
    return ep;
}

// One 16-byte piece (8 bf16) of a staged row to dst, of which n_left columns
// are inside C (N % 4 == 0: a piece is whole, half or out of range). The C
// stores of the epilogues are non-temporal: no kernel here reads C back, and
// written whole lines at a time they go out merged while the operands keep
// the caches (measured on MI355X: the MXFP4 MoE at Mixtral size 2.5-3.5%
// faster, the block-scale multiply-add epilogue 3%, the MXFP4 and block-scale
// GEMMs within 1%).
__device__ __forceinline__ void store_piece_bf16(uint16_t* dst, const v4i& v, int n_left, bool c16) {
    if (n_left >= 8) {
        if (c16) {
            __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(dst));
        } else {
            __builtin_nontemporal_store(v2i{v[0], v[1]}, reinterpret_cast<v2i*>(dst));
            __builtin_nontemporal_store(v2i{v[2], v[3]}, reinterpret_cast<v2i*>(dst + 4));
        }
    } else if (n_left > 0) {
        __builtin_nontemporal_store(v2i{v[0], v[1]}, reinterpret_cast<v2i*>(dst));
    }
}

template <int TM, int TN, typename RowScale, typename ColScale4, typename ColBias4, typename Elem = NoElem>
__device__ __forceinline__ void store_tile_bf16(v16f (&acc)[TN][TM], HKQ_LDS uint8_t* smem, int wave, int lane,
                                                uint16_t* C, int64_t ldc, int M, int N, int mw, int nw, bool c16,
                                                RowScale row_scale, ColScale4 col_scale4, ColBias4 col_bias4,
                                                Elem elem = Elem{}) {
    constexpr int PITCH = TN * 32 * 2 + 16;
    HKQ_LDS uint8_t* ep = stage_tile_bf16<TM, TN>(acc, smem, wave, lane, row_scale, col_scale4, col_bias4, elem);
    // LDS operations of a wave complete in order: the reads below see the writes above.
    constexpr int SEGS = TN * 32 * 2 / 16;  // 16-byte pieces per row
    constexpr int ROWS_PER_PASS = 64 / SEGS;
    constexpr int PASSES = TM * 32 / ROWS_PER_PASS;
    constexpr int BATCH = PASSES < 8 ? PASSES : 8;  // LDS reads in flight before their stores
    static_assert(PASSES % BATCH == 0, "whole batches");
    // derived from an opaque copy of the lane: otherwise the compiler computes
    // rl / seg in the kernel's prologue and keeps them live (or spilled)
    // through the main loop
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int rl = ln / SEGS, seg = ln % SEGS;
    if (c16 && mw + TM * 32 <= M && nw + TN * 32 <= N) {
        // the wave's sub-tile lies inside C: no per-piece checks
        uint16_t* dst = C + (int64_t)(mw + rl) * ldc + nw + seg * 8;
        const int64_t step = (int64_t)ROWS_PER_PASS * ldc;
#pragma unroll
        for (int b = 0; b < PASSES; b += BATCH) {
            v4i v[BATCH];
#pragma unroll
            for (int k = 0; k < BATCH; ++k) v[k] = lds_read16(ep + ((b + k) * ROWS_PER_PASS + rl) * PITCH + seg * 16);
#pragma unroll
            for (int k = 0; k < BATCH; ++k) __builtin_nontemporal_store(v[k], reinterpret_cast<v4i*>(dst + (b + k) * step));
        }
        return;
    }
#pragma unroll 4
    for (int r0 = 0; r0 < TM * 32; r0 += ROWS_PER_PASS) {
        const int r = r0 + rl;
        const v4i v = lds_read16(ep + r * PITCH + seg * 16);
        const int m = mw + r;
        const int n = nw + seg * 8;
        if (m < M) store_piece_bf16(C + (int64_t)m * ldc + n, v, N - n, c16);
    }
}

// As store_tile_bf16, with the rows scattered: wave row r (0 .. TM*32-1) goes
// to C row row_of(r), or nowhere when row_of(r) < 0.
template <int TM, int TN, typename RowOf, typename RowScale, typename ColScale4, typename ColBias4>
__device__ __forceinline__ void store_tile_bf16_rows(v16f (&acc)[TN][TM], HKQ_LDS uint8_t* smem, int wave, int lane,
                                                     uint16_t* C, int64_t ldc, int N, int nw, bool c16, RowOf row_of,
                                                     RowScale row_scale, ColScale4 col_scale4, ColBias4 col_bias4) {
    constexpr int PITCH = TN * 32 * 2 + 16;
    HKQ_LDS uint8_t* ep = stage_tile_bf16<TM, TN>(acc, smem, wave, lane, row_scale, col_scale4, col_bias4);
    constexpr int SEGS = TN * 32 * 2 / 16;
    constexpr int ROWS_PER_PASS = 64 / SEGS;
    constexpr int PASSES = TM * 32 / ROWS_PER_PASS;
    constexpr int BATCH = PASSES < 8 ? PASSES : 8;
    static_assert(PASSES % BATCH == 0, "whole batches");
    int ln = lane;  // opaque copy: keeps rl / seg out of the kernel's prologue
    asm volatile("" : "+v"(ln));
    const int rl = ln / SEGS, seg = ln % SEGS;
    if (c16 && nw + TN * 32 <= N) {
        // whole pieces: a batch's LDS reads and row ids are all in flight
        // before its stores. Measured on MI355X (MXFP4 MoE, Mixtral gate/up):
        // a 256-row tile's store loop 4.4 -> 2.9 us against one pass at a
        // time (each waiting on its read and its row id), the GEMM 0.589 ->
        // 0.576 ms; batches of 16 are no faster, write-back stores slower.
        uint16_t* cn = C + nw + seg * 8;
#pragma unroll
        for (int b = 0; b < PASSES; b += BATCH) {
            v4i v[BATCH];
            int64_t m[BATCH];
#pragma unroll
            for (int k = 0; k < BATCH; ++k) v[k] = lds_read16(ep + ((b + k) * ROWS_PER_PASS + rl) * PITCH + seg * 16);
#pragma unroll
            for (int k = 0; k < BATCH; ++k) m[k] = row_of((b + k) * ROWS_PER_PASS + rl);
#pragma unroll
            for (int k = 0; k < BATCH; ++k)
                if (m[k] >= 0) __builtin_nontemporal_store(v[k], reinterpret_cast<v4i*>(cn + m[k] * ldc));
        }
        return;
    }
#pragma unroll 4
    for (int r0 = 0; r0 < TM * 32; r0 += ROWS_PER_PASS) {
        const int r = r0 + rl;
        const v4i v = lds_read16(ep + r * PITCH + seg * 16);
        const int64_t m = row_of(r);
        const int n = nw + seg * 8;
        if (m >= 0) store_piece_bf16(C + m * ldc + n, v, N - n, c16);
    }
}

}  // namespace hkq
