// gemm_core.h -- building blocks of the CDNA4 scaled-MFMA GEMMs (dense A8W8,
// block-scale, MXFP4 and the MoE grouped GEMM).
//
// C[m, n] = sum_k A[m, k] * B[n, k]   (both operands K-contiguous, "NT")
//
// Shared design
//   * one workgroup per BM x BN tile of C; waves own (TM*32) x (TN*32) sub-tiles
//     held in TM*TN 32x32 fp32 accumulators of v_mfma_scale_f32_32x32x64_f8f6f4;
//   * K is consumed in K-tiles of 64 bytes per row (64 FP8 or 128 FP4 values),
//     staged HBM -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging) into
//     NS ring stages, so a tile is requested NS-1 K-tiles before it is needed;
//   * the MFMA "A" operand is the B tile (rows n) and the MFMA "B" operand is
//     the A tile (rows m): a lane's accumulator registers then hold four
//     consecutive n of one m.
//
// LDS K-tile layout: row r of 64 bytes = 4 chunks of 16 bytes; logical chunk c
// lives at physical chunk c ^ ((r >> 2) & 3). A fragment read has 16 lanes on
// 16 consecutive rows with one logical chunk; their 16-byte slots
// (r & 3) * 4 + (c ^ ((r >> 2) & 3)) modulo 256 bytes are all distinct, so the
// read is free of bank conflicts on the 64 x 4-byte LDS banks. A wave-wide
// LDS-direct load writes 1 KB = 16 rows contiguously; lane l carries row l/4,
// physical chunk l%4, hence logical chunk (l & 3) ^ ((l >> 4) & 3).
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

constexpr int KT_BYTES = 64;           // K-tile width in bytes per row
constexpr int ROWS_PER_LOAD = 16;      // rows written by one wave-wide 16-byte LDS-direct load
constexpr uint32_t OOB = 0x80000000u;  // buffer offset that always reads zero (num_records <= 2^31 - 1)

enum GemmMode { MODE_A8W8 = 0, MODE_BLOCKSCALE = 1, MODE_MXFP4 = 2 };

__device__ __forceinline__ int lds_swz(int r, int c) { return r * KT_BYTES + ((c ^ ((r >> 2) & 3)) << 4); }

// Logical chunk carried by `lane` in a wave-wide LDS-direct load.
__device__ __forceinline__ int load_chunk(int lane) { return (lane & 3) ^ ((lane >> 4) & 3); }

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
__device__ __forceinline__ void lds_load4(const void* base, uint32_t bytes, HKQ_LDS void* dst, uint32_t off) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(m0), "v"(off), "s"(buffer_desc(base, bytes))
                 : "memory", "m0");
}

__device__ __forceinline__ v4i lds_read16(const HKQ_LDS uint8_t* p) { return *reinterpret_cast<const HKQ_LDS v4i*>(p); }

template <bool FP4, int OPA, int OPB>
__device__ __forceinline__ v16f mfma_sel(const v8i& a, const v8i& b, const v16f& c, int sa, int sb) {
    if (FP4) return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 4, 4, OPA, sa, OPB, sb);
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, OPA, sa, OPB, sb);
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

}  // namespace hkq
