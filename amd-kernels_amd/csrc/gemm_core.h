// gemm_core.h -- the CDNA4 scaled-MFMA GEMM main loop shared by the dense
// A8W8, block-scale, MXFP4 and MoE entry points.
//
// C[m, n] = sum_k A[m, k] * B[n, k]   (both operands K-contiguous, "NT")
//
// Work decomposition
//   * one workgroup per BM x BN tile of C (BM = WAVES_M*TM*32, BN = WAVES_N*TN*32);
//   * K is consumed in tiles of 128 bytes per row (128 FP8 or 256 FP4 values),
//     staged HBM -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging),
//     two LDS stages so the next tile streams in while the current one feeds
//     the matrix cores;
//   * each wave owns a (TM*32) x (TN*32) sub-tile held in TM*TN 32x32 fp32
//     accumulators of v_mfma_scale_f32_32x32x64_f8f6f4;
//   * the MFMA "A" operand is the B tile (rows n) and the MFMA "B" operand is
//     the A tile (rows m), so that a lane's accumulator registers hold four
//     consecutive n of one m -- the epilogue stores 8 bytes of bf16 per lane.
//
// LDS tile layout: row r (0..BM-1) of 128 bytes = 8 chunks of 16 bytes; logical
// chunk c lives at physical chunk c ^ (r & 7), so the 32 lanes of a fragment
// read (32 rows, same logical chunk) spread over all banks.
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

constexpr int KT_BYTES = 128;  // K-tile width in bytes per row
constexpr uint32_t OOB = 0x80000000u;  // buffer offset that always reads zero (num_records <= 2^31 - 1)

enum GemmMode { MODE_A8W8 = 0, MODE_BLOCKSCALE = 1, MODE_MXFP4 = 2 };

__device__ __forceinline__ int lds_swz(int r, int c) { return r * KT_BYTES + ((c ^ (r & 7)) << 4); }

// Issue the LDS-direct loads of one K-tile of one operand: ROWS rows of 128
// bytes. Wave w, instruction i fills LDS bytes [(i*NW + w)*1024, +1024): rows
// (i*NW + w)*8 + lane/8, physical chunk lane%8. row_off[i] is the byte offset
// of that row inside the buffer (OOB for rows past the edge); chunk_off is the
// lane's logical chunk * 16.
template <int ROWS, int NW>
__device__ __forceinline__ void load_tile_lds(__amdgpu_buffer_rsrc_t rsrc, HKQ_LDS uint8_t* lds, int wave,
                                              const uint32_t (&row_off)[ROWS / 8 / NW], uint32_t chunk_off,
                                              bool k_tail, uint32_t k_left) {
#pragma unroll
    for (int i = 0; i < ROWS / 8 / NW; ++i) {
        uint32_t off = row_off[i] + chunk_off;
        if (k_tail) off = chunk_off < k_left ? off : OOB;
        HKQ_LDS void* dst = lds + (i * NW + wave) * 1024;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, off, 0, 0, 0);
    }
}

// One LDS-direct load of `size` (4 or 16) bytes per lane from [base, base + bytes)
// at byte offset `off` to `dst` + lane * size. Kept out of lambdas: a target
// builtin called directly in a lambda inside a kernel template makes the host
// pass drop that kernel's launch stub without a diagnostic.
__device__ __forceinline__ void lds_load16(const void* base, uint32_t bytes, HKQ_LDS void* dst, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(base, bytes), dst, 16, off, 0, 0, 0);
}
__device__ __forceinline__ void lds_load4(const void* base, uint32_t bytes, HKQ_LDS void* dst, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(base, bytes), dst, 4, off, 0, 0, 0);
}

// Per-lane constants of the load pattern: the lane's row within its 8-row
// group and logical chunk (so that physical chunk = lane % 8).
__device__ __forceinline__ void load_lane_coords(int lane, int wave, int NW, int i, int& row, int& chunk) {
    row = (i * NW + wave) * 8 + (lane >> 3);
    chunk = (lane & 7) ^ (row & 7);
}

// Read the FP8 fragment (32 bytes: logical chunks c0, c0+1) of row r.
__device__ __forceinline__ v8i read_frag_fp8(const HKQ_LDS uint8_t* tile, int r, int c0) {
    const v4i lo = *reinterpret_cast<const HKQ_LDS v4i*>(tile + lds_swz(r, c0));
    const v4i hi = *reinterpret_cast<const HKQ_LDS v4i*>(tile + lds_swz(r, c0 + 1));
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Read the FP4 fragment (16 bytes: logical chunk c) of row r.
__device__ __forceinline__ v8i read_frag_fp4(const HKQ_LDS uint8_t* tile, int r, int c) {
    const v4i v = *reinterpret_cast<const HKQ_LDS v4i*>(tile + lds_swz(r, c));
    return v8i{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
}

template <bool FP4>
__device__ __forceinline__ v16f mfma(const v8i& a, const v8i& b, const v16f& c, int sa, int sb) {
    if (FP4) return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 4, 4, 0, sa, 0, sb);
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}

template <bool FP4, int OPA, int OPB>
__device__ __forceinline__ v16f mfma_sel(const v8i& a, const v8i& b, const v16f& c, int sa, int sb) {
    if (FP4) return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 4, 4, OPA, sa, OPB, sb);
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, OPA, sa, OPB, sb);
}

// Workgroup barrier that also waits for this wave's LDS-direct loads
// (vmcnt): __syncthreads' workgroup-scope fence does not cover the
// buffer_load ... lds writes, so without the explicit wait a wave could read a
// K-tile that another wave's loads have not finished writing.
__device__ __forceinline__ void tile_barrier() {
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
    __syncthreads();
}

// Wait states after the last MFMA before its accumulators are read by VALU or
// memory instructions when the reads sit in another basic block (the compiler
// under-counts the 16-pass FP8 form across block boundaries).
__device__ __forceinline__ void mfma_drain() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_sched_barrier(0); asm volatile("s_nop 15");
    __builtin_amdgcn_sched_barrier(0); asm volatile("s_nop 15");
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
