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
//   hkq_gemm_blockscale  C = bf16(sum_kt (A_kt . B_kt^T) * sa[m,kt] * sb[kt,n/128])
//                        with 128-wide K groups (gemm_a8w8_blockscale/kernel.cpp:
//                        129-153; formula gemm_a8w8_blockscale/test_parity.py:57-76).
#include "gemm_core.h"
#include "hkq_host.h"

namespace hkq {

struct DenseParams {
    const uint8_t* A;
    const uint8_t* B;
    uint16_t* C;
    const void* sa;
    const void* sb;
    int M, N, K;          // K in elements
    int kbytes;           // K in bytes per row of A/B
    int64_t lda, ldb;     // bytes
    int64_t ldc;          // elements
    int64_t lsa, lsb;     // scale row strides (MXFP4: bytes; block-scale: floats)
    int tiles_m, tiles_n, group_m;
};

// Pipeline (per wave; one barrier per K-tile):
//   tile kt is consumed in SUB MFMA K-steps of 64 values (FP8: 2, FP4: 4);
//   fragments are double-buffered, so the LDS reads of step s+1 are issued
//   between the MFMAs of step s; half of the last step's MFMAs are issued before
//   the barrier (keeping the matrix pipe busy while waves meet), which (a) makes
//   tile kt+1's LDS-direct loads visible and (b) retires every wave's reads of
//   tile kt's stage; the other half is interleaved with the loads that refill
//   that stage with tile kt+2 and the reads of step 0 of tile kt+1. Chunks are
//   separated by sched_barrier so the compiler keeps this order.
template <int MODE, int WAVES_M, int WAVES_N, int TM, int TN>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N, 1) void dense_gemm_kernel(const DenseParams p) {
    constexpr int NW = WAVES_M * WAVES_N;
    constexpr int BM = WAVES_M * TM * 32, BN = WAVES_N * TN * 32;
    constexpr int LA = BM / 8 / NW, LB = BN / 8 / NW;
    constexpr bool FP4 = MODE == MODE_MXFP4;
    constexpr int SUB = FP4 ? 4 : 2;
    // FP4: the tile's e8m0 scales (8 bytes per row per K-tile) ride in LDS after the data
    constexpr int SCA = FP4 ? BM * 8 : 0, SCB = FP4 ? BN * 8 : 0;
    constexpr int LSA = FP4 ? BM / 32 / NW : 0, LSB = FP4 ? BN / 32 / NW : 0;
    constexpr int STAGE = (BM + BN) * KT_BYTES + SCA + SCB;
    constexpr int NLD = LA + LB + LSA + LSB;           // LDS-direct loads per K-tile
    constexpr int PARTS = FP4 ? 1 : 2;                 // ds_read_b128 per fragment
    constexpr int NRD = (TM + TN) * PARTS;             // fragment reads per K-step
    constexpr int NSC = FP4 ? TM + TN : 0;             // scale reads per K-tile
    constexpr int NMF = TM * TN;                       // MFMAs per K-step
    constexpr int HALF = NMF / 2;
    static_assert(LA >= 1 && LB >= 1, "tile too small for the wave count");
    static_assert(!FP4 || (LSA >= 1 && LSB >= 1), "scale tile too small for the wave count");
    static_assert(NRD <= NMF, "phase A pairs at most one fragment read with each MFMA");

    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int rows_a = min(p.M - m0, BM), rows_b = min(p.N - n0, BN);

    // global -> LDS load pattern (identical logical chunk for every instruction of a lane)
    const uint32_t chunk_off = (uint32_t)(((lane & 7) ^ (lane >> 3)) << 4);
    uint32_t a_off[LA], b_off[LB];
#pragma unroll
    for (int i = 0; i < LA; ++i) a_off[i] = (uint32_t)(((i * NW + wave) * 8 + (lane >> 3)) * p.lda);
#pragma unroll
    for (int i = 0; i < LB; ++i) b_off[i] = (uint32_t)(((i * NW + wave) * 8 + (lane >> 3)) * p.ldb);
    const uint8_t* a_base = p.A + (int64_t)m0 * p.lda;
    const uint8_t* b_base = p.B + (int64_t)n0 * p.ldb;
    const int64_t a_bytes = min((int64_t)rows_a * p.lda, (int64_t)0x7FFFFFFF);
    const int64_t b_bytes = min((int64_t)rows_b * p.ldb, (int64_t)0x7FFFFFFF);
    const uint8_t* as_base = FP4 ? static_cast<const uint8_t*>(p.sa) + (int64_t)m0 * p.lsa : nullptr;
    const uint8_t* bs_base = FP4 ? static_cast<const uint8_t*>(p.sb) + (int64_t)n0 * p.lsb : nullptr;
    const int64_t as_bytes = FP4 ? min((int64_t)rows_a * p.lsa, (int64_t)0x7FFFFFFF) : 0;
    const int64_t bs_bytes = FP4 ? min((int64_t)rows_b * p.lsb, (int64_t)0x7FFFFFFF) : 0;
    const int KT = (p.kbytes + KT_BYTES - 1) / KT_BYTES;

    // Where tile kt's loads come from; for kt >= KT all sizes are zero, so every
    // load reads zero (keeps the main loop free of branches). Plain fields only:
    // the buffer resources are built per load (a few scalar instructions).
    struct TileLoad {
        const uint8_t *a, *b, *sa, *sb;
        uint32_t na, nb, nsa, nsb, left;
        int stage;
        bool tail;
    };
    auto tile_load = [&](int kt, int stage) {
        TileLoad T;
        const int kb = kt * KT_BYTES;
        const bool live = kt < KT;
        T.tail = kb + KT_BYTES > p.kbytes;
        T.left = (uint32_t)(p.kbytes - kb);
        T.a = a_base + kb;
        T.b = b_base + kb;
        T.na = live ? (uint32_t)max(a_bytes - kb, (int64_t)0) : 0u;
        T.nb = live ? (uint32_t)max(b_bytes - kb, (int64_t)0) : 0u;
        T.sa = as_base + kt * 8;
        T.sb = bs_base + kt * 8;
        T.nsa = (FP4 && live) ? (uint32_t)max(as_bytes - kt * 8, (int64_t)0) : 0u;
        T.nsb = (FP4 && live) ? (uint32_t)max(bs_bytes - kt * 8, (int64_t)0) : 0u;
        T.stage = stage;
        return T;
    };
    // Load instruction idx of a tile: A rows, B rows, then (FP4) 4-byte scale
    // words, row = (i*NW + wave)*32 + lane/2, half = lane & 1.
    auto load_piece = [&](const TileLoad& T, int idx) {
        HKQ_LDS uint8_t* st = smem + T.stage * STAGE;
        if (idx < LA) {
            uint32_t off = a_off[idx] + chunk_off;
            if (T.tail) off = chunk_off < T.left ? off : OOB;
            lds_load16(T.a, T.na, st + (idx * NW + wave) * 1024, off);
        } else if (idx < LA + LB) {
            const int i = idx - LA;
            uint32_t off = b_off[i] + chunk_off;
            if (T.tail) off = chunk_off < T.left ? off : OOB;
            lds_load16(T.b, T.nb, st + BM * KT_BYTES + (i * NW + wave) * 1024, off);
        } else if (idx < LA + LB + LSA) {
            const int i = idx - LA - LB;
            const uint32_t off = (uint32_t)(((i * NW + wave) * 32 + (lane >> 1)) * p.lsa + (lane & 1) * 4);
            lds_load4(T.sa, T.nsa, st + (BM + BN) * KT_BYTES + (i * NW + wave) * 256, off);
        } else {
            const int i = idx - LA - LB - LSA;
            const uint32_t off = (uint32_t)(((i * NW + wave) * 32 + (lane >> 1)) * p.lsb + (lane & 1) * 4);
            lds_load4(T.sb, T.nsb, st + (BM + BN) * KT_BYTES + SCA + (i * NW + wave) * 256, off);
        }
    };

    const int arow = wm * TM * 32 + (lane & 31);
    const int brow = wn * TN * 32 + (lane & 31);
    const int khalf = lane >> 5;

    struct Frags {
        v4i a[TM][PARTS], b[TN][PARTS];
    };
    // Fragment read idx of K-step ks: A tiles then B tiles, PARTS 16-byte chunks each
    // (FP8: logical chunks ks*4 + 2*khalf + part; FP4: chunk ks*2 + khalf).
    auto read_piece = [&](int stage, int ks, Frags& f, int idx) {
        const HKQ_LDS uint8_t* At = smem + stage * STAGE;
        const bool isa = idx < TM * PARTS;
        const int t = (isa ? idx : idx - TM * PARTS) / PARTS, part = idx % PARTS;
        const int row = (isa ? arow : brow) + t * 32;
        const int chunk = FP4 ? ks * 2 + khalf : ks * 4 + khalf * 2 + part;
        const v4i v = *reinterpret_cast<const HKQ_LDS v4i*>(At + (isa ? 0 : BM * KT_BYTES) + lds_swz(row, chunk));
        if (isa) f.a[t][part] = v;
        else f.b[t][part] = v;
    };
    // MXFP4: per m/n-tile the 8 scale bytes of the tile for the lane's row,
    // shifted so bytes 0 and 2 of word w are the lane's K-block of steps 2w, 2w+1.
    struct Scales {
        int a[TM][2], b[TN][2];
    };
    auto read_scale = [&](int stage, Scales& s, int idx) {
        if constexpr (FP4) {
            const HKQ_LDS uint8_t* sca = smem + stage * STAGE + (BM + BN) * KT_BYTES;
            const bool isa = idx < TM;
            const int t = isa ? idx : idx - TM;
            const v2i v = *reinterpret_cast<const HKQ_LDS v2i*>(sca + (isa ? (arow + t * 32) * 8 : SCA + (brow + t * 32) * 8));
            const int sh = khalf * 8;
            if (isa) { s.a[t][0] = (int)((uint32_t)v[0] >> sh); s.a[t][1] = (int)((uint32_t)v[1] >> sh); }
            else { s.b[t][0] = (int)((uint32_t)v[0] >> sh); s.b[t][1] = (int)((uint32_t)v[1] >> sh); }
        }
    };

    v16f acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = v16f{};

    auto frag8 = [](const v4i (&h)[PARTS]) -> v8i {
        if constexpr (PARTS == 2) return v8i{h[0][0], h[0][1], h[0][2], h[0][3], h[1][0], h[1][1], h[1][2], h[1][3]};
        else return v8i{h[0][0], h[0][1], h[0][2], h[0][3], 0, 0, 0, 0};
    };
    // MFMA idx (accumulator i*TM + j) of K-step ks
    auto mfma_one = [&](const Frags& f, int ks, const Scales& s, int idx) {
        const int i = idx / TM, j = idx % TM;
        if constexpr (FP4) {
            if (ks & 1)
                acc[i][j] = mfma_sel<true, 2, 2>(frag8(f.b[i]), frag8(f.a[j]), acc[i][j], s.b[i][ks >> 1], s.a[j][ks >> 1]);
            else
                acc[i][j] = mfma_sel<true, 0, 0>(frag8(f.b[i]), frag8(f.a[j]), acc[i][j], s.b[i][ks >> 1], s.a[j][ks >> 1]);
        } else {
            acc[i][j] = mfma<false>(frag8(f.b[i]), frag8(f.a[j]), acc[i][j], 127, 127);
        }
    };

    Frags F[2];
    Scales S[2];
    {
        const TileLoad T0 = tile_load(0, 0), T1 = tile_load(1, 1);
#pragma unroll
        for (int i = 0; i < NLD; ++i) load_piece(T0, i);
#pragma unroll
        for (int i = 0; i < NLD; ++i) load_piece(T1, i);
    }
    tile_barrier();  // start-up only: both prologue tiles resident
#pragma unroll
    for (int i = 0; i < NRD; ++i) read_piece(0, 0, F[0], i);
#pragma unroll
    for (int i = 0; i < NSC; ++i) read_scale(0, S[0], i);

    for (int kt = 0; kt < KT; ++kt) {
        const int stage = kt & 1;
        // phase A: steps 0 .. SUB-2, one fragment read of the next step per MFMA
#pragma unroll
        for (int ks = 0; ks + 1 < SUB; ++ks) {
#pragma unroll
            for (int c = 0; c < NMF; ++c) {
                mfma_one(F[ks & 1], ks, S[0], c);
                if (c < NRD) read_piece(stage, ks + 1, F[(ks + 1) & 1], c);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // phase B: last step
        constexpr int LAST = SUB - 1;
#pragma unroll
        for (int c = 0; c < HALF; ++c) mfma_one(F[LAST & 1], LAST, S[0], c);
        __builtin_amdgcn_sched_barrier(0);
        tile_barrier();  // retires this stage's reads everywhere; tile kt+1 is resident
        __builtin_amdgcn_sched_barrier(0);
        const TileLoad T = tile_load(kt + 2, stage);
#pragma unroll
        for (int c = 0; c < HALF; ++c) {
            mfma_one(F[LAST & 1], LAST, S[0], HALF + c);
#pragma unroll
            for (int i = c * NLD / HALF; i < (c + 1) * NLD / HALF; ++i) load_piece(T, i);
#pragma unroll
            for (int i = c * NRD / HALF; i < (c + 1) * NRD / HALF; ++i) read_piece(stage ^ 1, 0, F[0], i);
#pragma unroll
            for (int i = c * NSC / HALF; i < (c + 1) * NSC / HALF; ++i) read_scale(stage ^ 1, S[1], i);
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (FP4) S[0] = S[1];
    }
    mfma_drain();

    // Epilogue: lane holds, for m-tile j and n-tile i, D[n][m] with
    // m = (lane & 31), n = 8*(r/4) + 4*(lane/32) + r%4.
    const float* sa = static_cast<const float*>(p.sa);
    const float* sb = static_cast<const float*>(p.sb);
    float ascale[TM];
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int m = m0 + arow + j * 32;
        ascale[j] = (MODE == MODE_A8W8 && m < p.M) ? sa[m] : 1.0f;
    }
#pragma unroll
    for (int i = 0; i < TN; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = n0 + wn * TN * 32 + i * 32 + 8 * g + 4 * khalf;
            if (n >= p.N) continue;
            float4 bs = make_float4(1.f, 1.f, 1.f, 1.f);
            if constexpr (MODE == MODE_A8W8) bs = *reinterpret_cast<const float4*>(sb + n);
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int m = m0 + arow + j * 32;
                if (m >= p.M) continue;
                const float a = ascale[j];
                uint32_t lo = f32_to_bf16(acc[i][j][4 * g + 0] * a * bs.x) | (f32_to_bf16(acc[i][j][4 * g + 1] * a * bs.y) << 16);
                uint32_t hi = f32_to_bf16(acc[i][j][4 * g + 2] * a * bs.z) | (f32_to_bf16(acc[i][j][4 * g + 3] * a * bs.w) << 16);
                *reinterpret_cast<uint2*>(p.C + (int64_t)m * p.ldc + n) = make_uint2(lo, hi);
            }
        }
    }
}

template <int MODE, int WAVES_M, int WAVES_N, int TM, int TN>
static int launch_dense(DenseParams& p, hipStream_t stream) {
    constexpr int BM = WAVES_M * TM * 32, BN = WAVES_N * TN * 32;
    constexpr int SC = MODE == MODE_MXFP4 ? (BM + BN) * 8 : 0;
    constexpr int LDS = 2 * ((BM + BN) * KT_BYTES + SC);
    auto kern = dense_gemm_kernel<MODE, WAVES_M, WAVES_N, TM, TN>;
    static bool attr_set = false;  // per instantiation; the attribute is per-process
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
        if (e != hipSuccess) {
            set_error("hipFuncSetAttribute(MaxDynamicSharedMemorySize=%d) failed: %s", LDS, hipGetErrorString(e));
            return (int)e;
        }
        attr_set = true;
    }
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + BN - 1) / BN;
    if (p.group_m <= 0) p.group_m = 8;
    const int64_t nblk = (int64_t)p.tiles_m * p.tiles_n;
    if (nblk == 0) return 0;
    kern<<<dim3((unsigned)nblk), 64 * WAVES_M * WAVES_N, LDS, stream>>>(p);
    return hkq_launch_status();
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

int hkq_gemm_a8w8(const void* A, const void* B, const float* sa, const float* sb, void* C, int64_t M, int64_t N,
                  int64_t K, int64_t lda, int64_t ldb, int64_t ldc, hipStream_t stream) {
    if (int e = check_common(M, N, K, ldc, C)) return e;
    HKQ_CHECK_ARG(K % 16 == 0, "K must be a multiple of 16");
    HKQ_CHECK_ARG(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0,
                  "lda/ldb must be >= K and multiples of 16");
    HKQ_CHECK_ALIGN(A, 16);
    HKQ_CHECK_ALIGN(B, 16);
    HKQ_CHECK_ALIGN(sb, 16);
    DenseParams p{};
    p.A = static_cast<const uint8_t*>(A);
    p.B = static_cast<const uint8_t*>(B);
    p.C = static_cast<uint16_t*>(C);
    p.sa = sa;
    p.sb = sb;
    p.M = (int)M; p.N = (int)N; p.K = (int)K; p.kbytes = (int)K;
    p.lda = lda; p.ldb = ldb; p.ldc = ldc;
    return launch_dense<MODE_A8W8, 2, 2, 4, 4>(p, stream);
}

int hkq_gemm_mxfp4(const void* A, const void* As, const void* B, const void* Bs, void* C, int64_t M, int64_t N,
                   int64_t K, int64_t lda, int64_t ldb, int64_t ldsa, int64_t ldsb, int64_t ldc, hipStream_t stream) {
    if (int e = check_common(M, N, K, ldc, C)) return e;
    HKQ_CHECK_ARG(K % 256 == 0, "K must be a multiple of 256");
    HKQ_CHECK_ARG(lda >= K / 2 && ldb >= K / 2 && lda % 16 == 0 && ldb % 16 == 0,
                  "lda/ldb (bytes) must be >= K/2 and multiples of 16");
    HKQ_CHECK_ARG(ldsa >= K / 32 && ldsb >= K / 32 && ldsa % 8 == 0 && ldsb % 8 == 0,
                  "scale row strides must be >= K/32 and multiples of 8");
    HKQ_CHECK_ALIGN(A, 16);
    HKQ_CHECK_ALIGN(B, 16);
    HKQ_CHECK_ALIGN(As, 8);
    HKQ_CHECK_ALIGN(Bs, 8);
    DenseParams p{};
    p.A = static_cast<const uint8_t*>(A);
    p.B = static_cast<const uint8_t*>(B);
    p.C = static_cast<uint16_t*>(C);
    p.sa = As;
    p.sb = Bs;
    p.M = (int)M; p.N = (int)N; p.K = (int)K; p.kbytes = (int)(K / 2);
    p.lda = lda; p.ldb = ldb; p.ldc = ldc;
    p.lsa = ldsa; p.lsb = ldsb;
    return launch_dense<MODE_MXFP4, 2, 2, 4, 4>(p, stream);
}

}  // extern "C"
