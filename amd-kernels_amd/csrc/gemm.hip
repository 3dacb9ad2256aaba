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
//                        pre-dequantized bf16).
#include "gemm_core.h"
#include "hkq_host.h"

#include <type_traits>

namespace hkq {

struct DenseParams {
    const uint8_t* A;
    const uint8_t* B;
    uint16_t* C;
    const void* sa;
    const void* sb;
    int M, N, K;          // K in elements
    int kbytes;           // K in bytes per row of A/B (a multiple of KT_BYTES)
    int64_t lda, ldb;     // bytes
    int64_t ldc;          // elements
    int64_t lsa, lsb;     // MXFP4 scale row strides (bytes)
    int tiles_m, tiles_n, group_m;
    int c16;              // rows of C are 16-byte aligned (ldc % 8 == 0, C 16-byte aligned)
};

template <int MODE, int WAVES_M, int WAVES_N, int TM, int TN>
struct DenseCfg {
    static constexpr int NW = WAVES_M * WAVES_N;
    static constexpr int BM = WAVES_M * TM * 32, BN = WAVES_N * TN * 32;
    static constexpr bool FP4 = MODE == MODE_MXFP4;
    static constexpr int SUB = FP4 ? 2 : 1;                    // 64-deep MFMA K-steps per K-tile
    static constexpr int LA = BM / ROWS_PER_LOAD / NW, LB = BN / ROWS_PER_LOAD / NW;
    // FP4: the K-tile's e8m0 scales (4 bytes per row: 128 values) ride in LDS
    // after the data; one 4-byte LDS-direct load per lane covers 64 rows.
    static constexpr int SCA = FP4 ? BM * 4 : 0, SCB = FP4 ? BN * 4 : 0;
    static constexpr int LSA = FP4 ? BM / 64 / NW : 0, LSB = FP4 ? BN / 64 / NW : 0;
    static constexpr int STAGE = (BM + BN) * KT_BYTES + SCA + SCB;
    static constexpr int NLD = LA + LB + LSA + LSB;           // LDS-direct loads per K-tile
    static constexpr int PARTS = FP4 ? 1 : 2;                 // ds_read_b128 per fragment
    static constexpr int NRD = 2 * PARTS * (TM > TN ? TM : TN);  // fragment read slots per K-step
    static constexpr int NSC = FP4 ? TM + TN : 0;             // scale reads per K-tile
    static constexpr int NMF = TM * TN, HALF = NMF / 2;       // MFMAs per K-step
    // epilogue: each wave stages its (TM*32) x (TN*32) bf16 sub-tile in LDS with a
    // padded row pitch, then writes whole 256-byte row segments of C
    static constexpr int EP_PITCH = TN * 32 * 2 + 16;
    static constexpr int EP_BYTES = NW * TM * 32 * EP_PITCH;
    static constexpr int lds_bytes(int ns) { return ns * STAGE > EP_BYTES ? ns * STAGE : EP_BYTES; }
    static_assert(LA >= 1 && LB >= 1, "tile too small for the wave count");
    static_assert(!FP4 || (LSA >= 1 && LSB >= 1), "scale tile too small for the wave count");
    static_assert(NRD <= NMF, "phase A pairs at most one fragment read with each MFMA");
    static_assert((TN * 32 * 2) % 256 == 0, "epilogue rows are whole 256-byte segments");
};

// Pipeline (per wave; one barrier per K-tile, NS ring stages):
//   K-tile kt lives in stage kt % NS. Its SUB K-steps run their MFMAs with
//   double-buffered fragments: the LDS reads of the next step are issued between
//   the MFMAs of the current one. In the last step, half of the MFMAs are issued
//   before the barrier (the matrix pipe stays busy while the waves meet); the
//   barrier (a) waits until K-tile kt+1 is resident (at most NS-2 K-tiles of
//   loads still in flight) and (b) retires every wave's reads of stage kt % NS,
//   which is then refilled with K-tile kt+NS while the other half of the MFMAs
//   issue together with the reads of K-tile kt+1's first step. sched_barrier
//   between chunks keeps this order through the compiler's scheduler.
template <int MODE, int WAVES_M, int WAVES_N, int TM, int TN, int NS>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N, 1) void dense_gemm_kernel(const DenseParams p) {
    using Cfg = DenseCfg<MODE, WAVES_M, WAVES_N, TM, TN>;
    constexpr int NW = Cfg::NW, BM = Cfg::BM, BN = Cfg::BN, SUB = Cfg::SUB;
    constexpr int LA = Cfg::LA, LB = Cfg::LB, LSA = Cfg::LSA, SCA = Cfg::SCA, STAGE = Cfg::STAGE;
    constexpr int NLD = Cfg::NLD, PARTS = Cfg::PARTS, NRD = Cfg::NRD, NSC = Cfg::NSC;
    constexpr int NMF = Cfg::NMF, HALF = Cfg::HALF;
    constexpr bool FP4 = Cfg::FP4;
    static_assert(NS >= 2 && (NS - 1) * NLD <= 63, "vmcnt budget");

    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int rows_a = min(p.M - m0, BM), rows_b = min(p.N - n0, BN);

    // global -> LDS: instruction i of this wave fills rows (i*NW + wave)*16 + lane/4
    const uint32_t chunk_off = (uint32_t)(load_chunk(lane) << 4);
    uint32_t a_off[LA], b_off[LB];
#pragma unroll
    for (int i = 0; i < LA; ++i) a_off[i] = (uint32_t)(((i * NW + wave) * ROWS_PER_LOAD + (lane >> 2)) * p.lda) + chunk_off;
#pragma unroll
    for (int i = 0; i < LB; ++i) b_off[i] = (uint32_t)(((i * NW + wave) * ROWS_PER_LOAD + (lane >> 2)) * p.ldb) + chunk_off;
    const uint8_t* a_base = p.A + (int64_t)m0 * p.lda;
    const uint8_t* b_base = p.B + (int64_t)n0 * p.ldb;
    const int64_t a_bytes = min((int64_t)rows_a * p.lda, (int64_t)0x7FFFFFFF);
    const int64_t b_bytes = min((int64_t)rows_b * p.ldb, (int64_t)0x7FFFFFFF);
    const uint8_t* as_base = FP4 ? static_cast<const uint8_t*>(p.sa) + (int64_t)m0 * p.lsa : nullptr;
    const uint8_t* bs_base = FP4 ? static_cast<const uint8_t*>(p.sb) + (int64_t)n0 * p.lsb : nullptr;
    const int64_t as_bytes = FP4 ? min((int64_t)rows_a * p.lsa, (int64_t)0x7FFFFFFF) : 0;
    const int64_t bs_bytes = FP4 ? min((int64_t)rows_b * p.lsb, (int64_t)0x7FFFFFFF) : 0;
    const int KT = p.kbytes / KT_BYTES;

    // Load instruction idx of K-tile kt into `stage`: A rows, B rows, then (FP4)
    // the 4-byte scale word of row (i*NW + wave)*64 + lane. For kt >= KT the
    // buffers are empty, so the loads read zero (the loop needs no branches).
    auto load_piece = [&](int kt, int stage, int idx) {
        const int kb = kt * KT_BYTES;
        const bool live = kt < KT;
        HKQ_LDS uint8_t* st = smem + stage * STAGE;
        if (idx < LA) {
            lds_load16(a_base + kb, live ? (uint32_t)(a_bytes - kb) : 0u, st + (idx * NW + wave) * 1024, a_off[idx]);
        } else if (idx < LA + LB) {
            const int i = idx - LA;
            lds_load16(b_base + kb, live ? (uint32_t)(b_bytes - kb) : 0u, st + BM * KT_BYTES + (i * NW + wave) * 1024,
                       b_off[i]);
        } else if (idx < LA + LB + LSA) {
            const int i = idx - LA - LB;
            const uint32_t off = (uint32_t)(((i * NW + wave) * 64 + lane) * p.lsa);
            lds_load4(as_base + kt * 4, live ? (uint32_t)(as_bytes - kt * 4) : 0u,
                      st + (BM + BN) * KT_BYTES + (i * NW + wave) * 256, off);
        } else {
            const int i = idx - LA - LB - LSA;
            const uint32_t off = (uint32_t)(((i * NW + wave) * 64 + lane) * p.lsb);
            lds_load4(bs_base + kt * 4, live ? (uint32_t)(bs_bytes - kt * 4) : 0u,
                      st + (BM + BN) * KT_BYTES + SCA + (i * NW + wave) * 256, off);
        }
    };

    const int arow = wm * TM * 32 + (lane & 31);
    const int brow = wn * TN * 32 + (lane & 31);
    const int khalf = lane >> 5;

    struct Frags {
        v4i a[TM][PARTS], b[TN][PARTS];
    };
    // Fragment read slot idx of K-step ks, A and B tiles interleaved
    // (a0 b0 a1 b1 ...) so the first MFMAs' operands arrive first; slots past
    // TM (A) or TN (B) tiles are empty. FP8: logical chunks 2*khalf + part;
    // FP4: chunk 2*ks + khalf.
    auto read_piece = [&](int stage, int ks, Frags& f, int idx) {
        const HKQ_LDS uint8_t* At = smem + stage * STAGE;
        const int t = idx / (2 * PARTS), isb = (idx / PARTS) & 1, part = idx % PARTS;
        if ((isb ? TN : TM) <= t) return;
        const int row = (isb ? brow : arow) + t * 32;
        const int chunk = FP4 ? ks * 2 + khalf : khalf * 2 + part;
        const v4i v = lds_read16(At + (isb ? BM * KT_BYTES : 0) + lds_swz(row, chunk));
        if (isb) f.b[t][part] = v;
        else f.a[t][part] = v;
    };
    // MXFP4: per m/n-tile the 4 scale bytes of the K-tile for the lane's row,
    // shifted so bytes 0 and 2 are the lane's K-block of steps 0 and 1.
    struct Scales {
        int a[TM], b[TN];
    };
    auto read_scale = [&](int stage, Scales& s, int idx) {
        if constexpr (FP4) {
            const HKQ_LDS uint8_t* sca = smem + stage * STAGE + (BM + BN) * KT_BYTES;
            const bool isa = idx < TM;
            const int t = isa ? idx : idx - TM;
            const uint32_t w = *reinterpret_cast<const HKQ_LDS uint32_t*>(
                sca + (isa ? (arow + t * 32) * 4 : SCA + (brow + t * 32) * 4));
            if (isa) s.a[t] = (int)(w >> (khalf * 8));
            else s.b[t] = (int)(w >> (khalf * 8));
        }
    };

    v16f acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = v16f{};

    // MFMA idx (accumulator i*TM + j) of K-step ks
    auto mfma_one = [&](const Frags& f, int ks, const Scales& s, int idx) {
        const int i = idx / TM, j = idx % TM;
        v8i a, b;
        if constexpr (PARTS == 2) {
            b = v8i{f.b[i][0][0], f.b[i][0][1], f.b[i][0][2], f.b[i][0][3], f.b[i][1][0], f.b[i][1][1], f.b[i][1][2], f.b[i][1][3]};
            a = v8i{f.a[j][0][0], f.a[j][0][1], f.a[j][0][2], f.a[j][0][3], f.a[j][1][0], f.a[j][1][1], f.a[j][1][2], f.a[j][1][3]};
        } else {
            b = v8i{f.b[i][0][0], f.b[i][0][1], f.b[i][0][2], f.b[i][0][3], 0, 0, 0, 0};
            a = v8i{f.a[j][0][0], f.a[j][0][1], f.a[j][0][2], f.a[j][0][3], 0, 0, 0, 0};
        }
        if constexpr (FP4) {
            if (ks & 1) acc[i][j] = mfma_sel<true, 2, 2>(b, a, acc[i][j], s.b[i], s.a[j]);
            else acc[i][j] = mfma_sel<true, 0, 0>(b, a, acc[i][j], s.b[i], s.a[j]);
        } else {
            acc[i][j] = mfma_sel<false, 0, 0>(b, a, acc[i][j], 127, 127);
        }
    };

    Frags F[2];
    Scales S[2];
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int i = 0; i < NLD; ++i) load_piece(t, t, i);
    tile_barrier<(NS - 1) * NLD>();  // K-tile 0 resident
#pragma unroll
    for (int i = 0; i < NRD; ++i) read_piece(0, 0, F[0], i);
#pragma unroll
    for (int i = 0; i < NSC; ++i) read_scale(0, S[0], i);

    // One K-tile; P is the tile's parity (fragment and scale buffers alternate).
    auto ktile = [&](int kt, int stage, auto parity) {
        constexpr int P = decltype(parity)::value;
        const int next_stage = stage + 1 == NS ? 0 : stage + 1;
        // phase A: steps 0 .. SUB-2, one fragment read of the next step per MFMA
#pragma unroll
        for (int ks = 0; ks + 1 < SUB; ++ks) {
#pragma unroll
            for (int c = 0; c < NMF; ++c) {
                mfma_one(F[(P * SUB + ks) & 1], ks, S[P], c);
                if (c < NRD) read_piece(stage, ks + 1, F[(P * SUB + ks + 1) & 1], c);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // phase B: last step
        constexpr int LAST = SUB - 1;
        const Frags& cur = F[(P * SUB + LAST) & 1];
        Frags& nxt = F[(P * SUB + LAST + 1) & 1];
#pragma unroll
        for (int c = 0; c < HALF; ++c) mfma_one(cur, LAST, S[P], c);
        __builtin_amdgcn_sched_barrier(0);
        tile_barrier<(NS - 2) * NLD>();  // K-tile kt+1 resident; stage kt % NS retired
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < HALF; ++c) {
            mfma_one(cur, LAST, S[P], HALF + c);
#pragma unroll
            for (int i = c * NLD / HALF; i < (c + 1) * NLD / HALF; ++i) load_piece(kt + NS, stage, i);
#pragma unroll
            for (int i = c * NRD / HALF; i < (c + 1) * NRD / HALF; ++i) read_piece(next_stage, 0, nxt, i);
#pragma unroll
            for (int i = c * NSC / HALF; i < (c + 1) * NSC / HALF; ++i) read_scale(next_stage, S[P ^ 1], i);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    int stage = 0;
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
        ktile(kt, stage, std::integral_constant<int, 0>{});
        stage = stage + 1 == NS ? 0 : stage + 1;
        ktile(kt + 1, stage, std::integral_constant<int, 1>{});
        stage = stage + 1 == NS ? 0 : stage + 1;
    }
    if (kt < KT) ktile(kt, stage, std::integral_constant<int, 0>{});
    mfma_drain();
    tile_barrier<0>();  // every wave is done with the stages and no load is in flight

    // Epilogue (scales of A8W8 applied in registers; MXFP4 has none left)
    const float* sa = static_cast<const float*>(p.sa);
    const float* sb = static_cast<const float*>(p.sb);
    const int mw = m0 + wm * TM * 32, nw = n0 + wn * TN * 32;
    store_tile_bf16<TM, TN>(
        acc, smem, wave, lane, p.C, p.ldc, p.M, p.N, mw, nw, p.c16 != 0,
        [&](int j) {
            const int m = mw + j * 32 + (lane & 31);
            return (MODE == MODE_A8W8 && m < p.M) ? sa[m] : 1.0f;
        },
        [&](int i, int g) {
            const int n = nw + i * 32 + 8 * g + 4 * khalf;
            return (MODE == MODE_A8W8 && n < p.N) ? *reinterpret_cast<const float4*>(sb + n) : make_float4(1.f, 1.f, 1.f, 1.f);
        });
}

template <int MODE, int WAVES_M, int WAVES_N, int TM, int TN, int NS>
static int launch_dense(DenseParams& p, hipStream_t stream) {
    using Cfg = DenseCfg<MODE, WAVES_M, WAVES_N, TM, TN>;
    constexpr int LDS = Cfg::lds_bytes(NS);
    static_assert(LDS <= 160 * 1024, "LDS budget of a CDNA4 CU");
    auto kern = dense_gemm_kernel<MODE, WAVES_M, WAVES_N, TM, TN, NS>;
    static bool attr_set = false;  // per instantiation; the attribute is per-process
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
        if (e != hipSuccess) {
            set_error("hipFuncSetAttribute(MaxDynamicSharedMemorySize=%d) failed: %s", LDS, hipGetErrorString(e));
            return (int)e;
        }
        attr_set = true;
    }
    p.tiles_m = (p.M + Cfg::BM - 1) / Cfg::BM;
    p.tiles_n = (p.N + Cfg::BN - 1) / Cfg::BN;
    if (p.group_m <= 0) p.group_m = 8;
    p.c16 = (p.ldc % 8 == 0) && (reinterpret_cast<uintptr_t>(p.C) % 16 == 0);
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
    HKQ_CHECK_ARG(K % 64 == 0, "K must be a multiple of 64");
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
    return launch_dense<MODE_A8W8, 2, 2, 4, 4, 4>(p, stream);
}

int hkq_gemm_mxfp4(const void* A, const void* As, const void* B, const void* Bs, void* C, int64_t M, int64_t N,
                   int64_t K, int64_t lda, int64_t ldb, int64_t ldsa, int64_t ldsb, int64_t ldc, hipStream_t stream) {
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
    DenseParams p{};
    p.A = static_cast<const uint8_t*>(A);
    p.B = static_cast<const uint8_t*>(B);
    p.C = static_cast<uint16_t*>(C);
    p.sa = As;
    p.sb = Bs;
    p.M = (int)M; p.N = (int)N; p.K = (int)K; p.kbytes = (int)(K / 2);
    p.lda = lda; p.ldb = ldb; p.ldc = ldc;
    p.lsa = ldsa; p.lsb = ldsb;
    return launch_dense<MODE_MXFP4, 2, 2, 4, 4, 4>(p, stream);
}

}  // extern "C"
