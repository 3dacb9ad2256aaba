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
#include "gemm_mainloop.h"
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
};

// Tile geometry of the dense GEMMs: 256 x 256 tiles computed by 4 waves of
// 128 x 128 (whole tiles) or 64 x 128 (M halves of a tile, 128 x 256). K-tiles
// are 128 bytes per row (whole 128-byte lines per row and load: half the
// cache-line requests of 64-byte K-tiles) in a 2-stage ring when K allows,
// else 64 bytes in a 4-stage ring.
constexpr int DENSE_WAVES_M = 2, DENSE_WAVES_N = 2, DENSE_TM = 4, DENSE_TN = 4;
constexpr int DENSE_BM = DENSE_WAVES_M * DENSE_TM * 32, DENSE_BN = DENSE_WAVES_N * DENSE_TN * 32;
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

// One (TM*64) x 256 block of C: rows [m0, m0 + TM*64) of tile (tm, tn) of the
// 256 x 256 tile grid, starting `half` * 128 rows into the tile.
template <int MODE, int TM, int KTB>
__device__ __forceinline__ void dense_block(const DenseParams& p, int tm, int tn, int half, HKQ_LDS uint8_t* smem) {
    constexpr int WAVES_M = DENSE_WAVES_M, WAVES_N = DENSE_WAVES_N, TN = DENSE_TN, NS = dense_ns<KTB>();
    using Cfg = DenseCfg<MODE, WAVES_M, WAVES_N, TM, TN, KTB>;
    constexpr int NW = Cfg::NW, BM = Cfg::BM, BN = Cfg::BN, LA = Cfg::LA, LB = Cfg::LB;
    constexpr bool FP4 = Cfg::FP4;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int khalf = lane >> 5;

    const int m0 = tm * DENSE_BM + half * BM, n0 = tn * BN;
    const int rows_a = min(p.M - m0, BM), rows_b = min(p.N - n0, BN);
    if (rows_a <= 0) return;  // the M half below the last row (uniform per workgroup)

    LoopSrc src;
    src.a = p.A + (int64_t)m0 * p.lda;
    src.b = p.B + (int64_t)n0 * p.ldb;
    src.a_bytes = min((int64_t)rows_a * p.lda, (int64_t)0x7FFFFFFF);
    src.b_bytes = min((int64_t)rows_b * p.ldb, (int64_t)0x7FFFFFFF);
    src.as = FP4 ? static_cast<const uint8_t*>(p.sa) + (int64_t)m0 * p.lsa : nullptr;
    src.bs = FP4 ? static_cast<const uint8_t*>(p.sb) + (int64_t)n0 * p.lsb : nullptr;
    src.as_bytes = FP4 ? min((int64_t)rows_a * p.lsa, (int64_t)0x7FFFFFFF) : 0;
    src.bs_bytes = FP4 ? min((int64_t)rows_b * p.lsb, (int64_t)0x7FFFFFFF) : 0;
    src.lsa = p.lsa;
    src.lsb = p.lsb;
    src.KT = p.kbytes / KTB;
    uint32_t a_off[LA], b_off[LB];
#pragma unroll
    for (int i = 0; i < LA; ++i) a_off[i] = dense_row_off<NW, KTB>(i, wave, lane, p.lda);
#pragma unroll
    for (int i = 0; i < LB; ++i) b_off[i] = dense_row_off<NW, KTB>(i, wave, lane, p.ldb);

    // A8W8: the tile's row and column scales go to LDS while the K loop runs
    // (rows past M / columns past N read zero); each wave loads 64 of each.
    // These loads are older than the K-tile loads, so the loop's vmcnt waits
    // cover them, and its final vmcnt(0) barrier makes them visible.
    HKQ_LDS uint8_t* scl = smem + dense_ring_lds<MODE, KTB>();
    if constexpr (MODE == MODE_A8W8) {
        const float* sa = static_cast<const float*>(p.sa) + m0;
        const float* sb = static_cast<const float*>(p.sb) + n0;
        lds_load4(sa, (uint32_t)rows_a * 4u, scl + wave * 256, (uint32_t)(wave * 64 + lane) * 4u);
        lds_load4(sb, (uint32_t)rows_b * 4u, scl + DENSE_BM * 4 + wave * 256, (uint32_t)(wave * 64 + lane) * 4u);
    }

    v16f acc[TN][TM];
    gemm_mainloop<MODE, WAVES_M, WAVES_N, TM, TN, KTB, NS>(src, a_off, b_off, smem, lane, wave, acc);

    // Epilogue (scales of A8W8 applied in registers; MXFP4 has none left)
    const int mw = m0 + wm * TM * 32, nw = n0 + wn * TN * 32;
    store_tile_bf16<TM, TN>(
        acc, smem, wave, lane, p.C, p.ldc, p.M, p.N, mw, nw, p.c16 != 0,
        [&](int j) {
            const int r = wm * TM * 32 + j * 32 + (lane & 31);
            return MODE == MODE_A8W8 ? *reinterpret_cast<const HKQ_LDS float*>(scl + r * 4) : 1.0f;
        },
        [&](int i, int g) {
            const int n = wn * TN * 32 + i * 32 + 8 * g + 4 * khalf;
            if constexpr (MODE == MODE_A8W8) {
                const v4f c = *reinterpret_cast<const HKQ_LDS v4f*>(scl + DENSE_BM * 4 + n * 4);
                return make_float4(c[0], c[1], c[2], c[3]);
            }
            return make_float4(1.f, 1.f, 1.f, 1.f);
        },
        [](int, int) { return make_float4(0.f, 0.f, 0.f, 0.f); });
}

// Workgroup u < n_whole computes tile u. When the last round of tiles would
// leave at least half of the CUs idle, its tiles are instead computed as M
// halves by twice as many workgroups: unit v = u - n_whole (XCD v & 7, as the
// dispatcher assigns workgroups round-robin) computes half (v >> 3) & 1 of tile
// n_whole + 8 * (v >> 4) + (v & 7), so both halves of a tile run on one XCD.
// Tile ids then go through tile_coords' XCD-aware order.
template <int MODE, int KTB>
__global__ __launch_bounds__(64 * DENSE_WAVES_M * DENSE_WAVES_N, 1) void dense_gemm_kernel(const DenseParams p) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;
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

template <int MODE, int KTB>
static int launch_dense_ktb(DenseParams& p, hipStream_t stream) {
    constexpr int LDS = dense_lds<MODE, KTB>();
    static_assert(LDS <= 160 * 1024, "LDS budget of a CDNA4 CU");
    auto kern = dense_gemm_kernel<MODE, KTB>;
    static bool attr_set = false;  // per instantiation; the attribute is per-process
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
        if (e != hipSuccess) {
            set_error("hipFuncSetAttribute(MaxDynamicSharedMemorySize=%d) failed: %s", LDS, hipGetErrorString(e));
            return (int)e;
        }
        attr_set = true;
    }
    p.tiles_m = (p.M + DENSE_BM - 1) / DENSE_BM;
    p.tiles_n = (p.N + DENSE_BN - 1) / DENSE_BN;
    if (p.group_m <= 0) p.group_m = 8;
    p.c16 = (p.ldc % 8 == 0) && (reinterpret_cast<uintptr_t>(p.C) % 16 == 0);
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    if (tiles == 0) return 0;
    // Split the last round into M halves when it would fill at most half of the
    // CUs and the tiles have rows in both halves.
    const int ncu = cu_count();
    const int64_t last = ncu > 0 ? tiles % ncu : 0;
    const int64_t split = (last > 0 && 2 * last <= ncu && p.M > DENSE_BM / 2) ? last : 0;
    p.n_whole = (int)(tiles - split);
    p.n_split = (int)split;
    const int64_t nblk = p.n_whole + 2 * ((split + 7) / 8 * 8);
    kern<<<dim3((unsigned)nblk), 64 * DENSE_WAVES_M * DENSE_WAVES_N, LDS, stream>>>(p);
    return hkq_launch_status();
}

// 128-byte K-tiles need whole 128-byte K-tiles in every row: a partial last
// K-tile would read the next row's bytes instead of zeros.
template <int MODE>
static int launch_dense(DenseParams& p, hipStream_t stream) {
    return p.kbytes % 128 == 0 ? launch_dense_ktb<MODE, 128>(p, stream) : launch_dense_ktb<MODE, 64>(p, stream);
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
    return launch_dense<MODE_A8W8>(p, stream);
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
    return launch_dense<MODE_MXFP4>(p, stream);
}

}  // extern "C"
