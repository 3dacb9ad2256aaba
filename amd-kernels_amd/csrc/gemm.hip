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
    int kbytes;           // K in bytes per row of A/B (a multiple of KT_BYTES)
    int64_t lda, ldb;     // bytes
    int64_t ldc;          // elements
    int64_t lsa, lsb;     // MXFP4 scale row strides (bytes)
    int tiles_m, tiles_n, group_m;
    int c16;              // rows of C are 16-byte aligned (ldc % 8 == 0, C 16-byte aligned)
};

template <int MODE, int WAVES_M, int WAVES_N, int TM, int TN, int NS>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N, 1) void dense_gemm_kernel(const DenseParams p) {
    using Cfg = DenseCfg<MODE, WAVES_M, WAVES_N, TM, TN>;
    constexpr int NW = Cfg::NW, BM = Cfg::BM, BN = Cfg::BN, LA = Cfg::LA, LB = Cfg::LB;
    constexpr bool FP4 = Cfg::FP4;

    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int khalf = lane >> 5;

    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int rows_a = min(p.M - m0, BM), rows_b = min(p.N - n0, BN);

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
    src.KT = p.kbytes / KT_BYTES;
    uint32_t a_off[LA], b_off[LB];
#pragma unroll
    for (int i = 0; i < LA; ++i) a_off[i] = dense_row_off<NW>(i, wave, lane, p.lda);
#pragma unroll
    for (int i = 0; i < LB; ++i) b_off[i] = dense_row_off<NW>(i, wave, lane, p.ldb);

    v16f acc[TN][TM];
    gemm_mainloop<MODE, WAVES_M, WAVES_N, TM, TN, NS>(src, a_off, b_off, smem, lane, wave, acc);

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
        },
        [](int, int) { return make_float4(0.f, 0.f, 0.f, 0.f); });
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
