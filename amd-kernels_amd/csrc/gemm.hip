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

template <int MODE, int WAVES_M, int WAVES_N, int TM, int TN>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N, 1) void dense_gemm_kernel(const DenseParams p) {
    constexpr int NW = WAVES_M * WAVES_N;
    constexpr int BM = WAVES_M * TM * 32, BN = WAVES_N * TN * 32;
    constexpr int LA = BM / 8 / NW, LB = BN / 8 / NW;
    constexpr bool FP4 = MODE == MODE_MXFP4;
    constexpr int STAGE = (BM + BN) * KT_BYTES;
    static_assert(LA >= 1 && LB >= 1, "tile too small for the wave count");

    extern __shared__ __attribute__((aligned(1024))) uint8_t smem_raw[];
    HKQ_LDS uint8_t* smem = (HKQ_LDS uint8_t*)smem_raw;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    int tm, tn;
    tile_coords(blockIdx.x, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int rows_a = min(p.M - m0, BM), rows_b = min(p.N - n0, BN);

    // load pattern: same logical chunk for every instruction of this lane
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
    const int KT = (p.kbytes + KT_BYTES - 1) / KT_BYTES;

    auto issue = [&](int kt, int stage) {
        const int kb = kt * KT_BYTES;
        const bool tail = kb + KT_BYTES > p.kbytes;
        const uint32_t left = (uint32_t)(p.kbytes - kb);
        auto ra = make_rsrc(a_base + kb, (uint32_t)max(a_bytes - kb, (int64_t)0));
        auto rb = make_rsrc(b_base + kb, (uint32_t)max(b_bytes - kb, (int64_t)0));
        HKQ_LDS uint8_t* st = smem + stage * STAGE;
        load_tile_lds<BM, NW>(ra, st, wave, a_off, chunk_off, tail, left);
        load_tile_lds<BN, NW>(rb, st + BM * KT_BYTES, wave, b_off, chunk_off, tail, left);
    };

    // MXFP4 scales: per m-tile / n-tile, the 8 e8m0 bytes of this K-tile for
    // the lane's row, pre-shifted so that bytes 0 and 2 of each word are the
    // lane's K-block for substeps (0,1) and (2,3).
    int sa_cur[TM][2], sb_cur[TN][2];
    const int srow_a = m0 + wm * TM * 32 + (lane & 31);
    const int srow_b = n0 + wn * TN * 32 + (lane & 31);
    auto load_scales = [&](int kt, int (&sa)[TM][2], int (&sb)[TN][2]) {
        const uint8_t* As = static_cast<const uint8_t*>(p.sa);
        const uint8_t* Bs = static_cast<const uint8_t*>(p.sb);
        const int sh = (lane >> 5) * 8;
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            const int m = srow_a + t * 32;
            uint2 v = m < p.M ? *reinterpret_cast<const uint2*>(As + (int64_t)m * p.lsa + kt * 8) : make_uint2(0, 0);
            sa[t][0] = (int)(v.x >> sh);
            sa[t][1] = (int)(v.y >> sh);
        }
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const int n = srow_b + t * 32;
            uint2 v = n < p.N ? *reinterpret_cast<const uint2*>(Bs + (int64_t)n * p.lsb + kt * 8) : make_uint2(0, 0);
            sb[t][0] = (int)(v.x >> sh);
            sb[t][1] = (int)(v.y >> sh);
        }
    };

    v16f acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = v16f{};

    issue(0, 0);
    if constexpr (FP4) load_scales(0, sa_cur, sb_cur);
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) lgkmcnt(0)
    __syncthreads();

    const int arow = wm * TM * 32 + (lane & 31);
    const int brow = wn * TN * 32 + (lane & 31);
    const int khalf = lane >> 5;

    for (int kt = 0; kt < KT; ++kt) {
        const int stage = kt & 1;
        int sa_nxt[TM][2], sb_nxt[TN][2];
        if (kt + 1 < KT) {
            issue(kt + 1, stage ^ 1);
            if constexpr (FP4) load_scales(kt + 1, sa_nxt, sb_nxt);
        }
        const HKQ_LDS uint8_t* At = smem + stage * STAGE;
        const HKQ_LDS uint8_t* Bt = At + BM * KT_BYTES;
        if constexpr (!FP4) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                v8i af[TM], bf[TN];
#pragma unroll
                for (int t = 0; t < TM; ++t) af[t] = read_frag_fp8(At, arow + t * 32, ks * 4 + khalf * 2);
#pragma unroll
                for (int t = 0; t < TN; ++t) bf[t] = read_frag_fp8(Bt, brow + t * 32, ks * 4 + khalf * 2);
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) acc[i][j] = mfma<false>(bf[i], af[j], acc[i][j], 127, 127);
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                v8i af[TM], bf[TN];
#pragma unroll
                for (int t = 0; t < TM; ++t) af[t] = read_frag_fp4(At, arow + t * 32, ks * 2 + khalf);
#pragma unroll
                for (int t = 0; t < TN; ++t) bf[t] = read_frag_fp4(Bt, brow + t * 32, ks * 2 + khalf);
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) {
                        if (ks & 1)
                            acc[i][j] = mfma_sel<true, 2, 2>(bf[i], af[j], acc[i][j], sb_cur[i][ks >> 1], sa_cur[j][ks >> 1]);
                        else
                            acc[i][j] = mfma_sel<true, 0, 0>(bf[i], af[j], acc[i][j], sb_cur[i][ks >> 1], sa_cur[j][ks >> 1]);
                    }
            }
            if (kt + 1 < KT) {
#pragma unroll
                for (int t = 0; t < TM; ++t) { sa_cur[t][0] = sa_nxt[t][0]; sa_cur[t][1] = sa_nxt[t][1]; }
#pragma unroll
                for (int t = 0; t < TN; ++t) { sb_cur[t][0] = sb_nxt[t][0]; sb_cur[t][1] = sb_nxt[t][1]; }
            }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
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
    constexpr int LDS = 2 * (BM + BN) * KT_BYTES;
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
