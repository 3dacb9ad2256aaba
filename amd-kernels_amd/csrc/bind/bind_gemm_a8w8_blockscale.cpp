// gemm_a8w8_blockscale_tk -- the reference module of
// kernels/gemm-basic/gemm_a8w8_blockscale/kernel.cpp:174-180:
// dispatch(A, B, C, a_scale, b_scale) (C third, as in the reference).
//   A [M, K], B [N, K]: E4M3FN codes (float8_e4m3fn or uint8)
//   a_scale fp32 [M, K/128]; b_scale fp32 [K/128, N] (per column, the
//   reference test's layout) or [K/128, ceil(N/128)] (128x128 weight blocks).
#include "bind_common.h"

using namespace hkqbind;

void dispatch(py::object A, py::object B, py::object C, py::object a_scale, py::object b_scale) {
    auto a = view(A, "A"), b = view(B, "B"), c = view(C, "C"), sa = view(a_scale, "a_scale"),
         sb = view(b_scale, "b_scale");
    if (a.dtype == kBF16 || b.dtype == kBF16)
        throw py::type_error("A and B must hold E4M3FN codes (torch.float8_e4m3fn or uint8); quantize with "
                             "quant_tk.group_quant_fwd (activations, 1x128) first");
    expect_dtype(a, "A", {kFP8, kU8});
    expect_dtype(b, "B", {kFP8, kU8});
    expect_dtype(sa, "a_scale", {kF32});
    expect_dtype(sb, "b_scale", {kF32});
    expect_dtype(c, "C", {kBF16});
    const int64_t lda = row_stride(a, "A"), ldb = row_stride(b, "B"), ldc = row_stride(c, "C");
    const int64_t M = a.dim(0), K = a.dim(1), N = b.dim(0);
    expect(b.dim(1) == K, "A and B must have the same K");
    expect(c.dim(0) == M && c.dim(1) == N, "C must be [M, N]");
    expect(K % 128 == 0, "K must be a multiple of 128");
    expect(sa.shape.size() == 2 && sa.dim(0) == M && sa.dim(1) == K / 128, "a_scale must be [M, K/128]");
    expect(sb.shape.size() == 2 && sb.dim(0) == K / 128, "b_scale must be [K/128, N] or [K/128, ceil(N/128)]");
    int64_t group_n;
    if (sb.dim(1) == N) group_n = 1;
    else if (sb.dim(1) == (N + 127) / 128) group_n = 128;
    else throw py::value_error("b_scale must be [K/128, N] or [K/128, ceil(N/128)]");
    const int64_t lsa = row_stride(sa, "a_scale"), lsb = row_stride(sb, "b_scale");
    check(hkq_gemm_blockscale((const void*)a.ptr, (const void*)b.ptr, (const float*)sa.ptr, (const float*)sb.ptr,
                              (void*)c.ptr, M, N, K, lda, ldb, lsa, lsb, ldc, group_n, current_stream()),
          "gemm_a8w8_blockscale");
}

PYBIND11_MODULE(gemm_a8w8_blockscale_tk, m) {
    m.doc() = "Block-scale FP8 GEMM: 1x128 activation and 128x128 (or 128x1) weight scales (gfx950)";
    m.def("dispatch", &dispatch, "C = sum_g (A_g . B_g^T) * a_scale[:, g] * b_scale[g, n / group_n]");
}
