// gemm_afp4wfp4_tk -- the reference module of kernels/gemm-basic/gemm_afp4wfp4/kernel.cpp:154-159.
// The reference's dispatch(A, B, C) takes FP4 values already dequantized to
// bf16; this build takes the packed MXFP4 format that file documents (:3-6):
// dispatch(A, B, C, A_scale, B_scale) with A uint8 [M, K/2] (two E2M1 codes per
// byte, even k in the low nibble), A_scale uint8 e8m0 [M, K/32], B uint8
// [N, K/2], B_scale uint8 [N, K/32], C bf16 [M, N].
#include "bind_common.h"

using namespace hkqbind;

void dispatch(py::object A, py::object B, py::object C, py::object A_scale, py::object B_scale) {
    auto a = view(A, "A"), b = view(B, "B"), c = view(C, "C"), sa = view(A_scale, "A_scale"),
         sb = view(B_scale, "B_scale");
    if (a.dtype == kBF16 || b.dtype == kBF16)
        throw py::type_error("A and B must be packed MXFP4 (uint8, two E2M1 codes per byte) with e8m0 scales; "
                             "quantize with quant_moe_tk.downcast_to_mxfp(..., is_fp4=True)");
    expect_dtype(a, "A", {kU8});
    expect_dtype(b, "B", {kU8});
    expect_dtype(sa, "A_scale", {kU8});
    expect_dtype(sb, "B_scale", {kU8});
    expect_dtype(c, "C", {kBF16});
    const int64_t lda = row_stride(a, "A"), ldb = row_stride(b, "B"), ldc = row_stride(c, "C");
    const int64_t M = a.dim(0), K = 2 * a.dim(1), N = b.dim(0);
    expect(b.dim(1) * 2 == K, "A and B must have the same K");
    expect(c.dim(0) == M && c.dim(1) == N, "C must be [M, N]");
    expect(sa.shape.size() == 2 && sa.dim(0) == M && sa.dim(1) == K / 32, "A_scale must be [M, K/32]");
    expect(sb.shape.size() == 2 && sb.dim(0) == N && sb.dim(1) == K / 32, "B_scale must be [N, K/32]");
    const int64_t lsa = row_stride(sa, "A_scale"), lsb = row_stride(sb, "B_scale");
    Workspace ws = workspace(hkq_gemm_mxfp4_workspace(M, N, K), A);
    check(hkq_gemm_mxfp4_ws((const void*)a.ptr, (const void*)sa.ptr, (const void*)b.ptr, (const void*)sb.ptr,
                            (void*)c.ptr, M, N, K, lda, ldb, lsa, lsb, ldc, ws.ptr, ws.bytes, current_stream()),
          "gemm_afp4wfp4");
}

PYBIND11_MODULE(gemm_afp4wfp4_tk, m) {
    m.doc() = "MXFP4 A4W4 GEMM with e8m0 per-32 scales on both operands (gfx950 scaled MFMA)";
    m.def("dispatch", &dispatch, "C = dequant(A) . dequant(B)^T", py::arg("A"), py::arg("B"), py::arg("C"),
          py::arg("A_scale"), py::arg("B_scale"));
}
