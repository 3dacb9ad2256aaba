// batched_gemm_a8w8_tk -- the reference module of
// kernels/gemm-batched/batched_gemm_a8w8/kernel.cpp:186-203:
// dispatch(A, B, a_scale, b_scale, C, bias) over the HipKittens 4-D layout
// (tests/test_gemm.py:349-390):
//   A (1, B, M, K) and B (1, B, N, K): E4M3FN codes (float8_e4m3fn or uint8)
//   a_scale (1, B, 1, M), b_scale (1, B, 1, N): fp32
//   C (1, B, M, N) bf16; bias (1, B, 1, N) bf16 or None
//   C[z] = bf16((A[z] . B[z]^T) * a_scale[z][m] * b_scale[z][n] + bias[z][n])
// (3-D (B, R, C) tensors are accepted as well.)
#include "gemm_bind.h"

using namespace hkqbind;

void dispatch(py::object A, py::object B, py::object a_scale, py::object b_scale, py::object C, py::object bias) {
    auto a = view(A, "A"), b = view(B, "B"), sa = view(a_scale, "a_scale"), sb = view(b_scale, "b_scale"),
         c = view(C, "C");
    if (a.dtype == kBF16 || b.dtype == kBF16)
        throw py::type_error(
            "A and B must hold E4M3FN codes (torch.float8_e4m3fn or uint8); bf16 tensors carrying int8 values "
            "are not accepted -- quantize with quant_tk.per_token_quant_fwd into a float8_e4m3fn tensor");
    expect_dtype(a, "A", {kFP8, kU8});
    expect_dtype(b, "B", {kFP8, kU8});
    expect_dtype(sa, "a_scale", {kF32});
    expect_dtype(sb, "b_scale", {kF32});
    expect_dtype(c, "C", {kBF16});
    const Batched ba = batched(a, "A"), bb = batched(b, "B"), bc = batched(c, "C");
    const int64_t Z = ba.batch, M = ba.rows, K = ba.cols, N = bb.rows;
    expect(bb.batch == Z && bc.batch == Z, "A, B and C must have the same batch count");
    expect(bb.cols == K, "A and B must have the same K");
    expect(bc.rows == M && bc.cols == N, "C must be (1, B, M, N)");
    const int64_t bsa = batched_vec(sa, "a_scale", Z, M), bsb = batched_vec(sb, "b_scale", Z, N);
    const void* bias_ptr = nullptr;
    int64_t bsbias = 0;
    if (!bias.is_none()) {
        auto bi = view(bias, "bias");
        expect_dtype(bi, "bias", {kBF16});
        bsbias = batched_vec(bi, "bias", Z, N);
        bias_ptr = (const void*)bi.ptr;
    }
    check(hkq_batched_gemm_a8w8((const void*)a.ptr, (const void*)b.ptr, (const float*)sa.ptr, (const float*)sb.ptr,
                                bias_ptr, (void*)c.ptr, Z, M, N, K, ba.ld, bb.ld, bc.ld, ba.bstride, bb.bstride,
                                bc.bstride, bsa, bsb, bsbias, current_stream()),
          "batched_gemm_a8w8");
}

PYBIND11_MODULE(batched_gemm_a8w8_tk, m) {
    m.doc() = "Batched FP8 A8W8 GEMM with per-token x per-channel scales and bias (gfx950 scaled MFMA)";
    m.def("dispatch", &dispatch, "C[z] = (A[z] . B[z]^T) * a_scale[z][m] * b_scale[z][n] + bias[z][n]",
          py::arg("A"), py::arg("B"), py::arg("a_scale"), py::arg("b_scale"), py::arg("C"),
          py::arg("bias") = py::none());
}
