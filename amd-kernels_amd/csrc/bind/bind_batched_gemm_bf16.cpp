// batched_gemm_bf16_tk -- the reference module of
// kernels/gemm-batched/batched_gemm_bf16/kernel.cpp:172-187: dispatch(A, B, C, bias)
// over the HipKittens 4-D layout (tests/test_gemm.py:316-347):
//   A (1, B, M, K), B (1, B, N, K), C (1, B, M, N): bf16; bias (1, B, 1, N)
//   bf16 or None; C[z] = bf16(A[z] . B[z]^T + bias[z][n]).
#include "gemm_bind.h"

using namespace hkqbind;

void dispatch(py::object A, py::object B, py::object C, py::object bias) {
    auto a = view(A, "A"), b = view(B, "B"), c = view(C, "C");
    expect_dtype(a, "A", {kBF16});
    expect_dtype(b, "B", {kBF16});
    expect_dtype(c, "C", {kBF16});
    const Batched ba = batched(a, "A"), bb = batched(b, "B"), bc = batched(c, "C");
    const int64_t Z = ba.batch, M = ba.rows, K = ba.cols, N = bb.rows;
    expect(bb.batch == Z && bc.batch == Z, "A, B and C must have the same batch count");
    expect(bb.cols == K, "A and B must have the same K");
    expect(bc.rows == M && bc.cols == N, "C must be (1, B, M, N)");
    const void* bias_ptr = nullptr;
    int64_t bsbias = 0;
    if (!bias.is_none()) {
        auto bi = view(bias, "bias");
        expect_dtype(bi, "bias", {kBF16});
        bsbias = batched_vec(bi, "bias", Z, N);
        bias_ptr = (const void*)bi.ptr;
    }
    check(hkq_batched_gemm_bf16((const void*)a.ptr, (const void*)b.ptr, bias_ptr, (void*)c.ptr, Z, M, N, K, ba.ld,
                                bb.ld, bc.ld, ba.bstride, bb.bstride, bc.bstride, bsbias, nullptr, 0,
                                current_stream()),
          "batched_gemm_bf16");
}

PYBIND11_MODULE(batched_gemm_bf16_tk, m) {
    m.doc() = "Batched bf16 GEMM with bias (gfx950 MFMA)";
    m.def("dispatch", &dispatch, "C[z] = A[z] . B[z]^T + bias[z][n]", py::arg("A"), py::arg("B"), py::arg("C"),
          py::arg("bias") = py::none());
}
