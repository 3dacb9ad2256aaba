// gemm_a16w16_tk -- the reference module of kernels/gemm-basic/gemm_a16w16 (no kernel
// source in the reference tree; its test is tests/test_gemm.py:21-42):
// dispatch(A, B, C): A [M, K], B [N, K], C [M, N], all bf16; C = bf16(A . B^T).
#include "gemm_bind.h"

using namespace hkqbind;

void dispatch(py::object A, py::object B, py::object C) { gemm_bf16(A, B, C, "gemm_a16w16"); }

PYBIND11_MODULE(gemm_a16w16_tk, m) {
    m.doc() = "bf16 GEMM (gfx950 MFMA)";
    m.def("dispatch", &dispatch, "C = A . B^T");
}
