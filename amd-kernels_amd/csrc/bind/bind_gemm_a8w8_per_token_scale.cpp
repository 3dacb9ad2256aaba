// gemm_a8w8_per_token_scale_tk -- the reference module of
// kernels/gemm-basic/gemm_a8w8_per_token_scale/kernel.cpp:165-171:
// dispatch(A, B, C, a_scale, b_scale) (C third, as in the reference).
#include "gemm_bind.h"

using namespace hkqbind;

void dispatch(py::object A, py::object B, py::object C, py::object a_scale, py::object b_scale) {
    gemm_a8w8(A, B, a_scale, b_scale, C);
}

PYBIND11_MODULE(gemm_a8w8_per_token_scale_tk, m) {
    m.doc() = "FP8 A8W8 GEMM with per-token x per-channel scales (gfx950 scaled MFMA)";
    m.def("dispatch", &dispatch, "C = (A . B^T) * a_scale[m] * b_scale[n]");
}
