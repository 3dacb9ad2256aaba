// gemm_a8w8_tk -- the reference module of kernels/gemm-basic/gemm_a8w8/kernel.cpp:169-175:
// dispatch(A, B, a_scale, b_scale, C).
#include "gemm_bind.h"

using namespace hkqbind;

void dispatch(py::object A, py::object B, py::object a_scale, py::object b_scale, py::object C) {
    gemm_a8w8(A, B, a_scale, b_scale, C);
}

PYBIND11_MODULE(gemm_a8w8_tk, m) {
    m.doc() = "FP8 A8W8 GEMM with per-token x per-channel scales (gfx950 scaled MFMA)";
    m.def("dispatch", &dispatch, "C = (A . B^T) * a_scale[m] * b_scale[n]");
}
