// gemm_a8w8_blockscale_tk -- the reference module of
// kernels/gemm-basic/gemm_a8w8_blockscale/kernel.cpp:174-180:
// dispatch(A, B, C, a_scale, b_scale) (C third, as in the reference).
//   A [M, K], B [N, K]: E4M3FN codes (float8_e4m3fn or uint8)
//   a_scale fp32 [M, K/128]; b_scale fp32 [K/128, N] (per column, the
//   reference test's layout) or [K/128, ceil(N/128)] (128x128 weight blocks).
#include "gemm_bind.h"

using namespace hkqbind;

void dispatch(py::object A, py::object B, py::object C, py::object a_scale, py::object b_scale) {
    gemm_blockscale(A, B, C, a_scale, b_scale, py::none(), py::none(), "gemm_a8w8_blockscale");
}

PYBIND11_MODULE(gemm_a8w8_blockscale_tk, m) {
    m.doc() = "Block-scale FP8 GEMM: 1x128 activation and 128x128 (or 128x1) weight scales (gfx950)";
    m.def("dispatch", &dispatch, "C = sum_g (A_g . B_g^T) * a_scale[:, g] * b_scale[g, n / group_n]");
}
