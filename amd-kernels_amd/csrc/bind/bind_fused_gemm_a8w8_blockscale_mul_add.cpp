// fused_gemm_a8w8_blockscale_mul_add_tk -- the reference module of
// kernels/gemm-fused/fused_gemm_a8w8_blockscale_mul_add/kernel.cpp:176-192:
// dispatch(a, b, c, a_scale, b_scale, c_a, c_b) (tests/test_gemm.py:498-533):
//   c = c_a * (sum_g (a_g . b_g^T) * a_scale[:, g] * b_scale[g, n / group_n]) + c_b
// with a [M, K], b [N, K] E4M3FN codes, the block-scale GEMM's scale layouts,
// c, c_a, c_b bf16 [M, N]; the multiply-add runs in the GEMM's epilogue on the
// fp32 sums.
#include "gemm_bind.h"

using namespace hkqbind;

void dispatch(py::object a, py::object b, py::object c, py::object a_scale, py::object b_scale, py::object c_a,
              py::object c_b) {
    if (c_a.is_none() || c_b.is_none()) throw py::type_error("c_a and c_b must be tensors");
    gemm_blockscale(a, b, c, a_scale, b_scale, c_a, c_b, "fused_gemm_a8w8_blockscale_mul_add");
}

PYBIND11_MODULE(fused_gemm_a8w8_blockscale_mul_add_tk, m) {
    m.doc() = "Block-scale FP8 GEMM with a multiply-add epilogue (gfx950)";
    m.def("dispatch", &dispatch, "c = c_a * blockscale_gemm(a, b) + c_b");
}
