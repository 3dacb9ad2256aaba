// fused_gemm_a8w8_blockscale_a16w16_tk -- the reference module of
// kernels/gemm-fused/fused_gemm_a8w8_blockscale_a16w16/kernel.cpp:251-270:
// dispatch(a_fp8, b_fp8, c_fp8, a_scale, b_scale, a_bf16, b_bf16, c_bf16)
// (tests/test_gemm.py:454-496): two independent GEMMs sharing M,
//   c_fp8  = block-scale FP8 GEMM of a_fp8 [M, K], b_fp8 [N8, K] (E4M3FN codes,
//            a_scale [M, K/128], b_scale [K/128, N8] or [K/128, ceil(N8/128)])
//   c_bf16 = a_bf16 [M, K16] . b_bf16 [N16, K16]^T (bf16)
// issued back to back on the current stream (they share no operand, so one
// launch would only save a launch).
#include "gemm_bind.h"

using namespace hkqbind;

void dispatch(py::object a_fp8, py::object b_fp8, py::object c_fp8, py::object a_scale, py::object b_scale,
              py::object a_bf16, py::object b_bf16, py::object c_bf16) {
    const int64_t m8 = view(a_fp8, "a_fp8").dim(0), m16 = view(a_bf16, "a_bf16").dim(0);
    expect(m8 == m16, "a_fp8 and a_bf16 must have the same number of rows");
    gemm_blockscale(a_fp8, b_fp8, c_fp8, a_scale, b_scale, py::none(), py::none(),
                    "fused_gemm_a8w8_blockscale_a16w16 (block-scale part)");
    gemm_bf16(a_bf16, b_bf16, c_bf16, "fused_gemm_a8w8_blockscale_a16w16 (bf16 part)");
}

PYBIND11_MODULE(fused_gemm_a8w8_blockscale_a16w16_tk, m) {
    m.doc() = "Block-scale FP8 GEMM and bf16 GEMM over the same rows (gfx950)";
    m.def("dispatch", &dispatch, "c_fp8 = blockscale_gemm(a_fp8, b_fp8); c_bf16 = a_bf16 . b_bf16^T");
}
