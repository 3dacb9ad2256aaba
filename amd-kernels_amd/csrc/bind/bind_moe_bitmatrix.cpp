// moe_bitmatrix_tk -- the reference module of kernels/moe-routing/moe_bitmatrix/kernel.cpp:318-377:
// sum_bitmatrix_rows(B, shape_bm, stride_bm, stride_bn, Ret, Partials, stride_pm,
// stride_pn, shape_pn, shape_bn) and sum_bitmatrix_rows_fused(B, shape_bm,
// stride_bm, stride_bn, Ret, N_BLKS_BITMATRIX). B int32/uint32 words; Ret gets
// 32 * shape_bn counts; Partials[t*stride_pm + e*stride_pn] for 128-row tiles t
// and expert columns e < shape_pn.
#include "routing_bind.h"

using namespace hkqbind;

static TensorView bits_arg(const py::object& B, int64_t rows, int64_t sbm, int64_t sbn, int64_t nw) {
    expect(rows >= 0 && nw >= 1 && sbm >= 0 && sbn >= 0, "shape_bm >= 0, shape_bn >= 1 and non-negative strides are required");
    return routing_tensor(B, "B", {kI32, kU32}, extent2(rows, sbm, nw, sbn));
}

void sum_bitmatrix_rows(py::object B, int64_t shape_bm, int64_t stride_bm, int64_t stride_bn, py::object Ret,
                        py::object Partials, int64_t stride_pm, int64_t stride_pn, int64_t shape_pn,
                        int64_t shape_bn) {
    auto b = bits_arg(B, shape_bm, stride_bm, stride_bn, shape_bn);
    auto r = routing_tensor(Ret, "Ret", {kI32, kU32}, 32 * shape_bn);
    expect(stride_pm >= 0 && stride_pn >= 0 && shape_pn >= 0, "Partials strides and shape_pn must be non-negative");
    const int64_t ntiles = (shape_bm + 127) / 128;
    auto p = routing_tensor(Partials, "Partials", {kI32, kU32},
                            extent2(ntiles, stride_pm, std::min<int64_t>(shape_pn, 32 * shape_bn), stride_pn));
    check(hkq_sum_bitmatrix_rows((const uint32_t*)b.ptr, shape_bm, stride_bm, stride_bn, (uint32_t*)r.ptr,
                                 (uint32_t*)p.ptr, stride_pm, stride_pn, shape_pn, shape_bn, current_stream()),
          "sum_bitmatrix_rows");
}

void sum_bitmatrix_rows_fused(py::object B, int64_t shape_bm, int64_t stride_bm, int64_t stride_bn, py::object Ret,
                              int64_t N_BLKS_BITMATRIX) {
    auto b = bits_arg(B, shape_bm, stride_bm, stride_bn, N_BLKS_BITMATRIX);
    auto r = routing_tensor(Ret, "Ret", {kI32, kU32}, 32 * N_BLKS_BITMATRIX);
    check(hkq_sum_bitmatrix_rows_fused((const uint32_t*)b.ptr, shape_bm, stride_bm, stride_bn, (uint32_t*)r.ptr,
                                       N_BLKS_BITMATRIX, current_stream()),
          "sum_bitmatrix_rows_fused");
}

PYBIND11_MODULE(moe_bitmatrix_tk, m) {
    m.doc() = "Column sums of the MoE expert bitmatrix with per-128-row exclusive partials (gfx950)";
    m.def("sum_bitmatrix_rows", &sum_bitmatrix_rows, "Per-expert counts and per-tile exclusive partials",
          py::arg("B"), py::arg("shape_bm"), py::arg("stride_bm"), py::arg("stride_bn"), py::arg("Ret"),
          py::arg("Partials"), py::arg("stride_pm"), py::arg("stride_pn"), py::arg("shape_pn"), py::arg("shape_bn"));
    m.def("sum_bitmatrix_rows_fused", &sum_bitmatrix_rows_fused, "Per-expert counts", py::arg("B"),
          py::arg("shape_bm"), py::arg("stride_bm"), py::arg("stride_bn"), py::arg("Ret"),
          py::arg("N_BLKS_BITMATRIX"));
}
