// moe_topk_tk -- the reference module of kernels/moe-routing/moe_topk/kernel.cpp:303-339:
// moe_topk(X, stride_xm, Yv, Yi, stride_ym, Bits, stride_bm, stride_bn, n_rows,
// n_expts_tot, K, apply_softmax). X bf16 logits; Yv bf16 / Yi int32 [n_rows, K]
// at stride_ym; Bits int32/uint32 (None: skipped), word w of row r at
// r*stride_bm + w*stride_bn, ceil(n_expts_tot / 32) words per row.
#include "routing_bind.h"

using namespace hkqbind;

void moe_topk(py::object X, int64_t stride_xm, py::object Yv, py::object Yi, int64_t stride_ym, py::object Bits,
              int64_t stride_bm, int64_t stride_bn, int64_t n_rows, int64_t n_expts_tot, int K, bool apply_softmax) {
    expect(n_rows >= 0 && n_expts_tot >= 1 && K >= 1, "n_rows >= 0, n_expts_tot >= 1 and K >= 1 are required");
    expect(stride_xm >= 0 && stride_ym >= 0 && stride_bm >= 0 && stride_bn >= 0, "strides must be non-negative");
    auto x = routing_tensor(X, "X", {kBF16}, extent2(n_rows, stride_xm, n_expts_tot, 1));
    auto yv = routing_tensor(Yv, "Yv", {kBF16}, extent2(n_rows, stride_ym, K, 1));
    auto yi = routing_tensor(Yi, "Yi", {kI32}, extent2(n_rows, stride_ym, K, 1));
    uint32_t* bits = nullptr;
    if (!Bits.is_none())
        bits = (uint32_t*)routing_tensor(Bits, "Bits", {kI32, kU32},
                                         extent2(n_rows, stride_bm, (n_expts_tot + 31) / 32, stride_bn))
                   .ptr;
    check(hkq_moe_topk((const void*)x.ptr, stride_xm, (void*)yv.ptr, (int32_t*)yi.ptr, stride_ym, bits, stride_bm,
                       stride_bn, n_rows, n_expts_tot, K, apply_softmax ? 1 : 0, current_stream()),
          "moe_topk");
}

PYBIND11_MODULE(moe_topk_tk, m) {
    m.doc() = "MoE top-K expert selection with softmax and bitmatrix packing (gfx950)";
    m.def("moe_topk", &moe_topk, "Top-K experts per row, values, indices and bitmatrix", py::arg("X"),
          py::arg("stride_xm"), py::arg("Yv"), py::arg("Yi"), py::arg("stride_ym"), py::arg("Bits"),
          py::arg("stride_bm"), py::arg("stride_bn"), py::arg("n_rows"), py::arg("n_expts_tot"), py::arg("K"),
          py::arg("apply_softmax"));
}
