// quant_moe_tk -- static FP8 and MX down/up-casts, the reference module of
// kernels/moe-misc/quant_moe/kernel.cpp:392-476 (same functions, argument
// names and order).
#include "bind_common.h"

using namespace hkqbind;

// x bf16 [M, N]; y uint8 / float8_e4m3fn [M, N]; scale fp32 [1].
void downcast_to_static_fp8(py::object x, py::object y, py::object scale, int64_t M, int64_t N) {
    auto xv = view(x, "x"), yv = view(y, "y"), sv = view(scale, "scale");
    expect_dtype(xv, "x", {kBF16});
    expect_dtype(yv, "y", {kU8, kFP8});
    expect_dtype(sv, "scale", {kF32});
    expect(xv.contiguous() && yv.contiguous(), "x and y must be contiguous");
    expect(xv.numel() >= M * N && yv.numel() >= M * N, "x and y must hold M * N elements");
    check(hkq_static_quant_fp8((const void*)xv.ptr, (void*)yv.ptr, (const float*)sv.ptr, M * N, current_stream()),
          "downcast_to_static_fp8");
}

// src bf16 [outer, quant]; mx_tensor uint8 [outer, quant / (2 if fp4 else 1)];
// mx_scale uint8 [outer, quant / 32].
void downcast_to_mxfp(py::object mx_tensor, py::object mx_scale, py::object src, int64_t outer_dim, int64_t quant_dim,
                      bool is_fp4) {
    auto q = view(mx_tensor, "mx_tensor"), s = view(mx_scale, "mx_scale"), x = view(src, "src");
    expect_dtype(x, "src", {kBF16});
    expect_dtype(q, "mx_tensor", {kU8, kFP8});
    expect_dtype(s, "mx_scale", {kU8});
    expect(x.contiguous() && q.contiguous() && s.contiguous(), "tensors must be contiguous");
    expect(x.numel() >= outer_dim * quant_dim, "src must hold outer_dim * quant_dim elements");
    expect(q.numel() >= outer_dim * quant_dim / (is_fp4 ? 2 : 1), "mx_tensor is too small");
    expect(s.numel() >= outer_dim * quant_dim / 32, "mx_scale is too small");
    check(hkq_mx_quant((const void*)x.ptr, (void*)q.ptr, (void*)s.ptr, outer_dim, quant_dim, quant_dim, is_fp4 ? 1 : 0,
                       current_stream()),
          "downcast_to_mxfp");
}

// out bf16 [outer, quant]
void upcast_from_mxfp(py::object out, py::object mx_scale, py::object mx_tensor, int64_t outer_dim, int64_t quant_dim,
                      bool is_fp4) {
    auto o = view(out, "out"), s = view(mx_scale, "mx_scale"), q = view(mx_tensor, "mx_tensor");
    expect_dtype(o, "out", {kBF16});
    expect_dtype(q, "mx_tensor", {kU8, kFP8});
    expect_dtype(s, "mx_scale", {kU8});
    expect(o.contiguous() && q.contiguous() && s.contiguous(), "tensors must be contiguous");
    expect(o.numel() >= outer_dim * quant_dim, "out must hold outer_dim * quant_dim elements");
    expect(q.numel() >= outer_dim * quant_dim / (is_fp4 ? 2 : 1), "mx_tensor is too small");
    expect(s.numel() >= outer_dim * quant_dim / 32, "mx_scale is too small");
    check(hkq_mx_dequant((const void*)q.ptr, (const void*)s.ptr, (void*)o.ptr, outer_dim, quant_dim, is_fp4 ? 1 : 0,
                         current_stream()),
          "upcast_from_mxfp");
}

PYBIND11_MODULE(quant_moe_tk, m) {
    m.def("downcast_to_static_fp8", &downcast_to_static_fp8, "Convert tensor to FP8 with static scaling",
          py::arg("x"), py::arg("y"), py::arg("scale"), py::arg("M"), py::arg("N"));
    m.def("downcast_to_mxfp", &downcast_to_mxfp, "Convert tensor to MX format (FP8/FP4 with per-32-element scales)",
          py::arg("mx_tensor"), py::arg("mx_scale"), py::arg("src"), py::arg("outer_dim"), py::arg("quant_dim"),
          py::arg("is_fp4"));
    m.def("upcast_from_mxfp", &upcast_from_mxfp, "Convert MX format back to bf16", py::arg("out"),
          py::arg("mx_scale"), py::arg("mx_tensor"), py::arg("outer_dim"), py::arg("quant_dim"), py::arg("is_fp4"));
}
