// fused_fp8_quant_tk -- the reference module of kernels/quantization/fused_fp8_quant/kernel.cpp:251-275:
// fused_rmsnorm_fp8_quant_fwd(input, weight, output, scales, eps). input bf16
// [M, D]; weight bf16 [D]; output [M, D] E4M3FN codes (float8_e4m3fn or
// uint8); scales fp32 [M, D/128]. D any multiple of 128 up to 8192 (the
// reference: 4096 or 8192).
#include "bind_common.h"

using namespace hkqbind;

void fused_rmsnorm_fp8_quant_fwd(py::object input, py::object weight, py::object output, py::object scales,
                                 float eps) {
    auto x = view(input, "input"), w = view(weight, "weight"), q = view(output, "output"), s = view(scales, "scales");
    expect_dtype(x, "input", {kBF16});
    expect_dtype(w, "weight", {kBF16});
    expect_dtype(q, "output", {kFP8, kU8});
    expect_dtype(s, "scales", {kF32});
    const int64_t ldx = row_stride(x, "input"), ldq = row_stride(q, "output");
    const int64_t M = x.dim(0), D = x.dim(1);
    expect(D % 128 == 0 && D <= 8192, "D must be a multiple of 128, at most 8192");
    expect(w.numel() == D && w.contiguous(), "weight must be a contiguous [D] tensor");
    expect(q.dim(0) == M && q.dim(1) == D, "output must be [M, D]");
    expect(s.shape.size() == 2 && s.dim(0) == M && s.dim(1) == D / 128, "scales must be [M, D/128]");
    const int64_t lds = row_stride(s, "scales");
    check(hkq_rmsnorm_quant((const void*)x.ptr, (const void*)w.ptr, (void*)q.ptr, (void*)s.ptr, M, D, ldx, ldq, lds,
                            eps, 0, current_stream()),
          "fused_rmsnorm_fp8_quant_fwd");
}

PYBIND11_MODULE(fused_fp8_quant_tk, m) {
    m.doc() = "Fused RMSNorm + 1x128 FP8 (E4M3FN) quantization (gfx950)";
    m.def("fused_rmsnorm_fp8_quant_fwd", &fused_rmsnorm_fp8_quant_fwd, "Fused RMSNorm + FP8 quantization forward pass",
          py::arg("input"), py::arg("weight"), py::arg("output"), py::arg("scales"), py::arg("eps"));
}
