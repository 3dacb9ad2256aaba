// fused_mxfp4_quant_tk -- the reference module of kernels/quantization/fused_mxfp4_quant/kernel.cpp:291-314:
// fused_rmsnorm_mxfp4_quant_fwd(input, weight, output, scales, eps). input bf16
// [M, D]; weight bf16 [D]; output uint8 [M, D/2] (two E2M1 codes per byte,
// even column in the low nibble); scales uint8 e8m0 [M, D/32]. D any multiple
// of 32 up to 8192 (the reference: 4096 or 8192). Elements take the
// reference's threshold ladder (kernel.cpp:128-150: the largest E2M1 magnitude
// at or below |y| * 2^-e), so codes and scales equal the reference module's.
#include "bind_common.h"

using namespace hkqbind;

void fused_rmsnorm_mxfp4_quant_fwd(py::object input, py::object weight, py::object output, py::object scales,
                                   float eps) {
    auto x = view(input, "input"), w = view(weight, "weight"), q = view(output, "output"), s = view(scales, "scales");
    expect_dtype(x, "input", {kBF16});
    expect_dtype(w, "weight", {kBF16});
    expect_dtype(q, "output", {kU8});
    expect_dtype(s, "scales", {kU8});
    const int64_t ldx = row_stride(x, "input"), ldq = row_stride(q, "output");
    const int64_t M = x.dim(0), D = x.dim(1);
    expect(D % 32 == 0 && D >= 128 && D <= 8192, "D must be a multiple of 32 in [128, 8192]");
    expect(w.numel() == D && w.contiguous(), "weight must be a contiguous [D] tensor");
    expect(q.dim(0) == M && q.dim(1) == D / 2, "output must be [M, D/2]");
    expect(s.shape.size() == 2 && s.dim(0) == M && s.dim(1) == D / 32, "scales must be [M, D/32]");
    const int64_t lds = row_stride(s, "scales");
    check(hkq_rmsnorm_quant((const void*)x.ptr, (const void*)w.ptr, (void*)q.ptr, (void*)s.ptr, M, D, ldx, ldq, lds,
                            eps, 2, current_stream()),
          "fused_rmsnorm_mxfp4_quant_fwd");
}

PYBIND11_MODULE(fused_mxfp4_quant_tk, m) {
    m.doc() = "Fused RMSNorm + MXFP4 quantization (gfx950)";
    m.def("fused_rmsnorm_mxfp4_quant_fwd", &fused_rmsnorm_mxfp4_quant_fwd,
          "Fused RMSNorm + MXFP4 quantization forward pass", py::arg("input"), py::arg("weight"), py::arg("output"),
          py::arg("scales"), py::arg("eps"));
}
