// quant_tk -- per-token dynamic quantization, the reference module of
// kernels/quantization/quant/kernel.cpp:159-171 (per_token_quant_fwd), plus a
// 1 x group variant (group_quant_fwd, an extension of this build).
#include "bind_common.h"

using namespace hkqbind;

static int kind_of(const TensorView& q) {
    expect_dtype(q, "output", {kI8, kFP8, kU8});
    return q.dtype == kI8 ? HKQ_KIND_INT8 : HKQ_KIND_FP8;
}

// input bf16 [M, D]; output int8 (QMAX 127) or float8_e4m3fn / uint8 (E4M3FN,
// QMAX 448) [M, D]; scales fp32 [M, 1] or [M].
void per_token_quant_fwd(py::object input, py::object output, py::object scales) {
    auto x = view(input, "input"), q = view(output, "output"), s = view(scales, "scales");
    expect_dtype(x, "input", {kBF16});
    expect_dtype(s, "scales", {kF32});
    const int kind = kind_of(q);
    const int64_t ldx = row_stride(x, "input"), ldq = row_stride(q, "output");
    const int64_t M = x.dim(0), K = x.dim(1);
    expect(q.dim(0) == M && q.dim(1) == K, "output must have the shape of input");
    expect(s.numel() == M && s.contiguous(), "scales must be a contiguous [M, 1] or [M] tensor");
    check(hkq_per_token_quant((const void*)x.ptr, (void*)q.ptr, (float*)s.ptr, M, K, ldx, ldq, kind, current_stream()),
          "per_token_quant_fwd");
}

// input bf16 [M, K]; output [M, K] as above; scales fp32 [M, K / group_size].
void group_quant_fwd(py::object input, py::object output, py::object scales, int64_t group_size) {
    auto x = view(input, "input"), q = view(output, "output"), s = view(scales, "scales");
    expect_dtype(x, "input", {kBF16});
    expect_dtype(s, "scales", {kF32});
    const int kind = kind_of(q);
    const int64_t ldx = row_stride(x, "input"), ldq = row_stride(q, "output");
    const int64_t M = x.dim(0), K = x.dim(1);
    expect(group_size > 0 && K % group_size == 0, "K must be a multiple of group_size");
    expect(q.dim(0) == M && q.dim(1) == K, "output must have the shape of input");
    expect(s.shape.size() == 2 && s.dim(0) == M && s.dim(1) == K / group_size,
           "scales must be [M, K / group_size]");
    const int64_t lds = row_stride(s, "scales");
    check(hkq_group_quant((const void*)x.ptr, (void*)q.ptr, (float*)s.ptr, M, K, ldx, ldq, lds, group_size, kind,
                          current_stream()),
          "group_quant_fwd");
}

PYBIND11_MODULE(quant_tk, m) {
    m.doc() = "Per-token / 1xG dynamic quantization (gfx950)";
    m.def("per_token_quant_fwd", &per_token_quant_fwd, "Per-token quantization (int8 or E4M3FN by output dtype)");
    m.def("group_quant_fwd", &group_quant_fwd, "1 x group_size quantization", py::arg("input"), py::arg("output"),
          py::arg("scales"), py::arg("group_size") = 128);
}
