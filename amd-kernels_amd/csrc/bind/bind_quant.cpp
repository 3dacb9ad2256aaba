// quant_tk -- per-token dynamic quantization, the reference module of
// kernels/quantization/quant/kernel.cpp:159-171 (per_token_quant_fwd), plus a
// 1 x group variant (group_quant_fwd) and SwiGLU + FP8 quantization
// (swiglu_quant_fwd), extensions of this build.
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

// input bf16 [M, 2F] (gate/up GEMM output); output [M, F] E4M3FN codes;
// scales fp32 [M] / [M, 1] (group_size 0: per token) or [M, F/128] (128).
void swiglu_quant_fwd(py::object input, py::object output, py::object scales, float alpha, bool interleaved,
                      int64_t group_size) {
    auto y = view(input, "input"), q = view(output, "output"), s = view(scales, "scales");
    expect_dtype(y, "input", {kBF16});
    expect_dtype(q, "output", {kFP8, kU8});
    expect_dtype(s, "scales", {kF32});
    expect(group_size == 0 || group_size == 128, "group_size must be 0 (per token) or 128");
    const int64_t ldy = row_stride(y, "input"), ldq = row_stride(q, "output");
    const int64_t M = y.dim(0), F = y.dim(1) / 2;
    expect(y.dim(1) % 2 == 0, "input must have an even number of columns (gate and up)");
    expect(q.dim(0) == M && q.dim(1) == F, "output must be [M, F]");
    int64_t lds = 0;
    if (group_size == 0) {
        expect(s.numel() == M && s.contiguous(), "scales must be a contiguous [M] or [M, 1] tensor");
    } else {
        expect(s.shape.size() == 2 && s.dim(0) == M && s.dim(1) == F / 128, "scales must be [M, F/128]");
        lds = row_stride(s, "scales");
    }
    check(hkq_swiglu_quant((const void*)y.ptr, (void*)q.ptr, (float*)s.ptr, M, F, ldy, ldq, lds, alpha,
                           interleaved ? 1 : 0, (int)group_size, current_stream()),
          "swiglu_quant_fwd");
}

PYBIND11_MODULE(quant_tk, m) {
    m.doc() = "Per-token / 1xG dynamic quantization (gfx950)";
    m.def("per_token_quant_fwd", &per_token_quant_fwd, "Per-token quantization (int8 or E4M3FN by output dtype)");
    m.def("group_quant_fwd", &group_quant_fwd, "1 x group_size quantization", py::arg("input"), py::arg("output"),
          py::arg("scales"), py::arg("group_size") = 128);
    m.def("swiglu_quant_fwd", &swiglu_quant_fwd, "SiLU-and-mul of a gate/up output + FP8 quantization",
          py::arg("input"), py::arg("output"), py::arg("scales"), py::arg("alpha") = 1.0f,
          py::arg("interleaved") = false, py::arg("group_size") = 0);
}
