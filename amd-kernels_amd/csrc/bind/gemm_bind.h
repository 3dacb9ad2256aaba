// gemm_bind.h -- argument handling shared by the dense GEMM modules.
#pragma once
#include "bind_common.h"

namespace hkqbind {

// A [M, K] and B [N, K] E4M3FN codes (float8_e4m3fn or their uint8 view);
// a_scale fp32 [M] / [M, 1]; b_scale fp32 [N] / [1, N] / [N, 1]; C bf16 [M, N].
inline void gemm_a8w8(py::object A, py::object B, py::object a_scale, py::object b_scale, py::object C) {
    auto a = view(A, "A"), b = view(B, "B"), sa = view(a_scale, "a_scale"), sb = view(b_scale, "b_scale"),
         c = view(C, "C");
    if (a.dtype == kBF16 || b.dtype == kBF16)
        throw py::type_error(
            "A and B must hold E4M3FN codes (torch.float8_e4m3fn or uint8); bf16 tensors carrying int8 values "
            "are not accepted -- quantize with quant_tk.per_token_quant_fwd into a float8_e4m3fn tensor");
    expect_dtype(a, "A", {kFP8, kU8});
    expect_dtype(b, "B", {kFP8, kU8});
    expect_dtype(sa, "a_scale", {kF32});
    expect_dtype(sb, "b_scale", {kF32});
    expect_dtype(c, "C", {kBF16});
    const int64_t lda = row_stride(a, "A"), ldb = row_stride(b, "B"), ldc = row_stride(c, "C");
    const int64_t M = a.dim(0), K = a.dim(1), N = b.dim(0);
    expect(b.dim(1) == K, "A and B must have the same K");
    expect(c.dim(0) == M && c.dim(1) == N, "C must be [M, N]");
    expect(sa.numel() == M && sa.contiguous(), "a_scale must be contiguous with M elements");
    expect(sb.numel() == N && sb.contiguous(), "b_scale must be contiguous with N elements");
    Workspace ws = workspace(hkq_gemm_a8w8_workspace(M, N, K), A);
    check(hkq_gemm_a8w8_ws((const void*)a.ptr, (const void*)b.ptr, (const float*)sa.ptr, (const float*)sb.ptr,
                           (void*)c.ptr, M, N, K, lda, ldb, ldc, ws.ptr, ws.bytes, current_stream()),
          "gemm_a8w8");
}

}  // namespace hkqbind
