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

// Block-scale FP8 GEMM: A [M, K], B [N, K] E4M3FN codes; a_scale fp32
// [M, K/128]; b_scale fp32 [K/128, N] (per column) or [K/128, ceil(N/128)]
// (128x128 weight blocks); C bf16 [M, N]. With c_a / c_b (bf16 [M, N], not
// None): C = c_a * GEMM + c_b, formed in fp32 before the one rounding to bf16.
inline void gemm_blockscale(py::object A, py::object B, py::object C, py::object a_scale, py::object b_scale,
                            py::object c_a, py::object c_b, const char* what) {
    auto a = view(A, "A"), b = view(B, "B"), c = view(C, "C"), sa = view(a_scale, "a_scale"),
         sb = view(b_scale, "b_scale");
    if (a.dtype == kBF16 || b.dtype == kBF16)
        throw py::type_error("A and B must hold E4M3FN codes (torch.float8_e4m3fn or uint8); quantize with "
                             "quant_tk.group_quant_fwd (activations, 1x128) first");
    expect_dtype(a, "A", {kFP8, kU8});
    expect_dtype(b, "B", {kFP8, kU8});
    expect_dtype(sa, "a_scale", {kF32});
    expect_dtype(sb, "b_scale", {kF32});
    expect_dtype(c, "C", {kBF16});
    const int64_t lda = row_stride(a, "A"), ldb = row_stride(b, "B"), ldc = row_stride(c, "C");
    const int64_t M = a.dim(0), K = a.dim(1), N = b.dim(0);
    expect(b.dim(1) == K, "A and B must have the same K");
    expect(c.dim(0) == M && c.dim(1) == N, "C must be [M, N]");
    expect(K % 128 == 0, "K must be a multiple of 128");
    expect(sa.shape.size() == 2 && sa.dim(0) == M && sa.dim(1) == K / 128, "a_scale must be [M, K/128]");
    expect(sb.shape.size() == 2 && sb.dim(0) == K / 128, "b_scale must be [K/128, N] or [K/128, ceil(N/128)]");
    int64_t group_n;
    if (sb.dim(1) == N) group_n = 1;
    else if (sb.dim(1) == (N + 127) / 128) group_n = 128;
    else throw py::value_error("b_scale must be [K/128, N] or [K/128, ceil(N/128)]");
    const int64_t lsa = row_stride(sa, "a_scale"), lsb = row_stride(sb, "b_scale");
    if (c_a.is_none() && c_b.is_none()) {
        check(hkq_gemm_blockscale((const void*)a.ptr, (const void*)b.ptr, (const float*)sa.ptr, (const float*)sb.ptr,
                                  (void*)c.ptr, M, N, K, lda, ldb, lsa, lsb, ldc, group_n, current_stream()),
              what);
        return;
    }
    auto ca = view(c_a, "c_a"), cb = view(c_b, "c_b");
    expect_dtype(ca, "c_a", {kBF16});
    expect_dtype(cb, "c_b", {kBF16});
    expect(ca.shape.size() == 2 && ca.dim(0) == M && ca.dim(1) == N, "c_a must be [M, N]");
    expect(cb.shape.size() == 2 && cb.dim(0) == M && cb.dim(1) == N, "c_b must be [M, N]");
    check(hkq_gemm_blockscale_mul_add((const void*)a.ptr, (const void*)b.ptr, (const float*)sa.ptr,
                                      (const float*)sb.ptr, (void*)c.ptr, (const void*)ca.ptr, (const void*)cb.ptr, M,
                                      N, K, lda, ldb, lsa, lsb, ldc, row_stride(ca, "c_a"), row_stride(cb, "c_b"),
                                      group_n, current_stream()),
          what);
}

// A [M, K], B [N, K], C [M, N]: bf16, last dimensions contiguous.
inline void gemm_bf16(py::object A, py::object B, py::object C, const char* what) {
    auto a = view(A, "A"), b = view(B, "B"), c = view(C, "C");
    expect_dtype(a, "A", {kBF16});
    expect_dtype(b, "B", {kBF16});
    expect_dtype(c, "C", {kBF16});
    const int64_t lda = row_stride(a, "A"), ldb = row_stride(b, "B"), ldc = row_stride(c, "C");
    const int64_t M = a.dim(0), K = a.dim(1), N = b.dim(0);
    expect(b.dim(1) == K, "A and B must have the same K");
    expect(c.dim(0) == M && c.dim(1) == N, "C must be [M, N]");
    Workspace ws = workspace(hkq_gemm_bf16_workspace(M, N, K), A);
    check(hkq_batched_gemm_bf16((const void*)a.ptr, (const void*)b.ptr, nullptr, (void*)c.ptr, 1, M, N, K, lda, ldb,
                                ldc, 0, 0, 0, 0, ws.ptr, ws.bytes, current_stream()),
          what);
}

// A batch of row-major matrices: the reference's 4-D (1, B, R, C) layout or a
// plain (B, R, C) tensor, last dimension contiguous.
struct Batched {
    int64_t batch, rows, cols, bstride, ld;
};
inline Batched batched(const TensorView& v, const char* name) {
    const size_t nd = v.shape.size();
    expect(nd == 3 || (nd == 4 && v.shape[0] == 1), std::string(name) + " must be (1, B, R, C) or (B, R, C)");
    const size_t o = nd - 3;
    Batched b{v.shape[o], v.shape[o + 1], v.shape[o + 2], v.stride[o], v.stride[o + 1]};
    expect(v.stride[o + 2] == 1 || b.cols == 1, std::string(name) + " must have a contiguous last dimension");
    if (b.rows <= 1) b.ld = std::max<int64_t>(b.cols, b.ld);
    return b;
}

// A per-batch vector of n values: (1, B, 1, n), (B, 1, n) or (B, n), contiguous
// within a batch; returns the batch stride (elements).
inline int64_t batched_vec(const TensorView& v, const char* name, int64_t batch, int64_t n) {
    const size_t nd = v.shape.size();
    int64_t lead = 1, total = 1;
    for (size_t i = 0; i < nd; ++i) total *= v.shape[i];
    expect(nd >= 2 && v.shape[nd - 1] == n && total == batch * n,
           std::string(name) + " must hold " + std::to_string(n) + " values per batch ((1, B, 1, " + std::to_string(n) +
               ") or (B, " + std::to_string(n) + "))");
    expect(v.stride[nd - 1] == 1 || n == 1, std::string(name) + " must be contiguous within a batch");
    // the batch dimension is the last one of size B before the vector
    for (int i = (int)nd - 2; i >= 0; --i)
        if (v.shape[i] == batch) {
            lead = v.stride[i];
            break;
        }
    return batch <= 1 ? 0 : lead;
}

}  // namespace hkqbind
