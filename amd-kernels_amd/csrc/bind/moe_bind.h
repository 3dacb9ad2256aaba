// moe_bind.h -- argument handling shared by the two MoE GEMM modules
// (reference argument names and orders; strides in elements).
#pragma once
#include "bind_common.h"

namespace hkqbind {

struct MoeScales {
    const float* xs = nullptr;
    int64_t xs_tok = 0;
    const float* ws = nullptr;
    int64_t ws_e = 0, ws_n = 0, ws_gn = 1;
};

inline void moe_call(py::object X, py::object W, py::object Y, const MoeScales& sc, py::object bias,
                     py::object GatherIndx, py::object ExptHist, py::object ExptOffs, py::object ExptData, int N,
                     int K, int grid_m, int n_expts_act, int stride_ym, int stride_yn, int stride_xm, int stride_xk,
                     int stride_we, int stride_wk, int stride_wn) {
    auto x = view(X, "X"), w = view(W, "W"), y = view(Y, "Y");
    if (x.dtype == kBF16 || x.dtype == kI8 || w.dtype == kBF16 || w.dtype == kI8)
        throw py::type_error("X and W must hold E4M3FN codes (torch.float8_e4m3fn or uint8)");
    expect_dtype(x, "X", {kFP8, kU8});
    expect_dtype(w, "W", {kFP8, kU8});
    expect_dtype(y, "Y", {kBF16});
    expect(stride_xk == 1, "X must be K-contiguous (stride_xk == 1)");
    expect(stride_yn == 1, "Y must be N-contiguous (stride_yn == 1)");
    expect(stride_wk == 1,
           "W must be K-contiguous (stride_wk == 1): pass W[e] as [N, K], e.g. W.transpose(1, 2).contiguous() "
           "with strides (N*K, 1, K)");
    auto hist = view(ExptHist, "ExptHist"), offs = view(ExptOffs, "ExptOffs"), ed = view(ExptData, "ExptData");
    expect_dtype(hist, "ExptHist", {kI32});
    expect_dtype(offs, "ExptOffs", {kI32});
    expect_dtype(ed, "ExptData", {kI32});
    expect(ed.numel() >= grid_m, "ExptData must hold grid_m entries");
    const int64_t E = hist.numel();
    expect(offs.numel() == E, "ExptHist and ExptOffs must have one entry per expert");
    const int32_t* gather = nullptr;
    int64_t glen = 0;
    if (!GatherIndx.is_none()) {
        auto g = view(GatherIndx, "GatherIndx");
        expect_dtype(g, "GatherIndx", {kI32});
        gather = (const int32_t*)g.ptr;
        glen = g.numel();
    }
    const float* b = nullptr;
    if (!bias.is_none()) {
        auto bv = view(bias, "bias");
        expect_dtype(bv, "bias", {kF32});
        expect(bv.numel() >= E * N && bv.contiguous(), "bias must be a contiguous [E, N] fp32 tensor");
        b = (const float*)bv.ptr;
    }
    const int64_t T = x.dim(0);
    const int64_t y_rows = y.dim(0);
    check(hkq_moe_a8w8((const void*)x.ptr, (const void*)w.ptr, (void*)y.ptr, sc.xs, sc.xs_tok, sc.ws, sc.ws_e,
                       sc.ws_n, sc.ws_gn, b, N, gather, (const int32_t*)hist.ptr, (const int32_t*)offs.ptr,
                       (const int32_t*)ed.ptr, T, E, N, K, grid_m, n_expts_act, stride_xm, stride_we, stride_wn,
                       stride_ym, y_rows, glen, current_stream()),
          "moe");
}

}  // namespace hkqbind
