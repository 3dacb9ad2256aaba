// moe_bind.h -- argument handling shared by the two A8W8 MoE GEMM modules
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

// Tensors and strides of one MoE call after validation. W points at
// K-contiguous rows (stride_wn), or (kn) at the reference's N-contiguous
// [E, K, N] weights, read in place (stride_wk) when K is a multiple of
// kn_kmul (the kernels' K-tile; 0: never); other N-contiguous weights are
// copied K-major into `packed` (kept alive until the launch is queued).
struct MoeArgs {
    const void* X = nullptr;
    const void* W = nullptr;
    void* Y = nullptr;
    const float* bias = nullptr;
    const int32_t *gather = nullptr, *hist = nullptr, *offs = nullptr, *ed = nullptr;
    int64_t T = 0, E = 0, glen = 0, y_rows = 0;
    int64_t stride_xm = 0, stride_we = 0, stride_wn = 0, stride_wk = 0, stride_ym = 0;
    bool kn = false;
    Workspace packed;
};

inline MoeArgs moe_prepare(py::object X, py::object W, py::object Y, py::object bias, py::object GatherIndx,
                           py::object ExptHist, py::object ExptOffs, py::object ExptData, int N, int K, int grid_m,
                           int stride_ym, int stride_yn, int stride_xm, int stride_xk, int stride_we, int stride_wk,
                           int stride_wn, int kn_kmul = 0) {
    auto x = view(X, "X"), w = view(W, "W"), y = view(Y, "Y");
    if (x.dtype == kBF16 || x.dtype == kI8 || w.dtype == kBF16 || w.dtype == kI8)
        throw py::type_error("X and W must hold E4M3FN codes (torch.float8_e4m3fn or uint8)");
    expect_dtype(x, "X", {kFP8, kU8});
    expect_dtype(w, "W", {kFP8, kU8});
    expect_dtype(y, "Y", {kBF16});
    expect(stride_xk == 1, "X must be K-contiguous (stride_xk == 1)");
    expect(stride_yn == 1, "Y must be N-contiguous (stride_yn == 1)");
    expect(stride_wk == 1 || stride_wn == 1, "W must be K-contiguous (stride_wk == 1) or N-contiguous (stride_wn == 1)");
    auto hist = view(ExptHist, "ExptHist"), offs = view(ExptOffs, "ExptOffs"), ed = view(ExptData, "ExptData");
    expect_dtype(hist, "ExptHist", {kI32});
    expect_dtype(offs, "ExptOffs", {kI32});
    expect_dtype(ed, "ExptData", {kI32});
    expect(ed.numel() >= grid_m, "ExptData must hold grid_m entries");
    MoeArgs a;
    a.E = hist.numel();
    expect(offs.numel() == a.E, "ExptHist and ExptOffs must have one entry per expert");
    if (!GatherIndx.is_none()) {
        auto g = view(GatherIndx, "GatherIndx");
        expect_dtype(g, "GatherIndx", {kI32});
        a.gather = (const int32_t*)g.ptr;
        a.glen = g.numel();
    }
    if (!bias.is_none()) {
        auto bv = view(bias, "bias");
        expect_dtype(bv, "bias", {kF32});
        expect(bv.numel() >= a.E * N && bv.contiguous(), "bias must be a contiguous [E, N] fp32 tensor");
        a.bias = (const float*)bv.ptr;
    }
    a.X = (const void*)x.ptr;
    a.Y = (void*)y.ptr;
    a.hist = (const int32_t*)hist.ptr;
    a.offs = (const int32_t*)offs.ptr;
    a.ed = (const int32_t*)ed.ptr;
    a.T = x.dim(0);
    a.y_rows = y.dim(0);
    a.stride_xm = stride_xm;
    a.stride_ym = stride_ym;
    if (stride_wk == 1) {
        a.W = (const void*)w.ptr;
        a.stride_we = stride_we;
        a.stride_wn = stride_wn;
    } else if (kn_kmul > 0 && K % kn_kmul == 0) {
        // the reference's [E, K, N] layout (tests/test_moe.py:723-729), read in place
        expect(w.numel() >= (a.E - 1) * (int64_t)stride_we + (int64_t)(K - 1) * stride_wk + N,
               "W is smaller than its strides say");
        a.W = (const void*)w.ptr;
        a.stride_we = stride_we;
        a.stride_wk = stride_wk;
        a.kn = true;
    } else {
        // the reference's [E, K, N] layout (tests/test_moe.py:723-729): rows of
        // K per output channel are what the kernels stream, so copy it K-major
        expect(w.numel() >= (a.E - 1) * (int64_t)stride_we + (int64_t)(K - 1) * stride_wk + N,
               "W is smaller than its strides say");
        a.packed = pack_kmajor(W, w.ptr, a.E, K, N, stride_we, stride_wk, "moe weight prepack");
        a.W = a.packed.ptr;
        a.stride_we = (int64_t)N * K;
        a.stride_wn = K;
    }
    return a;
}

inline void moe_call(py::object X, py::object W, py::object Y, const MoeScales& sc, py::object bias,
                     py::object GatherIndx, py::object ExptHist, py::object ExptOffs, py::object ExptData, int N,
                     int K, int grid_m, int n_expts_act, int stride_ym, int stride_yn, int stride_xm, int stride_xk,
                     int stride_we, int stride_wk, int stride_wn) {
    MoeArgs a = moe_prepare(X, W, Y, bias, GatherIndx, ExptHist, ExptOffs, ExptData, N, K, grid_m, stride_ym,
                            stride_yn, stride_xm, stride_xk, stride_we, stride_wk, stride_wn, 128);
    auto fn = a.kn ? hkq_moe_a8w8_kn : hkq_moe_a8w8;
    check(fn(a.X, a.W, a.Y, sc.xs, sc.xs_tok, sc.ws, sc.ws_e, sc.ws_n, sc.ws_gn, a.bias, N, a.gather, a.hist, a.offs,
             a.ed, a.T, a.E, N, K, grid_m, n_expts_act, a.stride_xm, a.stride_we, a.kn ? a.stride_wk : a.stride_wn,
             a.stride_ym, a.y_rows, a.glen, current_stream()),
          "moe");
}

}  // namespace hkqbind
