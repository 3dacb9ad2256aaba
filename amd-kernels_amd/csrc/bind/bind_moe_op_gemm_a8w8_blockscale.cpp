// moe_op_gemm_a8w8_blockscale_tk -- the reference module of
// kernels/moe-gemm/moe_op_gemm_a8w8_blockscale/kernel.cpp:244-280 (same
// function, argument names and order): X_scale [T, K/group_k] (strides
// xsm/xsk) and W_scale [E, K/group_k, ceil(N/group_n)] (strides wse/wsk/wsn),
// any group_k that is a multiple of 64 and group_n >= 1. group_k == K
// (per-token x per-channel-group scales) runs on the per-token MoE kernel,
// smaller groups on the per-group promotion kernel. W may be K-contiguous
// ([E, N, K]) or the reference's N-contiguous [E, K, N], read in place.
#include "moe_bind.h"

using namespace hkqbind;

void moe_a8w8_blockscale(py::object X, py::object W, py::object Y, py::object X_scale, py::object W_scale,
                         py::object bias, py::object GatherIndx, py::object ExptHist, py::object ExptOffs,
                         py::object ExptData, int N, int K, int group_k, int group_n, int grid_m, int grid_n,
                         int n_expts_act, int stride_ym, int stride_yn, int stride_xm, int stride_xk, int stride_we,
                         int stride_wk, int stride_wn, int stride_xsm, int stride_xsk, int stride_wse,
                         int stride_wsk, int stride_wsn) {
    (void)grid_n;
    expect(group_n >= 1, "group_n must be >= 1");
    expect(group_k == K || (group_k >= 64 && group_k % 64 == 0), "group_k must be K or a positive multiple of 64");
    if (group_k == K) {
        (void)stride_xsk;
        (void)stride_wsk;
        MoeScales sc;
        if (!X_scale.is_none()) {
            auto v = view(X_scale, "X_scale");
            expect_dtype(v, "X_scale", {kF32});
            sc.xs = (const float*)v.ptr;
            sc.xs_tok = stride_xsm;
        }
        if (!W_scale.is_none()) {
            auto v = view(W_scale, "W_scale");
            expect_dtype(v, "W_scale", {kF32});
            sc.ws = (const float*)v.ptr;
            sc.ws_e = stride_wse;
            sc.ws_n = stride_wsn;
            sc.ws_gn = group_n;
        }
        moe_call(X, W, Y, sc, bias, GatherIndx, ExptHist, ExptOffs, ExptData, N, K, grid_m, n_expts_act, stride_ym,
                 stride_yn, stride_xm, stride_xk, stride_we, stride_wk, stride_wn);
        return;
    }
    auto xs = view(X_scale, "X_scale"), ws = view(W_scale, "W_scale");
    expect_dtype(xs, "X_scale", {kF32});
    expect_dtype(ws, "W_scale", {kF32});
    MoeArgs a = moe_prepare(X, W, Y, bias, GatherIndx, ExptHist, ExptOffs, ExptData, N, K, grid_m, stride_ym,
                            stride_yn, stride_xm, stride_xk, stride_we, stride_wk, stride_wn, 64);
    const int64_t G = (K + group_k - 1) / group_k, C = (N + group_n - 1) / group_n;
    expect(a.T == 0 || xs.numel() >= (a.T - 1) * (int64_t)stride_xsm + (G - 1) * (int64_t)stride_xsk + 1,
           "X_scale is smaller than its strides say");
    expect(ws.numel() >= (a.E - 1) * (int64_t)stride_wse + (G - 1) * (int64_t)stride_wsk +
                             (C - 1) * (int64_t)stride_wsn + 1,
           "W_scale is smaller than its strides say");
    auto fn = a.kn ? hkq_moe_a8w8_blockscale_kn : hkq_moe_a8w8_blockscale;
    check(fn(a.X, a.W, a.Y, (const float*)xs.ptr, stride_xsm, stride_xsk, (const float*)ws.ptr, stride_wse, stride_wsk,
             stride_wsn, group_k, group_n, a.bias, N, a.gather, a.hist, a.offs, a.ed, a.T, a.E, N, K, grid_m,
             n_expts_act, a.stride_xm, a.stride_we, a.kn ? a.stride_wk : a.stride_wn, a.stride_ym, a.y_rows, a.glen,
             current_stream()),
          "moe_a8w8_blockscale");
}

PYBIND11_MODULE(moe_op_gemm_a8w8_blockscale_tk, m) {
    m.def("moe_a8w8_blockscale", &moe_a8w8_blockscale,
          "MoE E4M3FN grouped GEMM with per-K-group activation and weight scales", py::arg("X"),
          py::arg("W"), py::arg("Y"), py::arg("X_scale"), py::arg("W_scale"), py::arg("bias"), py::arg("GatherIndx"),
          py::arg("ExptHist"), py::arg("ExptOffs"), py::arg("ExptData"), py::arg("N"), py::arg("K"),
          py::arg("group_k"), py::arg("group_n"), py::arg("grid_m"), py::arg("grid_n"), py::arg("n_expts_act"),
          py::arg("stride_ym"), py::arg("stride_yn"), py::arg("stride_xm"), py::arg("stride_xk"),
          py::arg("stride_we"), py::arg("stride_wk"), py::arg("stride_wn"), py::arg("stride_xsm"),
          py::arg("stride_xsk"), py::arg("stride_wse"), py::arg("stride_wsk"), py::arg("stride_wsn"));
}
