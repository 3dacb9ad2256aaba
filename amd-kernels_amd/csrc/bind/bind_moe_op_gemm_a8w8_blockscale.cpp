// moe_op_gemm_a8w8_blockscale_tk -- the reference module of
// kernels/moe-gemm/moe_op_gemm_a8w8_blockscale/kernel.cpp:244-280 (same
// function, argument names and order). Supported granularity: group_k == K,
// i.e. X_scale [T, 1] (per token, strides xsm/xsk) and W_scale
// [E, 1, ceil(N/group_n)] (per expert x output-channel group, strides
// wse/wsk/wsn) -- with group_n == 1 this is per-token x per-channel scaling.
// group_k < K raises ValueError.
#include "moe_bind.h"

using namespace hkqbind;

void moe_a8w8_blockscale(py::object X, py::object W, py::object Y, py::object X_scale, py::object W_scale,
                         py::object bias, py::object GatherIndx, py::object ExptHist, py::object ExptOffs,
                         py::object ExptData, int N, int K, int group_k, int group_n, int grid_m, int grid_n,
                         int n_expts_act, int stride_ym, int stride_yn, int stride_xm, int stride_xk, int stride_we,
                         int stride_wk, int stride_wn, int stride_xsm, int stride_xsk, int stride_wse,
                         int stride_wsk, int stride_wsn) {
    (void)grid_n;
    (void)stride_xsk;
    (void)stride_wsk;
    expect(group_k == K, "group_k < K (per-K-group promotion) is not supported by this MoE kernel; "
                         "use group_k == K (per-token x per-channel scales)");
    expect(group_n >= 1, "group_n must be >= 1");
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
}

PYBIND11_MODULE(moe_op_gemm_a8w8_blockscale_tk, m) {
    m.def("moe_a8w8_blockscale", &moe_a8w8_blockscale,
          "MoE E4M3FN grouped GEMM with strided per-token / per-channel-group scales (group_k == K)", py::arg("X"),
          py::arg("W"), py::arg("Y"), py::arg("X_scale"), py::arg("W_scale"), py::arg("bias"), py::arg("GatherIndx"),
          py::arg("ExptHist"), py::arg("ExptOffs"), py::arg("ExptData"), py::arg("N"), py::arg("K"),
          py::arg("group_k"), py::arg("group_n"), py::arg("grid_m"), py::arg("grid_n"), py::arg("n_expts_act"),
          py::arg("stride_ym"), py::arg("stride_yn"), py::arg("stride_xm"), py::arg("stride_xk"),
          py::arg("stride_we"), py::arg("stride_wk"), py::arg("stride_wn"), py::arg("stride_xsm"),
          py::arg("stride_xsk"), py::arg("stride_wse"), py::arg("stride_wsk"), py::arg("stride_wsn"));
}
