// moe_op_gemm_a8w8_tk -- the reference module of
// kernels/moe-gemm/moe_op_gemm_a8w8/kernel.cpp:244-271 (same function, argument
// names and order). X_scale: None, numel 1 (per tensor, the reference's) or T
// (per token); W_scale: None, numel E (per expert, the reference's) or E*N (per
// output channel). W may be K-contiguous ([E, N, K]) or the reference's
// N-contiguous [E, K, N] (read in place when K % 128 == 0, else copied
// K-major first). apply_swiglu / swiglu_alpha
// are accepted and, as in the reference, do not change the output.
#include "moe_bind.h"

using namespace hkqbind;

void moe_a8w8(py::object X, py::object W, py::object Y, py::object X_scale, py::object W_scale, py::object bias,
              py::object GatherIndx, py::object ExptHist, py::object ExptOffs, py::object ExptData, int N, int K,
              int grid_m, int grid_n, int n_expts_act, int stride_ym, int stride_yn, int stride_xm, int stride_xk,
              int stride_we, int stride_wk, int stride_wn, bool apply_swiglu, float swiglu_alpha) {
    (void)grid_n;
    (void)apply_swiglu;
    (void)swiglu_alpha;
    MoeScales sc;
    const int64_t T = view(X, "X").dim(0), E = view(ExptHist, "ExptHist").numel();
    if (!X_scale.is_none()) {
        auto v = view(X_scale, "X_scale");
        expect_dtype(v, "X_scale", {kF32});
        expect(v.numel() == 1 || (v.numel() == T && v.contiguous()), "X_scale must hold 1 (per tensor) or T (per token) values");
        sc.xs = (const float*)v.ptr;
        sc.xs_tok = v.numel() == 1 ? 0 : 1;
    }
    if (!W_scale.is_none()) {
        auto v = view(W_scale, "W_scale");
        expect_dtype(v, "W_scale", {kF32});
        expect(v.contiguous() && (v.numel() == E || v.numel() == E * N),
               "W_scale must hold E (per expert) or E*N (per channel) values");
        sc.ws = (const float*)v.ptr;
        if (v.numel() == E) { sc.ws_e = 1; sc.ws_n = 0; }
        else { sc.ws_e = N; sc.ws_n = 1; }
    }
    moe_call(X, W, Y, sc, bias, GatherIndx, ExptHist, ExptOffs, ExptData, N, K, grid_m, n_expts_act, stride_ym,
             stride_yn, stride_xm, stride_xk, stride_we, stride_wk, stride_wn);
}

PYBIND11_MODULE(moe_op_gemm_a8w8_tk, m) {
    m.def("moe_a8w8", &moe_a8w8, "MoE E4M3FN (A8W8) grouped GEMM over OGS routing metadata (gfx950 scaled MFMA)",
          py::arg("X"), py::arg("W"), py::arg("Y"), py::arg("X_scale"), py::arg("W_scale"), py::arg("bias"),
          py::arg("GatherIndx"), py::arg("ExptHist"), py::arg("ExptOffs"), py::arg("ExptData"), py::arg("N"),
          py::arg("K"), py::arg("grid_m"), py::arg("grid_n"), py::arg("n_expts_act"), py::arg("stride_ym"),
          py::arg("stride_yn"), py::arg("stride_xm"), py::arg("stride_xk"), py::arg("stride_we"),
          py::arg("stride_wk"), py::arg("stride_wn"), py::arg("apply_swiglu"), py::arg("swiglu_alpha"));
}
