// moe_op_mxfp4_tk -- the reference module of kernels/moe-gemm/moe_op_mxfp4/kernel.cpp:263-330
// (same function, argument names and order):
// moe_mxfp4(A, B, C, A_mx_scale, B_mx_scale, A_scale, B_scale, topk_weights,
//           sorted_token_ids, expert_ids, N, K, num_valid_tokens, top_k,
//           mul_routed_weight, stride_am, stride_ak, stride_be, stride_bk,
//           stride_bn, stride_cm, stride_cn, stride_amxm, stride_amxk,
//           stride_bmxe, stride_bmxk, stride_bmxn, grid_m, grid_n).
// Strides are in elements of each tensor (bytes for the uint8 ones). B and
// B_mx_scale may be K-contiguous (stride_bk == stride_bmxk == 1: B[e] is
// [N, K/2]) or the reference test's N-contiguous [E, K/2, N] / [E, K/32, N]
// (stride_bn == stride_bmxn == 1), which the kernels read in place
// (hkq_moe_mxfp4_kn) when K % 256 == 0 and the strides are multiples of 16,
// and which are otherwise copied K-major on the stream before the GEMM
// (hkq_moe_pack_kmajor). Every index the call can reach is checked against the
// tensors' sizes before the launch.
#include "bind_common.h"

using namespace hkqbind;

static int64_t extent(std::initializer_list<std::pair<int64_t, int64_t>> dims) {
    int64_t e = 1;
    for (auto& d : dims) {
        if (d.first <= 0) return 0;
        e += (d.first - 1) * d.second;
    }
    return e;
}

void moe_mxfp4(py::object A, py::object B, py::object C, py::object A_mx_scale, py::object B_mx_scale,
               py::object A_scale, py::object B_scale, py::object topk_weights, py::object sorted_token_ids,
               py::object expert_ids, int N, int K, int num_valid_tokens, int top_k, bool mul_routed_weight,
               int stride_am, int stride_ak, int stride_be, int stride_bk, int stride_bn, int stride_cm,
               int stride_cn, int stride_amxm, int stride_amxk, int stride_bmxe, int stride_bmxk, int stride_bmxn,
               int grid_m, int grid_n) {
    (void)grid_n;
    auto a = view(A, "A"), b = view(B, "B"), c = view(C, "C"), as = view(A_mx_scale, "A_mx_scale"),
         bs = view(B_mx_scale, "B_mx_scale"), ids = view(sorted_token_ids, "sorted_token_ids"),
         eids = view(expert_ids, "expert_ids");
    expect_dtype(a, "A", {kU8});
    expect_dtype(b, "B", {kU8});
    expect_dtype(as, "A_mx_scale", {kU8});
    expect_dtype(bs, "B_mx_scale", {kU8});
    expect_dtype(c, "C", {kBF16});
    expect_dtype(ids, "sorted_token_ids", {kI32});
    expect_dtype(eids, "expert_ids", {kI32});
    expect(stride_ak == 1 && stride_amxk == 1, "A and A_mx_scale must be K-contiguous (stride_ak == stride_amxk == 1)");
    const bool kmajor = stride_bk == 1 && stride_bmxk == 1;
    expect(kmajor || (stride_bn == 1 && stride_bmxn == 1),
           "B and B_mx_scale must both be K-contiguous (stride_bk == stride_bmxk == 1) or both N-contiguous "
           "(stride_bn == stride_bmxn == 1)");
    expect(stride_cn == 1, "C must be N-contiguous (stride_cn == 1)");
    expect(a.contiguous() && b.contiguous() && as.contiguous() && bs.contiguous() && c.contiguous() &&
               ids.contiguous() && eids.contiguous(),
           "all tensors must be contiguous");
    expect(N >= 0 && K > 0 && K % 128 == 0 && top_k > 0 && grid_m >= 0, "K must be a positive multiple of 128");
    const int64_t tokens = a.dim(0), E = b.dim(0);
    expect(a.numel() >= extent({{tokens, stride_am}, {K / 2, 1}}), "A is smaller than its strides say");
    expect(as.numel() >= extent({{tokens, stride_amxm}, {K / 32, 1}}), "A_mx_scale is smaller than its strides say");
    expect(b.numel() >= extent({{E, stride_be}, {N, stride_bn}, {K / 2, stride_bk}}), "B is smaller than its strides say");
    expect(bs.numel() >= extent({{E, stride_bmxe}, {N, stride_bmxn}, {K / 32, stride_bmxk}}),
           "B_mx_scale is smaller than its strides say");
    // N-contiguous weights and scales (tests/test_moe.py:909-925 of the
    // reference): read in place where the kernels can, else K-major copies
    // [E, N, K/2] and [E, N, K/32] for this call
    const bool in_place = !kmajor && K % 256 == 0 && stride_bk % 16 == 0 && stride_bmxk % 16 == 0 &&
                          stride_be % 16 == 0 && stride_bmxe % 16 == 0 && bs.ptr % 16 == 0 && b.ptr % 16 == 0;
    Workspace bp, bsp;
    uint64_t b_ptr = b.ptr, bs_ptr = bs.ptr;
    if (!kmajor && !in_place) {
        bp = pack_kmajor(B, b.ptr, E, K / 2, N, stride_be, stride_bk, "moe_mxfp4 weight prepack");
        bsp = pack_kmajor(B, bs.ptr, E, K / 32, N, stride_bmxe, stride_bmxk, "moe_mxfp4 scale prepack");
        b_ptr = (uint64_t)bp.ptr;
        bs_ptr = (uint64_t)bsp.ptr;
        stride_be = (K / 2) * N;
        stride_bn = K / 2;
        stride_bmxe = (K / 32) * N;
        stride_bmxn = K / 32;
    }
    expect(ids.numel() >= (int64_t)grid_m * 128, "sorted_token_ids must hold grid_m * 128 entries");
    expect(eids.numel() >= grid_m, "expert_ids must hold grid_m entries");
    expect(c.numel() >= extent({{num_valid_tokens, stride_cm}, {N, 1}}), "C must hold num_valid_tokens rows");
    const float *sa = nullptr, *sb = nullptr, *tw = nullptr;
    if (!A_scale.is_none()) {
        auto v = view(A_scale, "A_scale");
        expect_dtype(v, "A_scale", {kF32});
        expect(v.numel() >= 1, "A_scale must hold one value");
        sa = (const float*)v.ptr;
    }
    if (!B_scale.is_none()) {
        auto v = view(B_scale, "B_scale");
        expect_dtype(v, "B_scale", {kF32});
        expect(v.numel() >= E && v.contiguous(), "B_scale must hold one value per expert");
        sb = (const float*)v.ptr;
    }
    if (mul_routed_weight) {
        auto v = view(topk_weights, "topk_weights");
        expect_dtype(v, "topk_weights", {kF32});
        expect(v.numel() >= num_valid_tokens && v.contiguous(), "topk_weights must hold num_valid_tokens values");
        tw = (const float*)v.ptr;
    }
    auto fn = in_place ? hkq_moe_mxfp4_kn : hkq_moe_mxfp4;
    check(fn((const void*)a.ptr, (const void*)b_ptr, (void*)c.ptr, (const void*)as.ptr, (const void*)bs_ptr, sa, sb, tw,
             (const int32_t*)ids.ptr, (const int32_t*)eids.ptr, N, K, num_valid_tokens, top_k,
             mul_routed_weight ? 1 : 0, stride_am, stride_be, in_place ? stride_bk : stride_bn, stride_cm, stride_amxm,
             stride_bmxe, in_place ? stride_bmxk : stride_bmxn, tokens, E, grid_m, current_stream()),
          "moe_mxfp4");
}

PYBIND11_MODULE(moe_op_mxfp4_tk, m) {
    m.doc() = "MXFP4 MoE GEMM over block-sorted routing (gfx950 scaled MFMA)";
    m.def("moe_mxfp4", &moe_mxfp4, "MoE MXFP4 GEMM kernel", py::arg("A"), py::arg("B"), py::arg("C"),
          py::arg("A_mx_scale"), py::arg("B_mx_scale"), py::arg("A_scale"), py::arg("B_scale"),
          py::arg("topk_weights"), py::arg("sorted_token_ids"), py::arg("expert_ids"), py::arg("N"), py::arg("K"),
          py::arg("num_valid_tokens"), py::arg("top_k"), py::arg("mul_routed_weight"), py::arg("stride_am"),
          py::arg("stride_ak"), py::arg("stride_be"), py::arg("stride_bk"), py::arg("stride_bn"), py::arg("stride_cm"),
          py::arg("stride_cn"), py::arg("stride_amxm"), py::arg("stride_amxk"), py::arg("stride_bmxe"),
          py::arg("stride_bmxk"), py::arg("stride_bmxn"), py::arg("grid_m"), py::arg("grid_n"));
}
