// moe_routing_tk -- the gate placement of kernels/moe-routing/moe_routing/kernel.cpp:209-306,
// which the reference compiles without a Python binding; the module exposes its
// two launchers with their argument order:
// routing_compute_indx(GatherIndx, ScatterIndx, GateScal, ExptScal, ExptIndx,
// PartialOffs, stride_pm, stride_pn, TokensStart, n_gates, N_EXPTS_ACT) and
// routing_compute_indx_fused(GatherIndx, ScatterIndx, GateScal, ExptScal,
// ExptIndx, TokensStart, n_gates, N_EXPTS_ACT). int32 index tensors, bf16
// GateScal / ExptScal (both None: skipped). GatherIndx / GateScal are indexed
// by device-computed positions; they must hold every gate (n_gates entries).
#include "routing_bind.h"

using namespace hkqbind;

static void run(py::object GatherIndx, py::object ScatterIndx, py::object GateScal, py::object ExptScal,
                py::object ExptIndx, py::object PartialOffs, int64_t stride_pm, int64_t stride_pn,
                py::object TokensStart, int64_t n_gates, int N_EXPTS_ACT) {
    expect(n_gates >= 0 && N_EXPTS_ACT >= 1, "n_gates >= 0 and N_EXPTS_ACT >= 1 are required");
    auto g = routing_tensor(GatherIndx, "GatherIndx", {kI32}, n_gates);
    auto s = routing_tensor(ScatterIndx, "ScatterIndx", {kI32}, n_gates);
    auto x = routing_tensor(ExptIndx, "ExptIndx", {kI32}, n_gates);
    auto ts = routing_tensor(TokensStart, "TokensStart", {kI32}, 1);
    expect(GateScal.is_none() == ExptScal.is_none(), "GateScal and ExptScal must both be given or both be None");
    void* gs = nullptr;
    const void* es = nullptr;
    if (!GateScal.is_none()) {
        gs = (void*)routing_tensor(GateScal, "GateScal", {kBF16}, n_gates).ptr;
        es = (const void*)routing_tensor(ExptScal, "ExptScal", {kBF16}, n_gates).ptr;
    }
    if (PartialOffs.is_none()) {
        check(hkq_routing_compute_indx_fused((int32_t*)g.ptr, (int32_t*)s.ptr, gs, es, (const int32_t*)x.ptr,
                                             (const int32_t*)ts.ptr, n_gates, N_EXPTS_ACT, current_stream()),
              "routing_compute_indx_fused");
        return;
    }
    auto po = routing_tensor(PartialOffs, "PartialOffs", {kI32, kU32}, 1);
    check(hkq_routing_compute_indx((int32_t*)g.ptr, (int32_t*)s.ptr, gs, es, (const int32_t*)x.ptr,
                                   (const int32_t*)po.ptr, stride_pm, stride_pn, (const int32_t*)ts.ptr, n_gates,
                                   N_EXPTS_ACT, current_stream()),
          "routing_compute_indx");
}

void routing_compute_indx(py::object GatherIndx, py::object ScatterIndx, py::object GateScal, py::object ExptScal,
                          py::object ExptIndx, py::object PartialOffs, int64_t stride_pm, int64_t stride_pn,
                          py::object TokensStart, int64_t n_gates, int N_EXPTS_ACT) {
    expect(!PartialOffs.is_none(), "PartialOffs is required (routing_compute_indx_fused works without it)");
    run(GatherIndx, ScatterIndx, GateScal, ExptScal, ExptIndx, PartialOffs, stride_pm, stride_pn, TokensStart,
        n_gates, N_EXPTS_ACT);
}

void routing_compute_indx_fused(py::object GatherIndx, py::object ScatterIndx, py::object GateScal,
                                py::object ExptScal, py::object ExptIndx, py::object TokensStart, int64_t n_gates,
                                int N_EXPTS_ACT) {
    run(GatherIndx, ScatterIndx, GateScal, ExptScal, ExptIndx, py::none(), 0, 0, TokensStart, n_gates, N_EXPTS_ACT);
}

PYBIND11_MODULE(moe_routing_tk, m) {
    m.doc() = "MoE gate placement: gather/scatter indices and gate scales in expert-sorted order (gfx950)";
    m.def("routing_compute_indx", &routing_compute_indx, "Gate placement with per-block partial offsets",
          py::arg("GatherIndx"), py::arg("ScatterIndx"), py::arg("GateScal"), py::arg("ExptScal"), py::arg("ExptIndx"),
          py::arg("PartialOffs"), py::arg("stride_pm"), py::arg("stride_pn"), py::arg("TokensStart"),
          py::arg("n_gates"), py::arg("N_EXPTS_ACT"));
    m.def("routing_compute_indx_fused", &routing_compute_indx_fused, "Gate placement counted in one workgroup",
          py::arg("GatherIndx"), py::arg("ScatterIndx"), py::arg("GateScal"), py::arg("ExptScal"), py::arg("ExptIndx"),
          py::arg("TokensStart"), py::arg("n_gates"), py::arg("N_EXPTS_ACT"));
}
