// moe_expt_data_tk -- the reference module of kernels/moe-routing/moe_expt_data/kernel.cpp:219-325:
// expt_data_stage1(Hist, TokenStart, TileStart, MDTileInfo, n_expts_tot,
// max_num_tiles, n_gates, tile_dim_log2), expt_data_stage2(Hist, TileStart,
// TileInfo, n_expts_tot, tile_dim_log2), expt_data_stage2_fused(Hist,
// TileStart, TileInfo, n_expts_tot) and expt_data_compute(..., use_fused_stage2).
// int32 tensors; MDTileInfo / TileInfo int32 or uint32.
#include "routing_bind.h"

using namespace hkqbind;

void expt_data_stage1(py::object Hist, py::object TokenStart, py::object TileStart, py::object MDTileInfo,
                      int64_t n_expts_tot, int64_t max_num_tiles, int64_t n_gates, int tile_dim_log2) {
    expect(n_expts_tot >= 1 && max_num_tiles >= 0, "n_expts_tot >= 1 and max_num_tiles >= 0 are required");
    auto h = routing_tensor(Hist, "Hist", {kI32}, n_expts_tot);
    auto ts = routing_tensor(TokenStart, "TokenStart", {kI32}, n_expts_tot + 1);
    auto tl = routing_tensor(TileStart, "TileStart", {kI32}, n_expts_tot + 1);
    auto md = routing_tensor(MDTileInfo, "MDTileInfo", {kI32, kU32}, max_num_tiles);
    check(hkq_expt_data_stage1((const int32_t*)h.ptr, (int32_t*)ts.ptr, (int32_t*)tl.ptr, (uint32_t*)md.ptr,
                               n_expts_tot, max_num_tiles, n_gates, tile_dim_log2, current_stream()),
          "expt_data_stage1");
}

// Stage 2 writes up to TileStart[E] tiles, a device value: TileInfo is only
// checked to be non-empty here.
void expt_data_stage2(py::object Hist, py::object TileStart, py::object TileInfo, int64_t n_expts_tot,
                      int tile_dim_log2) {
    expect(n_expts_tot >= 1, "n_expts_tot >= 1 is required");
    auto h = routing_tensor(Hist, "Hist", {kI32}, n_expts_tot);
    auto tl = routing_tensor(TileStart, "TileStart", {kI32}, n_expts_tot);
    auto md = routing_tensor(TileInfo, "TileInfo", {kI32, kU32}, 1);
    check(hkq_expt_data_stage2((const int32_t*)h.ptr, (const int32_t*)tl.ptr, (uint32_t*)md.ptr, n_expts_tot,
                               tile_dim_log2, current_stream()),
          "expt_data_stage2");
}

void expt_data_stage2_fused(py::object Hist, py::object TileStart, py::object TileInfo, int64_t n_expts_tot) {
    expect(n_expts_tot >= 1, "n_expts_tot >= 1 is required");
    auto h = routing_tensor(Hist, "Hist", {kI32}, n_expts_tot);
    auto tl = routing_tensor(TileStart, "TileStart", {kI32}, n_expts_tot);
    auto md = routing_tensor(TileInfo, "TileInfo", {kI32, kU32}, 1);
    check(hkq_expt_data_stage2_fused((const int32_t*)h.ptr, (const int32_t*)tl.ptr, (uint32_t*)md.ptr, n_expts_tot,
                                     current_stream()),
          "expt_data_stage2_fused");
}

void expt_data_compute(py::object Hist, py::object TokenStart, py::object TileStart, py::object MDTileInfo,
                       int64_t n_expts_tot, int64_t max_num_tiles, int64_t n_gates, int tile_dim_log2,
                       bool use_fused_stage2) {
    expect(n_expts_tot >= 1 && max_num_tiles >= 0, "n_expts_tot >= 1 and max_num_tiles >= 0 are required");
    auto h = routing_tensor(Hist, "Hist", {kI32}, n_expts_tot);
    auto ts = routing_tensor(TokenStart, "TokenStart", {kI32}, n_expts_tot + 1);
    auto tl = routing_tensor(TileStart, "TileStart", {kI32}, n_expts_tot + 1);
    auto md = routing_tensor(MDTileInfo, "MDTileInfo", {kI32, kU32}, max_num_tiles);
    check(hkq_expt_data_compute((const int32_t*)h.ptr, (int32_t*)ts.ptr, (int32_t*)tl.ptr, (uint32_t*)md.ptr,
                                n_expts_tot, max_num_tiles, n_gates, tile_dim_log2, use_fused_stage2 ? 1 : 0,
                                current_stream()),
          "expt_data_compute");
}

PYBIND11_MODULE(moe_expt_data_tk, m) {
    m.doc() = "OGS expert data: token/tile starts and per-tile (expert, block) metadata (gfx950)";
    m.def("expt_data_stage1", &expt_data_stage1, "Token and tile starts; 0xFFFFFFFF past the last tile",
          py::arg("Hist"), py::arg("TokenStart"), py::arg("TileStart"), py::arg("MDTileInfo"), py::arg("n_expts_tot"),
          py::arg("max_num_tiles"), py::arg("n_gates"), py::arg("tile_dim_log2"));
    m.def("expt_data_stage2", &expt_data_stage2, "Per-tile expert | block << 16", py::arg("Hist"),
          py::arg("TileStart"), py::arg("TileInfo"), py::arg("n_expts_tot"), py::arg("tile_dim_log2"));
    m.def("expt_data_stage2_fused", &expt_data_stage2_fused, "First tile of each expert", py::arg("Hist"),
          py::arg("TileStart"), py::arg("TileInfo"), py::arg("n_expts_tot"));
    m.def("expt_data_compute", &expt_data_compute, "Both stages", py::arg("Hist"), py::arg("TokenStart"),
          py::arg("TileStart"), py::arg("MDTileInfo"), py::arg("n_expts_tot"), py::arg("max_num_tiles"),
          py::arg("n_gates"), py::arg("tile_dim_log2"), py::arg("use_fused_stage2"));
}
