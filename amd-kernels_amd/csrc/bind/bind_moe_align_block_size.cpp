// moe_align_block_size_tk -- the reference module of
// kernels/moe-routing/moe_align_block_size/kernel.cpp:201-241:
// moe_align_block_size(topk_ids, sorted_token_ids, expert_ids,
// tokens_cnts_buffer, cumsum_buffer, total_tokens_post_pad, num_experts,
// block_size, numel). int32 tensors. sorted_token_ids / expert_ids must hold
// the padded total (a device value; at most numel + E * (block_size - 1)
// entries and that many / block_size blocks): they are only checked to be
// non-empty here.
#include "routing_bind.h"

using namespace hkqbind;

void moe_align_block_size(py::object topk_ids, py::object sorted_token_ids, py::object expert_ids,
                          py::object tokens_cnts_buffer, py::object cumsum_buffer, py::object total_tokens_post_pad,
                          int64_t num_experts, int64_t block_size, int64_t numel) {
    expect(num_experts >= 1 && block_size >= 1 && numel >= 0, "num_experts >= 1, block_size >= 1, numel >= 0");
    auto ids = routing_tensor(topk_ids, "topk_ids", {kI32}, numel);
    auto s = routing_tensor(sorted_token_ids, "sorted_token_ids", {kI32}, numel ? 1 : 0);
    auto e = routing_tensor(expert_ids, "expert_ids", {kI32}, numel ? 1 : 0);
    auto c = routing_tensor(tokens_cnts_buffer, "tokens_cnts_buffer", {kI32}, (num_experts + 1) * num_experts);
    auto cs = routing_tensor(cumsum_buffer, "cumsum_buffer", {kI32}, num_experts + 1);
    auto t = routing_tensor(total_tokens_post_pad, "total_tokens_post_pad", {kI32}, 1);
    check(hkq_moe_align_block_size((const int32_t*)ids.ptr, (int32_t*)s.ptr, (int32_t*)e.ptr, (int32_t*)c.ptr,
                                   (int32_t*)cs.ptr, (int32_t*)t.ptr, num_experts, block_size, numel,
                                   current_stream()),
          "moe_align_block_size");
}

PYBIND11_MODULE(moe_align_block_size_tk, m) {
    m.doc() = "Block-padded, expert-sorted token order for MoE GEMMs (gfx950)";
    m.def("moe_align_block_size", &moe_align_block_size, "MoE align block size", py::arg("topk_ids"),
          py::arg("sorted_token_ids"), py::arg("expert_ids"), py::arg("tokens_cnts_buffer"), py::arg("cumsum_buffer"),
          py::arg("total_tokens_post_pad"), py::arg("num_experts"), py::arg("block_size"), py::arg("numel"));
}
