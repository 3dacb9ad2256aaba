// bind_common.h -- shared helpers of the hipkittens-compatible pybind11
// modules. Tensors are read by duck typing (data_ptr(), shape, stride(),
// dtype, is_cuda), as the reference bindings do, so the modules do not link
// libtorch; every call forwards to the C ABI of libhkq.so.
#pragma once
#include <pybind11/pybind11.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "hkq.h"

namespace py = pybind11;

namespace hkqbind {

struct TensorView {
    uint64_t ptr = 0;
    std::vector<int64_t> shape, stride;
    std::string dtype;  // e.g. "torch.bfloat16"
    int64_t dim(int i) const { return shape.at(i < 0 ? shape.size() + i : i); }
    int64_t numel() const {
        int64_t n = 1;
        for (auto s : shape) n *= s;
        return n;
    }
    bool contiguous() const {
        int64_t expect = 1;
        for (int i = (int)shape.size() - 1; i >= 0; --i) {
            if (shape[i] != 1 && stride[i] != expect) return false;
            expect *= shape[i];
        }
        return true;
    }
};

inline TensorView view(const py::object& t, const char* name) {
    if (t.is_none()) throw py::type_error(std::string(name) + " must be a tensor, got None");
    if (!py::hasattr(t, "data_ptr")) throw py::type_error(std::string(name) + " must be a torch tensor");
    if (py::hasattr(t, "is_cuda") && !t.attr("is_cuda").cast<bool>())
        throw py::value_error(std::string(name) + " must be a GPU tensor");
    TensorView v;
    v.ptr = t.attr("data_ptr")().cast<uint64_t>();
    for (auto s : t.attr("shape").cast<py::tuple>()) v.shape.push_back(s.cast<int64_t>());
    for (auto s : t.attr("stride")().cast<py::tuple>()) v.stride.push_back(s.cast<int64_t>());
    v.dtype = py::str(t.attr("dtype")).cast<std::string>();
    return v;
}

inline void expect_dtype(const TensorView& v, const char* name, std::initializer_list<const char*> ok) {
    for (auto d : ok)
        if (v.dtype == d) return;
    std::string msg = std::string(name) + " has dtype " + v.dtype + "; expected one of:";
    for (auto d : ok) msg += std::string(" ") + d;
    throw py::type_error(msg);
}

inline void expect(bool cond, const std::string& msg) {
    if (!cond) throw py::value_error(msg);
}

// Row stride (elements) of a 2-D view whose last dim is contiguous.
inline int64_t row_stride(const TensorView& v, const char* name) {
    expect(v.shape.size() == 2, std::string(name) + " must be 2-D");
    expect(v.stride[1] == 1 || v.shape[1] == 1, std::string(name) + " must have a contiguous last dimension");
    return v.shape[0] <= 1 ? std::max<int64_t>(v.shape[1], v.stride[0]) : v.stride[0];
}

// torch's current stream when torch is loaded (the null stream by default, which
// is the stream the reference launches on), else the null stream.
inline hkq_stream_t current_stream() {
    static py::object cur;
    if (!cur) {
        py::dict mods = py::module_::import("sys").attr("modules");
        if (!mods.contains("torch")) return nullptr;
        cur = py::module_::import("torch").attr("cuda").attr("current_stream");
    }
    uint64_t s = cur().attr("cuda_stream").cast<uint64_t>();
    return reinterpret_cast<hkq_stream_t>(s);
}

// Device workspace of `bytes` bytes from torch's caching allocator on the
// device of `like`, alive while the returned object is (the allocator hands the
// memory out again only in the order of the work queued on the current stream,
// which is where the launch goes). Without torch loaded there is no workspace
// and the library runs the plan that needs none.
struct Workspace {
    py::object keep;
    void* ptr = nullptr;
    size_t bytes = 0;
};
inline Workspace workspace(size_t bytes, py::object like) {
    Workspace w;
    if (bytes == 0) return w;
    py::dict mods = py::module_::import("sys").attr("modules");
    if (!mods.contains("torch")) return w;
    py::object torch = py::module_::import("torch");
    w.keep = torch.attr("empty")(py::make_tuple(bytes), py::arg("dtype") = torch.attr("uint8"),
                                 py::arg("device") = like.attr("device"));
    w.ptr = reinterpret_cast<void*>(w.keep.attr("data_ptr")().cast<uint64_t>());
    w.bytes = bytes;
    return w;
}

inline void check(int rc, const char* what) {
    if (rc != 0) throw std::runtime_error(std::string(what) + ": " + hkq_last_error() + " (code " + std::to_string(rc) + ")");
}

// The K-contiguous copy [E, N, R] (strides R*N, R, 1) of E byte planes [R, N]
// (plane e at src + e*src_e, row r at + r*src_r, N contiguous), made on the
// current stream in a torch temporary that lives as long as the result:
// how the MoE modules take the reference's N-contiguous weights.
inline Workspace pack_kmajor(py::object like, uint64_t src, int64_t E, int64_t R, int64_t N, int64_t src_e,
                             int64_t src_r, const char* what) {
    Workspace w = workspace((size_t)(E * R * N), like);
    if (E * R * N > 0 && w.ptr == nullptr)
        throw py::value_error(std::string(what) + ": N-contiguous weights need torch for the K-major copy");
    check(hkq_moe_pack_kmajor((const void*)src, w.ptr, E, R, N, src_e, src_r, R * N, R, current_stream()), what);
    return w;
}

inline const char* kBF16 = "torch.bfloat16";
inline const char* kF32 = "torch.float32";
inline const char* kFP8 = "torch.float8_e4m3fn";
inline const char* kU8 = "torch.uint8";
inline const char* kI8 = "torch.int8";
inline const char* kI32 = "torch.int32";

}  // namespace hkqbind
