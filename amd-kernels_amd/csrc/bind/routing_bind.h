// routing_bind.h -- argument checks shared by the MoE routing modules. The
// reference's routing bindings take raw data_ptr()s plus explicit sizes and
// strides; these modules take the same arguments and, before launching, check
// that every element the call will read or write lies inside the tensor passed
// (contiguous tensors, extent = numel), so a size/stride mismatch raises
// instead of touching memory past an allocation.
#pragma once
#include "bind_common.h"

namespace hkqbind {

inline const char* kU32 = "torch.uint32";

// Contiguous GPU tensor of one of the given dtypes holding at least `need` elements.
inline TensorView routing_tensor(const py::object& t, const char* name, std::initializer_list<const char*> dt,
                                 int64_t need) {
    auto v = view(t, name);
    expect_dtype(v, name, dt);
    expect(v.contiguous(), std::string(name) + " must be contiguous");
    expect(v.numel() >= need, std::string(name) + " holds " + std::to_string(v.numel()) + " elements; the call needs " +
                                  std::to_string(need));
    return v;
}

// 1 + the largest offset of a 2-D index space [n0, n1) x [0, n1) with strides s0, s1.
inline int64_t extent2(int64_t n0, int64_t s0, int64_t n1, int64_t s1) {
    if (n0 <= 0 || n1 <= 0) return 0;
    return (n0 - 1) * s0 + (n1 - 1) * s1 + 1;
}

}  // namespace hkqbind
