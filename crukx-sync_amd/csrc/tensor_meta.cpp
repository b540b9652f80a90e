// Batched tensor metadata for the Python layer (crukx_sync/codec.py): one call reads, for every tensor
// of a list, what the codec's entry points need (device address, element count, device, dtype and
// contiguity, version counter), in place of several Python attribute reads per tensor (for the 339
// tensors of a 7B state dict, about 0.15 ms per list).  Built as a torch C++ extension by the
// repository's build step (it reads at::Tensor fields); nothing here touches tensor data.
#include <torch/extension.h>

#include <cstdint>
#include <vector>

namespace {

// Per tensor: address, element count, device index (-1 off the GPU), flags (bit 0: bf16 or int16,
// bit 1: contiguous) and version counter, as five packed arrays (u64, u64, i32, i32, u64).
py::tuple meta(const std::vector<at::Tensor> &ts) {
    const size_t n = ts.size();
    std::vector<uint64_t> ptr(n), numel(n), ver(n);
    std::vector<int32_t> dev(n), flags(n);
    for (size_t i = 0; i < n; ++i) {
        const at::Tensor &t = ts[i];
        ptr[i] = (uint64_t)(uintptr_t)t.data_ptr();
        numel[i] = (uint64_t)t.numel();
        dev[i] = t.device().is_cuda() ? (int32_t)t.device().index() : -1;
        const auto st = t.scalar_type();
        flags[i] = ((st == at::kBFloat16 || st == at::kShort) ? 1 : 0) | (t.is_contiguous() ? 2 : 0);
        ver[i] = (uint64_t)t._version();
    }
    return py::make_tuple(py::bytes(reinterpret_cast<const char *>(ptr.data()), 8 * n),
                          py::bytes(reinterpret_cast<const char *>(numel.data()), 8 * n),
                          py::bytes(reinterpret_cast<const char *>(dev.data()), 4 * n),
                          py::bytes(reinterpret_cast<const char *>(flags.data()), 4 * n),
                          py::bytes(reinterpret_cast<const char *>(ver.data()), 8 * n));
}

// Whether a[i] and b[i] have the same shape, for every i (the lists have equal length).
bool same_shapes(const std::vector<at::Tensor> &a, const std::vector<at::Tensor> &b) {
    if (a.size() != b.size()) return false;
    for (size_t i = 0; i < a.size(); ++i)
        if (a[i].sizes() != b[i].sizes()) return false;
    return true;
}

// The encoder's inputs in one call: meta() of both lists and whether their shapes agree pairwise (each
// list is converted from Python once instead of twice).
py::tuple meta_pair(const std::vector<at::Tensor> &a, const std::vector<at::Tensor> &b) {
    return py::make_tuple(meta(a), meta(b), same_shapes(a, b));
}

// Version counters only (after an in-place write), as packed u64.
py::bytes versions(const std::vector<at::Tensor> &ts) {
    std::vector<uint64_t> ver(ts.size());
    for (size_t i = 0; i < ts.size(); ++i) ver[i] = (uint64_t)ts[i]._version();
    return py::bytes(reinterpret_cast<const char *>(ver.data()), 8 * ver.size());
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("meta", &meta, "address, numel, device, flags, version of every tensor of a list");
    m.def("same_shapes", &same_shapes, "whether two lists of tensors agree in shape pairwise");
    m.def("meta_pair", &meta_pair, "meta of two lists and whether their shapes agree pairwise");
    m.def("versions", &versions, "version counters of a list of tensors");
}
