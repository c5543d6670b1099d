// Kernel-side access to a Tensor's buffer (the reference's src/core/tensor_access.hpp).
#pragma once

#include "core/storage.hpp"
#include "mensurflow/tensor.hpp"

namespace mensurflow::detail {

struct TensorAccess {
    static Buffer& buffer(const Tensor& t) { return *t.storage_->buffer; }
    static Storage& storage(const Tensor& t) { return *t.storage_; }

    // Address of the tensor's first element, for backends whose native() is an address.
    template <typename T> static T* data(const Tensor& t) {
        auto* base = static_cast<std::byte*>(buffer(t).native());
        return reinterpret_cast<T*>(base + static_cast<std::size_t>(t.offset()) * t.itemsize());
    }
};

} // namespace mensurflow::detail
