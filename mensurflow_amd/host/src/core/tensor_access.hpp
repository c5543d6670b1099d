// Backend-side access to a Tensor's memory, outside Tensor's public surface (the helper
// mensurflow's core gives kernels, src/core/tensor_access.hpp). `data<T>` is the element address
// for backends whose Buffer::native() is a plain address; T is the element type, so the offset
// is counted in sizeof(T) steps.
#pragma once

#include "core/storage.hpp"
#include "mensurflow/tensor.hpp"

namespace mensurflow::detail {

struct TensorAccess {
    static Buffer& buffer(const Tensor& t) { return *t.storage_->buffer; }
    static Storage& storage(const Tensor& t) { return *t.storage_; }

    template <typename T> static T* data(const Tensor& t) {
        std::byte* const first = static_cast<std::byte*>(buffer(t).native()) +
                                 static_cast<std::size_t>(t.offset()) * sizeof(T);
        return reinterpret_cast<T*>(first);
    }
};

} // namespace mensurflow::detail
