// Storage: allocation through the device's backend, bounds-checked host transfers.
#include "core/storage.hpp"

#include "core/registry.hpp"

#include <stdexcept>
#include <string>

namespace mensurflow::detail {

namespace {

void require_inside(std::size_t offset, std::size_t bytes, std::size_t capacity, const char* who) {
    const bool inside = offset <= capacity && bytes <= capacity - offset;
    if (!inside) {
        throw std::out_of_range(std::string(who) + ": range exceeds the allocation");
    }
}

} // namespace

Storage::Storage(Device where, std::size_t size)
    : device(where), nbytes(size), backend_(&Registry::instance().get(where)) {
    buffer = backend_->allocate(where.index, size);
}

std::byte* Storage::host_data() const { return static_cast<std::byte*>(buffer->host_ptr()); }

Stream& Storage::stream() const { return backend_->stream(device.index); }

void Storage::copy_from_host(std::size_t offset, const void* src, std::size_t bytes) {
    if (bytes > 0) {
        require_inside(offset, bytes, nbytes, "Storage::copy_from_host");
        stream().copy_h2d(*buffer, offset, src, bytes);
    }
}

void Storage::copy_to_host(void* dst, std::size_t offset, std::size_t bytes) const {
    if (bytes > 0) {
        require_inside(offset, bytes, nbytes, "Storage::copy_to_host");
        stream().copy_d2h(dst, *buffer, offset, bytes);
    }
}

} // namespace mensurflow::detail
