// One allocation that Tensors view, held through its backend's Buffer (the reference's
// src/core/storage.hpp). Backends live for the whole program.
#pragma once

#include "backends/backend.hpp"
#include "mensurflow/device.hpp"

#include <cstddef>
#include <memory>

namespace mensurflow::detail {

struct Storage {
    Storage(Device device, std::size_t nbytes); // runtime_error if the device is unavailable
    Storage(const Storage&) = delete;
    Storage& operator=(const Storage&) = delete;

    std::byte* host_data() const; // nullptr for device-only memory
    void copy_from_host(std::size_t offset, const void* src, std::size_t bytes);
    void copy_to_host(void* dst, std::size_t offset, std::size_t bytes) const;
    Stream& stream() const;

    Device device;
    std::size_t nbytes;
    std::shared_ptr<Buffer> buffer;

  private:
    Backend* backend_;
};

} // namespace mensurflow::detail
