// The allocation behind one or more Tensors: a backend Buffer plus the device it lives on. The
// members and calls are those mensurflow's core defines (src/core/storage.hpp); `stream()` is an
// addition that device-side copies use. Backends outlive every Storage.
#pragma once

#include "backends/backend.hpp"
#include "mensurflow/device.hpp"

#include <cstddef>
#include <memory>

namespace mensurflow::detail {

struct Storage {
    // runtime_error when `device` is not available.
    Storage(Device device, std::size_t nbytes);
    Storage(const Storage&) = delete;
    Storage& operator=(const Storage&) = delete;

    // Host-addressable bytes, or nullptr for device-only (or empty) memory.
    std::byte* host_data() const;

    // Byte ranges in and out of the allocation, finished on return; the read also waits for work
    // already queued on the device. out_of_range for a range past the end.
    void copy_from_host(std::size_t offset, const void* src, std::size_t bytes);
    void copy_to_host(void* dst, std::size_t offset, std::size_t bytes) const;

    // The queue the device's kernels and copies run on.
    Stream& stream() const;

    Device device;
    std::size_t nbytes;
    std::shared_ptr<Buffer> buffer;

  private:
    Backend* backend_;
};

} // namespace mensurflow::detail
