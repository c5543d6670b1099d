// The interface every backend implements (the reference's src/backends/backend.hpp:16-68): one
// allocation (Buffer), an ordered queue with host transfers (Stream), and the backend itself.
// Nothing above the dispatcher includes a vendor header; the ROCm backend reaches HIP only
// through the C ABI of include/mfr_rocm.h.
#pragma once

#include "mensurflow/device.hpp"

#include <cstddef>
#include <memory>
#include <string>

namespace mensurflow::detail {

class Dispatcher;

class Buffer {
  public:
    virtual ~Buffer() = default;
    virtual std::size_t size() const = 0;
    // The backend's handle (a device address for CPU and ROCm); null for a zero-byte buffer.
    virtual void* native() const = 0;
    // Host-addressable memory, or nullptr for device-only memory.
    virtual void* host_ptr() const { return nullptr; }
};

class Stream {
  public:
    virtual ~Stream() = default;
    // Complete on return: src may be reused. d2h also waits for earlier work on the stream.
    virtual void copy_h2d(Buffer& dst, std::size_t offset, const void* src, std::size_t bytes) = 0;
    virtual void copy_d2h(void* dst, const Buffer& src, std::size_t offset, std::size_t bytes) = 0;
    virtual void synchronize() = 0;
    // A copy between two buffers of this stream's device, ordered with its other work. Added for
    // device-resident Tensor::copy_from; the default stages the bytes through host memory.
    virtual void copy_d2d(Buffer& dst, std::size_t dst_offset, const Buffer& src,
                          std::size_t src_offset, std::size_t bytes);
};

struct DeviceInfo {
    std::string name;
    std::size_t memory_bytes = 0;
};

class Backend {
  public:
    virtual ~Backend() = default;
    virtual DeviceType type() const = 0;
    // 0 when the backend is built in but finds no hardware; must not throw.
    virtual int device_count() const = 0;
    virtual DeviceInfo info(int index) const = 0;
    virtual std::shared_ptr<Buffer> allocate(int index, std::size_t bytes) = 0;
    // The stream kernels for this device run on (one per device).
    virtual Stream& stream(int index) = 0;
    virtual void register_kernels(Dispatcher& dispatcher) = 0;
};

} // namespace mensurflow::detail
