// What a backend provides to mensurflow's core (the classes of src/backends/backend.hpp): memory
// (Buffer), an in-order queue with host transfers (Stream), and the device family itself
// (Backend). The ROCm backend implements them on top of include/mfr_rocm.h, so no vendor header
// is visible above this line.
#pragma once

#include "mensurflow/device.hpp"

#include <cstddef>
#include <memory>
#include <string>
#include <vector>

namespace mensurflow::detail {

class Dispatcher;

class Buffer {
  public:
    virtual ~Buffer() = default;
    virtual std::size_t size() const = 0;
    // The backend's handle for the memory (a device address on CPU and ROCm); null when size() is
    // 0. Only the owning backend's kernels interpret it.
    virtual void* native() const = 0;
    // Memory the host can address directly, else nullptr.
    virtual void* host_ptr() const { return nullptr; }
};

class Stream {
  public:
    virtual ~Stream() = default;
    // Transfers that are finished on return (the source may be reused, the destination read).
    // copy_d2h first waits for what is already queued.
    virtual void copy_h2d(Buffer& dst, std::size_t offset, const void* src, std::size_t bytes) = 0;
    virtual void copy_d2h(void* dst, const Buffer& src, std::size_t offset, std::size_t bytes) = 0;
    // Returns once everything queued has finished.
    virtual void synchronize() = 0;
    // Bytes from one buffer of this stream's device to another, in queue order. An addition of
    // this backend's integration (device-side Tensor::copy_from); a backend without a native copy
    // gets this host round trip.
    virtual void copy_d2d(Buffer& dst, std::size_t dst_offset, const Buffer& src,
                          std::size_t src_offset, std::size_t bytes) {
        std::vector<std::byte> bounce(bytes);
        copy_d2h(bounce.data(), src, src_offset, bytes);
        copy_h2d(dst, dst_offset, bounce.data(), bytes);
    }
};

struct DeviceInfo {
    std::string name;
    std::size_t memory_bytes = 0; // 0 when the runtime does not say
};

class Backend {
  public:
    virtual ~Backend() = default;
    virtual DeviceType type() const = 0;
    // Devices of this type that can be used; 0 (never an exception) when the hardware or its
    // runtime is missing, so the registry can drop the backend.
    virtual int device_count() const = 0;
    virtual DeviceInfo info(int index) const = 0;
    virtual std::shared_ptr<Buffer> allocate(int index, std::size_t bytes) = 0;
    // The queue every kernel of device `index` runs on.
    virtual Stream& stream(int index) = 0;
    virtual void register_kernels(Dispatcher& dispatcher) = 0;
};

} // namespace mensurflow::detail
