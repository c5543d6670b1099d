// Backend discovery, the default-device policy, and Storage (the reference's
// src/core/{registry,device_selection,storage}.cpp).
#include "core/registry.hpp"

#include "core/storage.hpp"

#include <cstdlib>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <vector>

namespace mensurflow::detail {

Registry::Registry() {
    register_cpu_backend(*this); // required: a failure here propagates
    // A GPU backend whose runtime or device is missing is skipped, not fatal.
    try {
        register_rocm_backend(*this);
    } catch (const std::exception&) {
    }
}

Registry& Registry::instance() {
    static Registry registry;
    return registry;
}

void Registry::add(std::unique_ptr<Backend> backend) {
    if (backend->device_count() <= 0) {
        return;
    }
    backend->register_kernels(dispatcher_);
    backends_.push_back(std::move(backend));
}

Backend* Registry::find(DeviceType type) const {
    for (const auto& backend : backends_) {
        if (backend->type() == type) {
            return backend.get();
        }
    }
    return nullptr;
}

Backend& Registry::get(Device device) const {
    Backend* backend = find(device.type);
    if (backend == nullptr || device.index < 0 || device.index >= backend->device_count()) {
        throw std::runtime_error("device " + to_string(device) + " is not available");
    }
    return *backend;
}

std::vector<Device> Registry::devices() const {
    std::vector<Device> out;
    for (const auto& backend : backends_) {
        for (int i = 0; i < backend->device_count(); ++i) {
            out.push_back({backend->type(), i});
        }
    }
    return out;
}

void Stream::copy_d2d(Buffer& dst, std::size_t dst_offset, const Buffer& src,
                      std::size_t src_offset, std::size_t bytes) {
    std::vector<std::byte> staged(bytes);
    copy_d2h(staged.data(), src, src_offset, bytes);
    copy_h2d(dst, dst_offset, staged.data(), bytes);
}

Storage::Storage(Device device, std::size_t nbytes)
    : device(device), nbytes(nbytes), backend_(&Registry::instance().get(device)) {
    buffer = backend_->allocate(device.index, nbytes);
}

std::byte* Storage::host_data() const { return static_cast<std::byte*>(buffer->host_ptr()); }

Stream& Storage::stream() const { return backend_->stream(device.index); }

void Storage::copy_from_host(std::size_t offset, const void* src, std::size_t bytes) {
    if (bytes == 0) {
        return;
    }
    if (offset > nbytes || bytes > nbytes - offset) {
        throw std::out_of_range("Storage::copy_from_host: range exceeds the allocation");
    }
    stream().copy_h2d(*buffer, offset, src, bytes);
}

void Storage::copy_to_host(void* dst, std::size_t offset, std::size_t bytes) const {
    if (bytes == 0) {
        return;
    }
    if (offset > nbytes || bytes > nbytes - offset) {
        throw std::out_of_range("Storage::copy_to_host: range exceeds the allocation");
    }
    stream().copy_d2h(dst, *buffer, offset, bytes);
}

} // namespace mensurflow::detail

namespace mensurflow {

std::vector<Device> list_devices() { return detail::Registry::instance().devices(); }

bool device_available(Device device) {
    for (Device d : list_devices()) {
        if (d == device) {
            return true;
        }
    }
    return false;
}

Device default_device() {
    if (const char* env = std::getenv("MENSURFLOW_DEVICE")) {
        const Device wanted = parse_device(env);
        if (!device_available(wanted)) {
            throw std::runtime_error("MENSURFLOW_DEVICE=" + std::string(env) + " is not available");
        }
        return wanted;
    }
    for (DeviceType type :
         {DeviceType::CUDA, DeviceType::Metal, DeviceType::ROCm, DeviceType::Vulkan}) {
        if (device_available({type, 0})) {
            return {type, 0};
        }
    }
    return {DeviceType::CPU, 0};
}

} // namespace mensurflow
