// Backend discovery and the device-choice policy built on it (behaviour of mensurflow's
// src/core/registry.cpp and src/core/device_selection.cpp, plus the ROCm backend).
#include "core/registry.hpp"

#include <algorithm>
#include <cstdlib>
#include <exception>
#include <stdexcept>
#include <string>

namespace mensurflow::detail {

namespace {

std::size_t slot_of(DeviceType type) { return static_cast<std::size_t>(type); }

struct BackendHook {
    void (*install)(Registry&);
    bool optional; // a failure leaves the backend out instead of failing the process
};

// The CPU must come up. A GPU backend whose driver, runtime or device is missing throws or reports
// zero devices; either way the library keeps running on the CPU.
constexpr BackendHook kHooks[] = {
    {register_cpu_backend, false},
    {register_rocm_backend, true},
};

} // namespace

Registry::Registry() {
    for (const BackendHook& hook : kHooks) {
        if (!hook.optional) {
            hook.install(*this);
            continue;
        }
        try {
            hook.install(*this);
        } catch (const std::exception&) {
            // left out: find() reports it absent
        }
    }
}

Registry& Registry::instance() {
    static Registry registry;
    return registry;
}

void Registry::add(std::unique_ptr<Backend> backend) {
    if (backend->device_count() < 1) {
        return;
    }
    const DeviceType type = backend->type();
    std::unique_ptr<Backend>& slot = by_type_.at(slot_of(type));
    if (slot != nullptr) {
        throw std::logic_error(std::string("backend registered twice: ") + device_type_name(type));
    }
    backend->register_kernels(dispatcher_);
    slot = std::move(backend);
    arrival_.push_back(type);
}

Backend* Registry::find(DeviceType type) const {
    const std::size_t slot = slot_of(type);
    return slot < by_type_.size() ? by_type_[slot].get() : nullptr;
}

Backend& Registry::get(Device device) const {
    if (Backend* backend = find(device.type)) {
        if (device.index >= 0 && device.index < backend->device_count()) {
            return *backend;
        }
    }
    throw std::runtime_error("device " + to_string(device) + " is not available");
}

std::vector<Device> Registry::devices() const {
    std::vector<Device> out;
    for (const DeviceType type : arrival_) {
        const int count = find(type)->device_count();
        for (int index = 0; index < count; ++index) {
            out.push_back(Device{type, index});
        }
    }
    return out;
}

} // namespace mensurflow::detail

namespace mensurflow {

std::vector<Device> list_devices() { return detail::Registry::instance().devices(); }

bool device_available(Device device) {
    const std::vector<Device> usable = list_devices();
    return std::find(usable.begin(), usable.end(), device) != usable.end();
}

Device default_device() {
    if (const char* forced = std::getenv("MENSURFLOW_DEVICE")) {
        const Device wanted = parse_device(forced);
        if (device_available(wanted)) {
            return wanted;
        }
        throw std::runtime_error("MENSURFLOW_DEVICE=" + std::string(forced) + " is not available");
    }
    // Accelerators before the CPU; ROCm sits with the vendor backends, before Vulkan.
    constexpr DeviceType kPreference[] = {DeviceType::CUDA, DeviceType::Metal, DeviceType::ROCm,
                                          DeviceType::Vulkan};
    for (const DeviceType type : kPreference) {
        if (device_available(Device{type, 0})) {
            return Device{type, 0};
        }
    }
    return Device{DeviceType::CPU, 0};
}

} // namespace mensurflow
