// Backends with usable hardware, plus the op table they filled (the reference's
// src/core/registry.hpp). The CPU backend is always present; the ROCm backend is added when
// its runtime finds a gfx950 device and dropped silently otherwise.
#pragma once

#include "backends/backend.hpp"
#include "core/dispatcher.hpp"

#include <memory>
#include <vector>

namespace mensurflow::detail {

class Registry {
  public:
    static Registry& instance();
    Backend* find(DeviceType type) const;  // nullptr when absent
    Backend& get(Device device) const;     // runtime_error("device rocm:1 is not available")
    std::vector<Device> devices() const;   // CPU first
    Dispatcher& dispatcher() { return dispatcher_; }
    const Dispatcher& dispatcher() const { return dispatcher_; }
    // Keeps the backend (and registers its kernels) only when it has a device.
    void add(std::unique_ptr<Backend> backend);

  private:
    Registry();
    std::vector<std::unique_ptr<Backend>> backends_;
    Dispatcher dispatcher_;
};

void register_cpu_backend(Registry& registry);
void register_rocm_backend(Registry& registry);

} // namespace mensurflow::detail
