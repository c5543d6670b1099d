// The backends of this process that found hardware, and the op table their kernels fill. The
// interface is mensurflow's (src/core/registry.hpp): a backend registers through
// register_<name>_backend and is kept only when it reports at least one device.
#pragma once

#include "backends/backend.hpp"
#include "core/dispatcher.hpp"

#include <array>
#include <memory>
#include <vector>

namespace mensurflow::detail {

class Registry {
  public:
    // Built on first use: the CPU backend (required), then every optional backend whose runtime
    // comes up.
    static Registry& instance();

    // The backend of this type, or nullptr when it is absent.
    Backend* find(DeviceType type) const;

    // The backend holding `device`; runtime_error("device rocm:1 is not available") otherwise.
    Backend& get(Device device) const;

    // Every usable device, CPU first, then in registration order.
    std::vector<Device> devices() const;

    Dispatcher& dispatcher() { return dispatcher_; }
    const Dispatcher& dispatcher() const { return dispatcher_; }

    // Called by a register_*_backend function. A backend without devices is dropped before it
    // registers anything; otherwise its kernels go into the op table and it is kept.
    void add(std::unique_ptr<Backend> backend);

  private:
    Registry();

    static constexpr std::size_t kDeviceTypes = 5; // DeviceType's enumerators
    std::array<std::unique_ptr<Backend>, kDeviceTypes> by_type_{};
    std::vector<DeviceType> arrival_; // types in the order they were added
    Dispatcher dispatcher_;
};

void register_cpu_backend(Registry& registry);
void register_rocm_backend(Registry& registry);

} // namespace mensurflow::detail
