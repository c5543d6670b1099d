// Where a Tensor's memory lives and where an op runs. Mirrors include/mensurflow/device.hpp of
// the reference, with one addition: DeviceType::ROCm ("rocm"), the MI355X backend.
#pragma once

#include <string>
#include <string_view>
#include <vector>

namespace mensurflow {

enum class DeviceType { CPU, CUDA, Metal, Vulkan, ROCm };

struct Device {
    DeviceType type = DeviceType::CPU;
    int index = 0;
};

inline bool operator==(Device a, Device b) { return a.type == b.type && a.index == b.index; }
inline bool operator!=(Device a, Device b) { return !(a == b); }

// "cpu", "cuda", "metal", "vulkan", "rocm".
const char* device_type_name(DeviceType type);

// "rocm:0": the index is always printed.
std::string to_string(Device device);

// Parses "cpu", "rocm", "rocm:1" (any case; a missing index is 0). Throws invalid_argument.
Device parse_device(std::string_view text);

// Devices usable now, CPU first. A backend without hardware does not appear.
std::vector<Device> list_devices();

bool device_available(Device device);

// MENSURFLOW_DEVICE if set (throws if that device is unavailable); otherwise the first
// available of CUDA, Metal, ROCm, Vulkan; otherwise the CPU.
Device default_device();

} // namespace mensurflow
