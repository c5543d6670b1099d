// dtype, execution and device naming, and shape arithmetic: the small value-type helpers of the
// public headers (behaviour of the reference's src/core/{dtype,execution,device,shape}.cpp).
#include "mensurflow/device.hpp"
#include "mensurflow/dtype.hpp"
#include "mensurflow/execution.hpp"
#include "mensurflow/shape.hpp"

#include <algorithm>
#include <cctype>
#include <limits>
#include <stdexcept>

namespace mensurflow {

std::size_t dtype_size(DType dtype) {
    switch (dtype) {
    case DType::F32:
    case DType::I32:
        return 4;
    case DType::F16:
    case DType::BF16:
        return 2;
    case DType::I64:
        return 8;
    case DType::U8:
    case DType::Bool:
        return 1;
    }
    throw std::invalid_argument("invalid DType");
}

const char* dtype_name(DType dtype) {
    switch (dtype) {
    case DType::F32: return "f32";
    case DType::F16: return "f16";
    case DType::BF16: return "bf16";
    case DType::I32: return "i32";
    case DType::I64: return "i64";
    case DType::U8: return "u8";
    case DType::Bool: return "bool";
    }
    throw std::invalid_argument("invalid DType");
}

bool is_floating_point(DType dtype) {
    return dtype == DType::F32 || dtype == DType::F16 || dtype == DType::BF16;
}

const char* execution_name(Execution execution) {
    switch (execution) {
    case Execution::Auto: return "auto";
    case Execution::CPU: return "cpu";
    case Execution::GPU: return "gpu";
    }
    throw std::invalid_argument("invalid Execution value");
}

namespace {
constexpr DeviceType kAllTypes[] = {DeviceType::CPU, DeviceType::CUDA, DeviceType::Metal,
                                    DeviceType::Vulkan, DeviceType::ROCm};
}

const char* device_type_name(DeviceType type) {
    switch (type) {
    case DeviceType::CPU: return "cpu";
    case DeviceType::CUDA: return "cuda";
    case DeviceType::Metal: return "metal";
    case DeviceType::Vulkan: return "vulkan";
    case DeviceType::ROCm: return "rocm";
    }
    throw std::invalid_argument("invalid DeviceType");
}

std::string to_string(Device device) {
    return std::string(device_type_name(device.type)) + ":" + std::to_string(device.index);
}

Device parse_device(std::string_view text) {
    std::string lower(text);
    for (char& ch : lower) {
        ch = static_cast<char>(std::tolower(static_cast<unsigned char>(ch)));
    }
    const auto colon = lower.find(':');
    const std::string name = lower.substr(0, colon);
    Device device;
    bool known = false;
    for (DeviceType type : kAllTypes) {
        if (name == device_type_name(type)) {
            device.type = type;
            known = true;
        }
    }
    if (!known) {
        throw std::invalid_argument("unknown device type: " + std::string(text));
    }
    if (colon != std::string::npos) {
        const std::string digits = lower.substr(colon + 1);
        if (digits.empty() || digits.size() > 6 ||
            digits.find_first_not_of("0123456789") != std::string::npos) {
            throw std::invalid_argument("invalid device index: " + std::string(text));
        }
        device.index = std::stoi(digits);
    }
    return device;
}

void validate_shape(const Shape& shape) {
    std::int64_t count = 1;
    for (std::int64_t d : shape) {
        if (d < 0) {
            throw std::invalid_argument("negative dimension in shape " + to_string(shape));
        }
        if (d != 0 && count > std::numeric_limits<std::int64_t>::max() / d) {
            throw std::invalid_argument("element count overflows in shape " + to_string(shape));
        }
        count *= d;
    }
}

std::int64_t numel(const Shape& shape) {
    std::int64_t count = 1;
    for (std::int64_t d : shape) {
        count *= d;
    }
    return count;
}

Strides contiguous_strides(const Shape& shape) {
    Strides strides(shape.size());
    std::int64_t step = 1;
    for (std::size_t i = shape.size(); i-- > 0;) {
        strides[i] = step;
        step *= shape[i];
    }
    return strides;
}

bool is_contiguous(const Shape& shape, const Strides& strides) {
    if (shape.size() != strides.size()) {
        return false;
    }
    if (numel(shape) == 0) {
        return true;
    }
    std::int64_t want = 1;
    for (std::size_t i = shape.size(); i-- > 0;) {
        if (shape[i] != 1 && strides[i] != want) {
            return false;
        }
        want *= shape[i];
    }
    return true;
}

Shape broadcast_shapes(const Shape& a, const Shape& b) {
    const std::size_t nd = std::max(a.size(), b.size());
    Shape out(nd);
    for (std::size_t i = 0; i < nd; ++i) {
        const std::int64_t da = i < a.size() ? a[a.size() - 1 - i] : 1;
        const std::int64_t db = i < b.size() ? b[b.size() - 1 - i] : 1;
        if (da != db && da != 1 && db != 1) {
            throw std::invalid_argument("cannot broadcast shapes " + to_string(a) + " and " +
                                        to_string(b));
        }
        out[nd - 1 - i] = da == 1 ? db : da;
    }
    return out;
}

Strides broadcast_strides(const Shape& shape, const Strides& strides, const Shape& target) {
    if (shape.size() > target.size() || shape.size() != strides.size()) {
        throw std::invalid_argument("cannot broadcast " + to_string(shape) + " to " +
                                    to_string(target));
    }
    const std::size_t lead = target.size() - shape.size();
    Strides out(target.size(), 0);
    for (std::size_t i = 0; i < shape.size(); ++i) {
        if (shape[i] == target[lead + i]) {
            out[lead + i] = strides[i];
        } else if (shape[i] != 1) {
            throw std::invalid_argument("cannot broadcast " + to_string(shape) + " to " +
                                        to_string(target));
        }
    }
    return out;
}

int normalize_dim(int dim, int ndim) {
    const int out = dim < 0 ? dim + ndim : dim;
    if (out < 0 || out >= ndim) {
        throw std::out_of_range("dim " + std::to_string(dim) + " out of range for " +
                                std::to_string(ndim) + "-d tensor");
    }
    return out;
}

std::string to_string(const Shape& shape) {
    std::string out = "[";
    for (std::size_t i = 0; i < shape.size(); ++i) {
        out += (i ? ", " : "") + std::to_string(shape[i]);
    }
    return out + "]";
}

} // namespace mensurflow
