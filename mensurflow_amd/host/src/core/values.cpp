// The value types of the public headers: element types, execution modes, device names and shape
// arithmetic. Names, messages and the exceptions thrown are mensurflow's (src/core/{dtype,
// execution,device,shape}.cpp); the lookups here are tables, so adding a device type or a dtype
// is one row.
#include "mensurflow/device.hpp"
#include "mensurflow/dtype.hpp"
#include "mensurflow/execution.hpp"
#include "mensurflow/shape.hpp"

#include <algorithm>
#include <cctype>
#include <numeric>
#include <sstream>
#include <stdexcept>

namespace mensurflow {

namespace {

struct DTypeRow {
    DType type;
    const char* name;
    std::size_t bytes;
    bool floating;
};

constexpr DTypeRow kDTypeRows[] = {
    {DType::F32, "f32", 4, true},  {DType::F16, "f16", 2, true}, {DType::BF16, "bf16", 2, true},
    {DType::I32, "i32", 4, false}, {DType::I64, "i64", 8, false}, {DType::U8, "u8", 1, false},
    {DType::Bool, "bool", 1, false},
};

const DTypeRow& row_of(DType type) {
    for (const DTypeRow& row : kDTypeRows) {
        if (row.type == type) {
            return row;
        }
    }
    throw std::invalid_argument("invalid DType");
}

struct DeviceRow {
    DeviceType type;
    const char* name;
};

// Every device type a name can denote ("rocm" is this build's addition).
constexpr DeviceRow kDeviceRows[] = {
    {DeviceType::CPU, "cpu"},       {DeviceType::CUDA, "cuda"}, {DeviceType::Metal, "metal"},
    {DeviceType::Vulkan, "vulkan"}, {DeviceType::ROCm, "rocm"},
};

// Extent `back` places from the end of `shape` (0 = last); 1 past its front, as broadcasting
// pads a shorter shape on the left.
std::int64_t extent_from_back(const Shape& shape, std::size_t back) {
    return back < shape.size() ? shape[shape.size() - 1 - back] : 1;
}

} // namespace

std::size_t dtype_size(DType dtype) { return row_of(dtype).bytes; }

const char* dtype_name(DType dtype) { return row_of(dtype).name; }

bool is_floating_point(DType dtype) {
    for (const DTypeRow& row : kDTypeRows) {
        if (row.type == dtype) {
            return row.floating;
        }
    }
    return false;
}

const char* execution_name(Execution execution) {
    switch (execution) {
    case Execution::Auto: return "auto";
    case Execution::CPU: return "cpu";
    case Execution::GPU: return "gpu";
    }
    throw std::invalid_argument("invalid Execution value");
}

const char* device_type_name(DeviceType type) {
    const auto* row = std::find_if(std::begin(kDeviceRows), std::end(kDeviceRows),
                                   [type](const DeviceRow& r) { return r.type == type; });
    if (row == std::end(kDeviceRows)) {
        throw std::invalid_argument("invalid DeviceType");
    }
    return row->name;
}

std::string to_string(Device device) {
    std::string text = device_type_name(device.type);
    text += ':';
    text += std::to_string(device.index);
    return text;
}

Device parse_device(std::string_view text) {
    std::string folded(text.size(), '\0');
    std::transform(text.begin(), text.end(), folded.begin(),
                   [](char c) { return static_cast<char>(std::tolower(static_cast<unsigned char>(c))); });
    const std::size_t colon = folded.find(':');
    const std::string_view type_part = std::string_view(folded).substr(0, colon);
    const auto* row = std::find_if(std::begin(kDeviceRows), std::end(kDeviceRows),
                                   [type_part](const DeviceRow& r) { return type_part == r.name; });
    if (row == std::end(kDeviceRows)) {
        throw std::invalid_argument("unknown device type: " + std::string(text));
    }
    Device device{row->type, 0};
    if (colon == std::string::npos) {
        return device;
    }
    // An index is 1 to 6 decimal digits and nothing else ("rocm:", "rocm:-1", "rocm:1x" fail).
    const std::string_view digits = std::string_view(folded).substr(colon + 1);
    const bool well_formed = !digits.empty() && digits.size() <= 6 &&
                             std::all_of(digits.begin(), digits.end(),
                                         [](char c) { return c >= '0' && c <= '9'; });
    if (!well_formed) {
        throw std::invalid_argument("invalid device index: " + std::string(text));
    }
    device.index = std::accumulate(digits.begin(), digits.end(), 0,
                                   [](int value, char c) { return value * 10 + (c - '0'); });
    return device;
}

void validate_shape(const Shape& shape) {
    // One pass, so the first offending extent decides which error is reported.
    std::int64_t product = 1;
    for (const std::int64_t extent : shape) {
        if (extent < 0) {
            throw std::invalid_argument("negative dimension in shape " + to_string(shape));
        }
        if (__builtin_mul_overflow(product, extent, &product)) {
            throw std::invalid_argument("element count overflows in shape " + to_string(shape));
        }
    }
}

std::int64_t numel(const Shape& shape) {
    return std::accumulate(shape.begin(), shape.end(), std::int64_t{1},
                           [](std::int64_t acc, std::int64_t e) { return acc * e; });
}

Strides contiguous_strides(const Shape& shape) {
    Strides strides(shape.size());
    std::int64_t span = 1;
    std::transform(shape.rbegin(), shape.rend(), strides.rbegin(), [&span](std::int64_t extent) {
        const std::int64_t stride = span;
        span *= extent;
        return stride;
    });
    return strides;
}

bool is_contiguous(const Shape& shape, const Strides& strides) {
    if (shape.size() != strides.size()) {
        return false;
    }
    if (numel(shape) == 0) {
        return true; // nothing is addressed
    }
    const Strides packed = contiguous_strides(shape);
    for (std::size_t d = 0; d < shape.size(); ++d) {
        // An extent-1 dimension is never stepped along, so its stride is free.
        if (shape[d] != 1 && strides[d] != packed[d]) {
            return false;
        }
    }
    return true;
}

Shape broadcast_shapes(const Shape& a, const Shape& b) {
    Shape out(std::max(a.size(), b.size()));
    for (std::size_t back = 0; back < out.size(); ++back) {
        const std::int64_t ea = extent_from_back(a, back);
        const std::int64_t eb = extent_from_back(b, back);
        if (ea != eb && ea != 1 && eb != 1) {
            throw std::invalid_argument("cannot broadcast shapes " + to_string(a) + " and " +
                                        to_string(b));
        }
        out[out.size() - 1 - back] = ea == 1 ? eb : ea;
    }
    return out;
}

Strides broadcast_strides(const Shape& shape, const Strides& strides, const Shape& target) {
    const auto refuse = [&] {
        return std::invalid_argument("cannot broadcast " + to_string(shape) + " to " +
                                     to_string(target));
    };
    if (shape.size() > target.size() || shape.size() != strides.size()) {
        throw refuse();
    }
    // Leading dimensions the view gains, and extent-1 dimensions it stretches, repeat one element:
    // stride 0.
    Strides out(target.size(), 0);
    for (std::size_t back = 0; back < shape.size(); ++back) {
        const std::size_t from = shape.size() - 1 - back;
        const std::size_t to = target.size() - 1 - back;
        if (shape[from] == target[to]) {
            out[to] = strides[from];
        } else if (shape[from] != 1) {
            throw refuse();
        }
    }
    return out;
}

int normalize_dim(int dim, int ndim) {
    const int wrapped = dim >= 0 ? dim : dim + ndim;
    if (wrapped >= 0 && wrapped < ndim) {
        return wrapped;
    }
    throw std::out_of_range("dim " + std::to_string(dim) + " out of range for " +
                            std::to_string(ndim) + "-d tensor");
}

std::string to_string(const Shape& shape) {
    std::ostringstream text;
    text << '[';
    const char* separator = "";
    for (const std::int64_t extent : shape) {
        text << separator << extent;
        separator = ", ";
    }
    text << ']';
    return text.str();
}

} // namespace mensurflow
