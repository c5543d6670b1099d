// Tensor creation, views and transfers (behaviour of the reference's src/core/tensor.cpp,
// without autograd). Device-resident strided views are packed on the device when the backend
// registers OpId::StridedCopy for the dtype; otherwise they are staged through host memory.
#include "mensurflow/tensor.hpp"

#include "core/dispatcher.hpp"
#include "core/registry.hpp"
#include "core/storage.hpp"
#include "core/tensor_access.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>

namespace mensurflow {

namespace {

void validate_fill_value(double value, DType dtype) {
    if (!std::isfinite(value)) {
        if (dtype != DType::F32) {
            throw std::invalid_argument("full: non-finite values require f32 dtype");
        }
        return;
    }
    auto whole_in = [&](double lo, double hi) {
        return std::trunc(value) == value && value >= lo && value <= hi;
    };
    switch (dtype) {
    case DType::F32:
        if (std::fabs(value) > std::numeric_limits<float>::max()) {
            throw std::invalid_argument("full: value does not fit f32");
        }
        return;
    case DType::I32:
        if (!whole_in(std::numeric_limits<std::int32_t>::min(),
                      std::numeric_limits<std::int32_t>::max())) {
            throw std::invalid_argument("full: value does not fit i32");
        }
        return;
    case DType::I64:
        if (!whole_in(static_cast<double>(std::numeric_limits<std::int64_t>::min()),
                      static_cast<double>(std::numeric_limits<std::int64_t>::max()))) {
            throw std::invalid_argument("full: value does not fit i64");
        }
        return;
    case DType::U8:
        if (!whole_in(0, 255)) {
            throw std::invalid_argument("full: value does not fit u8");
        }
        return;
    case DType::Bool:
        return;
    case DType::F16:
    case DType::BF16:
        throw std::invalid_argument("full: f16 and bf16 construction is not supported");
    }
    throw std::invalid_argument("full: invalid dtype");
}

void write_fill(std::byte* data, std::size_t count, DType dtype, double value) {
    switch (dtype) {
    case DType::F32:
        std::fill_n(reinterpret_cast<float*>(data), count, static_cast<float>(value));
        return;
    case DType::I32:
        std::fill_n(reinterpret_cast<std::int32_t*>(data), count, static_cast<std::int32_t>(value));
        return;
    case DType::I64:
        std::fill_n(reinterpret_cast<std::int64_t*>(data), count, static_cast<std::int64_t>(value));
        return;
    case DType::U8:
        std::fill_n(data, count, static_cast<std::byte>(static_cast<std::uint8_t>(value)));
        return;
    case DType::Bool:
        std::fill_n(data, count, value == 0 ? std::byte{0} : std::byte{1});
        return;
    default:
        throw std::invalid_argument("full: unsupported dtype");
    }
}

// Row-major gather of a strided view from host-addressable memory: an odometer over the
// indices, copying the last dimension as one run when its stride is 1.
void gather(const std::byte* base, std::byte* out, const Shape& shape, const Strides& strides,
            std::size_t item) {
    const int nd = static_cast<int>(shape.size());
    const std::int64_t count = numel(shape);
    if (count == 0) {
        return;
    }
    if (nd == 0) {
        std::memcpy(out, base, item);
        return;
    }
    const bool unit_rows = strides[nd - 1] == 1;
    const std::int64_t run = unit_rows ? shape[nd - 1] : 1;
    const int outer = unit_rows ? nd - 1 : nd;
    std::vector<std::int64_t> index(static_cast<std::size_t>(nd), 0);
    std::int64_t pos = 0;
    for (std::int64_t done = 0; done < count; done += run) {
        std::memcpy(out, base + pos * static_cast<std::int64_t>(item),
                    static_cast<std::size_t>(run) * item);
        out += static_cast<std::size_t>(run) * item;
        for (int d = outer - 1; d >= 0; --d) {
            if (++index[d] < shape[d]) {
                pos += strides[d];
                break;
            }
            pos -= (shape[d] - 1) * strides[d];
            index[d] = 0;
        }
    }
}

bool packs_on_device(Device device, DType dtype) {
    return device.type != DeviceType::CPU &&
           detail::Registry::instance().dispatcher().find(
               {detail::OpId::StridedCopy, device.type, dtype}) != nullptr;
}

} // namespace

Tensor::Tensor(std::shared_ptr<detail::Storage> storage, std::int64_t offset, Shape shape,
               Strides strides, DType dtype)
    : storage_(std::move(storage)), offset_(offset), shape_(std::move(shape)),
      strides_(std::move(strides)), dtype_(dtype) {}

Tensor Tensor::empty(Shape shape, DType dtype, Device device) {
    validate_shape(shape);
    const auto bytes = static_cast<std::size_t>(mensurflow::numel(shape)) * dtype_size(dtype);
    auto storage = std::make_shared<detail::Storage>(device, bytes);
    Strides strides = contiguous_strides(shape);
    return Tensor(std::move(storage), 0, std::move(shape), std::move(strides), dtype);
}

Tensor Tensor::full(Shape shape, double value, DType dtype, Device device) {
    validate_shape(shape);
    validate_fill_value(value, dtype);
    const auto count = static_cast<std::size_t>(mensurflow::numel(shape));
    std::vector<std::byte> host(count * dtype_size(dtype));
    write_fill(host.data(), count, dtype, value);
    return from_host(host.data(), std::move(shape), dtype, device);
}

Tensor Tensor::constant(Shape shape, double value, DType dtype, Device device) {
    return full(std::move(shape), value, dtype, device);
}

Tensor Tensor::zeros(Shape shape, DType dtype, Device device) {
    validate_shape(shape);
    std::vector<std::byte> host(static_cast<std::size_t>(mensurflow::numel(shape)) *
                                dtype_size(dtype));
    return from_host(host.data(), std::move(shape), dtype, device);
}

Tensor Tensor::ones(Shape shape, DType dtype, Device device) {
    return full(std::move(shape), 1.0, dtype, device);
}

Tensor Tensor::eye(std::int64_t n, DType dtype, Device device) {
    if (n < 0) {
        throw std::invalid_argument("eye: dimension must be non-negative");
    }
    validate_fill_value(1.0, dtype);
    const auto count = static_cast<std::size_t>(n) * static_cast<std::size_t>(n);
    std::vector<std::byte> host(count * dtype_size(dtype));
    write_fill(host.data(), count, dtype, 0.0);
    for (std::int64_t i = 0; i < n; ++i) {
        write_fill(host.data() + static_cast<std::size_t>(i * n + i) * dtype_size(dtype), 1, dtype,
                   1.0);
    }
    return from_host(host.data(), {n, n}, dtype, device);
}

Tensor Tensor::zeros_like(const Tensor& other) {
    return zeros(other.shape(), other.dtype(), other.device());
}

Tensor Tensor::ones_like(const Tensor& other) {
    return ones(other.shape(), other.dtype(), other.device());
}

Tensor Tensor::full_like(const Tensor& other, double value) {
    return full(other.shape(), value, other.dtype(), other.device());
}

Tensor Tensor::from_host(const void* data, Shape shape, DType dtype, Device device) {
    Tensor out = empty(std::move(shape), dtype, device);
    if (out.nbytes() > 0) {
        if (data == nullptr) {
            throw std::invalid_argument("from_host: data is null");
        }
        out.storage_->copy_from_host(0, data, out.nbytes());
    }
    return out;
}

Tensor Tensor::to(Device target) const {
    require_defined();
    if (target == device()) {
        return *this;
    }
    Tensor out = empty(shape_, dtype_, target);
    if (out.nbytes() > 0) {
        std::vector<std::byte> host(out.nbytes());
        copy_to_host(host.data());
        out.storage_->copy_from_host(0, host.data(), host.size());
    }
    return out;
}

Tensor Tensor::contiguous() const {
    require_defined();
    if (is_contiguous()) {
        return *this;
    }
    Tensor out = empty(shape_, dtype_, device());
    if (const std::byte* host = storage_->host_data()) {
        gather(host + static_cast<std::size_t>(offset_) * itemsize(),
               static_cast<std::byte*>(out.storage_->host_data()), shape_, strides_, itemsize());
        return out;
    }
    if (packs_on_device(device(), dtype_)) {
        detail::dispatch(detail::OpId::StridedCopy, {{*this}, {out}}, Execution::GPU);
        return out;
    }
    std::vector<std::byte> staged(out.nbytes());
    copy_to_host(staged.data());
    out.storage_->copy_from_host(0, staged.data(), staged.size());
    return out;
}

void Tensor::copy_from(const Tensor& source) {
    require_defined();
    source.require_defined();
    if (shape_ != source.shape_ || dtype_ != source.dtype_ || device() != source.device()) {
        throw std::invalid_argument(
            "copy_from: tensors must have matching shape, dtype, and device");
    }
    if (nbytes() == 0) {
        return;
    }
    const Tensor packed = source.contiguous();
    const std::size_t item = itemsize();
    if (is_contiguous()) {
        if (storage_->host_data() != nullptr) {
            std::memmove(storage_->host_data() + static_cast<std::size_t>(offset_) * item,
                         packed.storage_->host_data() +
                             static_cast<std::size_t>(packed.offset_) * item,
                         nbytes());
        } else {
            storage_->stream().copy_d2d(*storage_->buffer,
                                        static_cast<std::size_t>(offset_) * item,
                                        *packed.storage_->buffer,
                                        static_cast<std::size_t>(packed.offset_) * item, nbytes());
        }
        return;
    }
    // A strided destination: write element by element through host memory.
    std::vector<std::byte> values(packed.nbytes());
    packed.copy_to_host(values.data());
    if (std::byte* host = storage_->host_data()) {
        const Shape& shape = shape_;
        std::vector<std::int64_t> index(shape.size(), 0);
        for (std::int64_t i = 0; i < numel(); ++i) {
            std::int64_t pos = offset_;
            std::int64_t rest = i;
            for (std::size_t d = shape.size(); d-- > 0;) {
                pos += (rest % shape[d]) * strides_[d];
                rest /= shape[d];
            }
            std::memcpy(host + pos * static_cast<std::int64_t>(item),
                        values.data() + i * static_cast<std::int64_t>(item), item);
        }
        return;
    }
    throw std::invalid_argument("copy_from: a strided destination must be host memory");
}

void Tensor::copy_to_host(void* dst) const {
    require_defined();
    if (nbytes() == 0) {
        return;
    }
    if (dst == nullptr) {
        throw std::invalid_argument("copy_to_host: dst is null");
    }
    const std::size_t item = itemsize();
    const std::size_t byte_offset = static_cast<std::size_t>(offset_) * item;
    if (is_contiguous()) {
        storage_->copy_to_host(dst, byte_offset, nbytes());
        return;
    }
    if (const std::byte* host = storage_->host_data()) {
        gather(host + byte_offset, static_cast<std::byte*>(dst), shape_, strides_, item);
        return;
    }
    if (packs_on_device(device(), dtype_)) {
        contiguous().copy_to_host(dst);
        return;
    }
    // Stage the allocation from the view's offset onward, then gather on the host.
    std::vector<std::byte> staged(storage_->nbytes - byte_offset);
    storage_->copy_to_host(staged.data(), byte_offset, staged.size());
    gather(staged.data(), static_cast<std::byte*>(dst), shape_, strides_, item);
}

Tensor Tensor::make_view(std::int64_t offset, Shape shape, Strides strides) const {
    return Tensor(storage_, offset, std::move(shape), std::move(strides), dtype_);
}

Tensor Tensor::transpose(int d0, int d1) const {
    const int a = normalize_dim(d0, dim());
    const int b = normalize_dim(d1, dim());
    Shape shape = shape_;
    Strides strides = strides_;
    std::swap(shape[a], shape[b]);
    std::swap(strides[a], strides[b]);
    return make_view(offset_, std::move(shape), std::move(strides));
}

Tensor Tensor::permute(const std::vector<int>& order) const {
    if (order.size() != static_cast<std::size_t>(dim())) {
        throw std::invalid_argument("permute: expected " + std::to_string(dim()) +
                                    " dimensions, got " + std::to_string(order.size()));
    }
    std::vector<bool> used(order.size(), false);
    Shape shape;
    Strides strides;
    for (int value : order) {
        int axis = 0;
        try {
            axis = normalize_dim(value, dim());
        } catch (const std::out_of_range&) {
            throw std::invalid_argument("permute: dimension " + std::to_string(value) +
                                        " is out of range");
        }
        if (used[static_cast<std::size_t>(axis)]) {
            throw std::invalid_argument("permute: dimension " + std::to_string(value) +
                                        " appears more than once");
        }
        used[static_cast<std::size_t>(axis)] = true;
        shape.push_back(shape_[static_cast<std::size_t>(axis)]);
        strides.push_back(strides_[static_cast<std::size_t>(axis)]);
    }
    return make_view(offset_, std::move(shape), std::move(strides));
}

Tensor Tensor::slice(int d, std::int64_t start, std::int64_t end, std::int64_t step) const {
    const int axis = normalize_dim(d, dim());
    if (step < 1) {
        throw std::invalid_argument("slice: step must be >= 1");
    }
    const std::int64_t n = shape_[axis];
    auto clamp = [n](std::int64_t i) { return std::clamp(i < 0 ? i + n : i, std::int64_t{0}, n); };
    start = clamp(start);
    end = std::max(clamp(end), start);
    Shape shape = shape_;
    Strides strides = strides_;
    shape[axis] = (end - start + step - 1) / step;
    strides[axis] *= step;
    return make_view(offset_ + start * strides_[axis], std::move(shape), std::move(strides));
}

Tensor Tensor::expand(const Shape& shape) const {
    validate_shape(shape);
    Strides strides = broadcast_strides(this->shape(), strides_, shape);
    return make_view(offset_, shape, std::move(strides));
}

Tensor Tensor::unsqueeze(int d) const {
    const int axis = normalize_dim(d, dim() + 1);
    Shape shape = shape_;
    Strides strides = strides_;
    const std::int64_t stride = axis < dim() ? shape_[axis] * strides_[axis] : 1;
    shape.insert(shape.begin() + axis, 1);
    strides.insert(strides.begin() + axis, stride);
    return make_view(offset_, std::move(shape), std::move(strides));
}

Tensor Tensor::view(Shape shape) const {
    if (!is_contiguous()) {
        throw std::invalid_argument("view: tensor is not contiguous");
    }
    auto inferred = shape.end();
    std::int64_t known = 1;
    for (auto it = shape.begin(); it != shape.end(); ++it) {
        if (*it == -1) {
            if (inferred != shape.end()) {
                throw std::invalid_argument("view: only one dimension can be -1");
            }
            inferred = it;
        } else {
            known *= *it;
        }
    }
    if (inferred != shape.end()) {
        if (known == 0 || numel() % known != 0) {
            throw std::invalid_argument("view: cannot infer -1 in " + to_string(shape));
        }
        *inferred = numel() / known;
    }
    validate_shape(shape);
    if (mensurflow::numel(shape) != numel()) {
        throw std::invalid_argument("view: shape " + to_string(shape) + " does not match " +
                                    std::to_string(numel()) + " elements");
    }
    Strides strides = contiguous_strides(shape);
    return make_view(offset_, std::move(shape), std::move(strides));
}

bool Tensor::shares_storage(const Tensor& other) const {
    return defined() && storage_ == other.storage_;
}

void Tensor::require_defined() const {
    if (!defined()) {
        throw std::logic_error("operation on an undefined Tensor");
    }
}

const Shape& Tensor::shape() const {
    require_defined();
    return shape_;
}

const Strides& Tensor::strides() const {
    require_defined();
    return strides_;
}

std::int64_t Tensor::offset() const {
    require_defined();
    return offset_;
}

DType Tensor::dtype() const {
    require_defined();
    return dtype_;
}

Device Tensor::device() const {
    require_defined();
    return storage_->device;
}

int Tensor::dim() const { return static_cast<int>(shape().size()); }

std::int64_t Tensor::size(int d) const {
    return shape()[static_cast<std::size_t>(normalize_dim(d, dim()))];
}

std::int64_t Tensor::numel() const { return mensurflow::numel(shape()); }

std::size_t Tensor::itemsize() const { return dtype_size(dtype()); }

std::size_t Tensor::nbytes() const { return static_cast<std::size_t>(numel()) * itemsize(); }

bool Tensor::is_contiguous() const { return mensurflow::is_contiguous(shape(), strides()); }

} // namespace mensurflow
