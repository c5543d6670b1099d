// Tensor creation, views and transfers. The behaviour (checks, messages, results) is mensurflow's
// src/core/tensor.cpp without autograd. The moves between memory and views are built on one
// walker: every strided view is visited as runs of consecutive elements, which packing (host
// gather), unpacking (host scatter) and the exact byte span a view reaches all share. Device
// views are packed on the device when its backend registers OpId::StridedCopy for the dtype.
#include "mensurflow/tensor.hpp"
#include "mensurflow/trace.hpp"

#include "core/dispatcher.hpp"
#include "core/registry.hpp"
#include "core/storage.hpp"
#include "core/tensor_access.hpp"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <limits>

namespace mensurflow {

namespace {

// ---- fill values ---------------------------------------------------------------------------------

// The bit pattern of `value` as one element of `dtype`, after the checks of mensurflow's Tensor::
// full (a value the dtype cannot hold exactly is refused).
struct Element {
    std::array<std::byte, 8> bytes{};
    std::size_t width = 0;
};

template <typename T> Element element_of(T value) {
    Element e;
    e.width = sizeof(T);
    std::memcpy(e.bytes.data(), &value, sizeof(T));
    return e;
}

bool whole_within(double value, double low, double high) {
    return std::trunc(value) == value && value >= low && value <= high;
}

Element fill_element(double value, DType dtype) {
    if (!std::isfinite(value) && dtype != DType::F32) {
        throw std::invalid_argument("full: non-finite values require f32 dtype");
    }
    switch (dtype) {
    case DType::F32:
        if (std::isfinite(value) && std::fabs(value) > std::numeric_limits<float>::max()) {
            throw std::invalid_argument("full: value does not fit f32");
        }
        return element_of(static_cast<float>(value));
    case DType::I32:
        if (!whole_within(value, std::numeric_limits<std::int32_t>::min(),
                          std::numeric_limits<std::int32_t>::max())) {
            throw std::invalid_argument("full: value does not fit i32");
        }
        return element_of(static_cast<std::int32_t>(value));
    case DType::I64:
        if (!whole_within(value, static_cast<double>(std::numeric_limits<std::int64_t>::min()),
                          static_cast<double>(std::numeric_limits<std::int64_t>::max()))) {
            throw std::invalid_argument("full: value does not fit i64");
        }
        return element_of(static_cast<std::int64_t>(value));
    case DType::U8:
        if (!whole_within(value, 0.0, 255.0)) {
            throw std::invalid_argument("full: value does not fit u8");
        }
        return element_of(static_cast<std::uint8_t>(value));
    case DType::Bool:
        return element_of(static_cast<std::uint8_t>(value != 0.0 ? 1 : 0));
    case DType::F16:
    case DType::BF16:
        throw std::invalid_argument("full: f16 and bf16 construction is not supported yet");
    }
    throw std::invalid_argument("full: invalid dtype");
}

// `count` copies of `element`, back to back.
std::vector<std::byte> repeated(const Element& element, std::size_t count) {
    std::vector<std::byte> out(count * element.width);
    for (std::size_t at = 0; at < out.size(); at += element.width) {
        std::memcpy(out.data() + at, element.bytes.data(), element.width);
    }
    return out;
}

// ---- strided views ---------------------------------------------------------------------------------

// Calls visit(first, length) for the elements of a (shape, strides) view in row-major order, as
// runs of `length` consecutive elements starting `first` elements from the view's origin. The
// innermost dimension forms one run when its stride is 1, else runs of one element.
template <typename Visit>
void walk(const Shape& shape, const Strides& strides, std::size_t d, std::int64_t base,
          Visit& visit) {
    const std::int64_t extent = shape[d];
    if (d + 1 == shape.size()) {
        if (strides[d] == 1) {
            visit(base, extent);
        } else {
            for (std::int64_t i = 0; i < extent; ++i) {
                visit(base + i * strides[d], std::int64_t{1});
            }
        }
        return;
    }
    for (std::int64_t i = 0; i < extent; ++i) {
        walk(shape, strides, d + 1, base + i * strides[d], visit);
    }
}

template <typename Visit> void for_each_run(const Shape& shape, const Strides& strides, Visit visit) {
    if (numel(shape) == 0) {
        return;
    }
    if (shape.empty()) {
        visit(std::int64_t{0}, std::int64_t{1}); // a 0-d view is one element
        return;
    }
    walk(shape, strides, 0, 0, visit);
}

// Packs the view whose origin is `origin` into contiguous `packed`.
void gather(const std::byte* origin, std::byte* packed, const Shape& shape, const Strides& strides,
            std::size_t item) {
    for_each_run(shape, strides, [&](std::int64_t first, std::int64_t length) {
        const std::size_t bytes = static_cast<std::size_t>(length) * item;
        std::memcpy(packed, origin + static_cast<std::ptrdiff_t>(first) * static_cast<std::ptrdiff_t>(item), bytes);
        packed += bytes;
    });
}

// The inverse: contiguous `packed` into the view whose origin is `origin`.
void scatter(const std::byte* packed, std::byte* origin, const Shape& shape, const Strides& strides,
             std::size_t item) {
    for_each_run(shape, strides, [&](std::int64_t first, std::int64_t length) {
        const std::size_t bytes = static_cast<std::size_t>(length) * item;
        std::memcpy(origin + static_cast<std::ptrdiff_t>(first) * static_cast<std::ptrdiff_t>(item), packed, bytes);
        packed += bytes;
    });
}

// Elements from a view's origin to one past the furthest element it reaches (views made by this
// class never have negative strides).
std::int64_t reach(const Shape& shape, const Strides& strides) {
    if (numel(shape) == 0) {
        return 0;
    }
    std::int64_t last = 0;
    for (std::size_t d = 0; d < shape.size(); ++d) {
        last += (shape[d] - 1) * strides[d];
    }
    return last + 1;
}

bool packs_on_device(Device device, DType dtype) {
    return device.type != DeviceType::CPU &&
           detail::Registry::instance().dispatcher().find(
               {detail::OpId::StridedCopy, device.type, dtype}) != nullptr;
}

// Packs the view (shape, strides) at element `offset` of device storage into host memory `dst`:
// only the bytes the view reaches come over, then they are packed on the host.
void gather_through_host(const detail::Storage& storage, std::int64_t offset, const Shape& shape,
                         const Strides& strides, std::size_t item, void* dst) {
    std::vector<std::byte> span(static_cast<std::size_t>(reach(shape, strides)) * item);
    storage.copy_to_host(span.data(), static_cast<std::size_t>(offset) * item, span.size());
    gather(span.data(), static_cast<std::byte*>(dst), shape, strides, item);
}

// Packs `view` (device memory) into `out` (contiguous, same shape, on the same device) with the
// device's strided copy. False when the device copy does not take the layout (it throws
// NotImplemented, e.g. for more dimensions than it handles): the caller packs through host
// memory instead.
bool pack_on_device(const Tensor& view, const Tensor& out) {
    try {
        detail::dispatch(detail::OpId::StridedCopy, {{view}, {out}}, Execution::GPU);
        return true;
    } catch (const detail::NotImplemented&) {
        return false;
    }
}

} // namespace

// ---- construction ---------------------------------------------------------------------------------

Tensor::Tensor(std::shared_ptr<detail::Storage> storage, std::int64_t offset, Shape shape,
               Strides strides, DType dtype)
    : storage_(std::move(storage)), offset_(offset), shape_(std::move(shape)),
      strides_(std::move(strides)), dtype_(dtype) {}

Tensor Tensor::empty(Shape shape, DType dtype, Device device) {
    validate_shape(shape);
    MENSURFLOW_TRACE("Tensor::empty", device, shape, dtype);
    const std::size_t bytes = static_cast<std::size_t>(mensurflow::numel(shape)) * dtype_size(dtype);
    Strides strides = contiguous_strides(shape);
    return Tensor(std::make_shared<detail::Storage>(device, bytes), 0, std::move(shape),
                  std::move(strides), dtype);
}

Tensor Tensor::full(Shape shape, double value, DType dtype, Device device) {
    validate_shape(shape);
    const Element element = fill_element(value, dtype);
    const auto host = repeated(element, static_cast<std::size_t>(mensurflow::numel(shape)));
    return from_host(host.data(), std::move(shape), dtype, device);
}

Tensor Tensor::constant(Shape shape, double value, DType dtype, Device device) {
    return full(std::move(shape), value, dtype, device);
}

Tensor Tensor::zeros(Shape shape, DType dtype, Device device) {
    validate_shape(shape);
    const std::vector<std::byte> host(static_cast<std::size_t>(mensurflow::numel(shape)) *
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
    const Element one = fill_element(1.0, dtype);
    std::vector<std::byte> host(static_cast<std::size_t>(n * n) * one.width);
    for (std::int64_t i = 0; i < n; ++i) {
        std::memcpy(host.data() + static_cast<std::size_t>(i * (n + 1)) * one.width,
                    one.bytes.data(), one.width);
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
    MENSURFLOW_TRACE("Tensor::from_host", device, shape, dtype);
    Tensor out = empty(std::move(shape), dtype, device);
    if (out.nbytes() == 0) {
        return out;
    }
    if (data == nullptr) {
        throw std::invalid_argument("from_host: data is null");
    }
    out.storage_->copy_from_host(0, data, out.nbytes());
    return out;
}

// ---- transfers ----------------------------------------------------------------------------------------

Tensor Tensor::to(Device target) const {
    require_defined();
    if (device() == target) {
        return *this;
    }
    MENSURFLOW_TRACE("Tensor::to", target, shape_, dtype_);
    // A strided host view bound for a device that packs views: the bytes it spans go over as
    // they lie, and the device packs them (a transposed 4096^2 operand is one 64 MiB transfer
    // and a device transpose instead of a host gather). Taken while the span is at most 4 times
    // the view's own bytes, so a sparse slice does not drag its whole base along.
    // A layout the device copy does not take goes on to the host gather below.
    if (const std::byte* src = storage_->host_data();
        src != nullptr && !is_contiguous() && packs_on_device(target, dtype_)) {
        const std::int64_t span = reach(shape_, strides_);
        if (span > 0 && span <= 4 * numel()) {
            Tensor raw = empty({span}, dtype_, target);
            raw.storage_->copy_from_host(0, src + static_cast<std::size_t>(offset_) * itemsize(),
                                         static_cast<std::size_t>(span) * itemsize());
            Tensor packed = empty(shape_, dtype_, target);
            if (pack_on_device(Tensor(raw.storage_, 0, shape_, strides_, dtype_), packed)) {
                return packed;
            }
        }
    }
    Tensor out = empty(shape_, dtype_, target);
    if (out.nbytes() == 0) {
        return out;
    }
    // Host memory on either side is read or written in place. A temporary host copy is made
    // only between two devices or from a strided host view that the branch above leaves:
    // building one for every transfer cost a fill, page faults and one more pass over host
    // memory (a 1 GiB operand moved at ~4 GB/s).
    if (std::byte* dst = out.storage_->host_data()) {
        copy_to_host(dst);
    } else if (const std::byte* src = storage_->host_data(); src != nullptr && is_contiguous()) {
        out.storage_->copy_from_host(0, src + static_cast<std::size_t>(offset_) * itemsize(),
                                     out.nbytes());
    } else {
        std::vector<std::byte> bounce(out.nbytes());
        copy_to_host(bounce.data());
        out.storage_->copy_from_host(0, bounce.data(), bounce.size());
    }
    return out;
}

Tensor Tensor::contiguous() const {
    require_defined();
    if (is_contiguous()) {
        return *this;
    }
    MENSURFLOW_TRACE("Tensor::contiguous", device(), shape_, dtype_);
    Tensor out = empty(shape_, dtype_, device());
    if (std::byte* host = storage_->host_data()) {
        gather(host + static_cast<std::size_t>(offset_) * itemsize(), out.storage_->host_data(),
               shape_, strides_, itemsize());
    } else if (!packs_on_device(device(), dtype_) || !pack_on_device(*this, out)) {
        // Through host memory: the span the view reaches comes over and is packed there.
        std::vector<std::byte> packed(out.nbytes());
        gather_through_host(*storage_, offset_, shape_, strides_, itemsize(), packed.data());
        out.storage_->copy_from_host(0, packed.data(), packed.size());
    }
    return out;
}

void Tensor::copy_to_host(void* dst) const {
    require_defined();
    if (nbytes() == 0) {
        return;
    }
    if (dst == nullptr) {
        throw std::invalid_argument("copy_to_host: dst is null");
    }
    MENSURFLOW_TRACE("Tensor::copy_to_host", device(), shape_, dtype_);
    const std::size_t item = itemsize();
    const std::size_t origin = static_cast<std::size_t>(offset_) * item;
    auto* out = static_cast<std::byte*>(dst);
    if (is_contiguous()) {
        storage_->copy_to_host(out, origin, nbytes());
    } else if (const std::byte* host = storage_->host_data()) {
        gather(host + origin, out, shape_, strides_, item);
    } else {
        if (packs_on_device(device(), dtype_)) {
            Tensor packed = empty(shape_, dtype_, device());
            if (pack_on_device(*this, packed)) {
                packed.copy_to_host(out);
                return;
            }
        }
        gather_through_host(*storage_, offset_, shape_, strides_, item, out);
    }
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
    MENSURFLOW_TRACE("Tensor::copy_from", device(), shape_, dtype_);
    const Tensor packed = source.contiguous();
    const std::size_t item = itemsize();
    const std::size_t origin = static_cast<std::size_t>(offset_) * item;
    const std::size_t packed_origin = static_cast<std::size_t>(packed.offset_) * item;
    std::byte* host = storage_->host_data();
    if (is_contiguous()) {
        if (host != nullptr) {
            std::memmove(host + origin, packed.storage_->host_data() + packed_origin, nbytes());
        } else {
            storage_->stream().copy_d2d(*storage_->buffer, origin, *packed.storage_->buffer,
                                        packed_origin, nbytes());
        }
        return;
    }
    // A strided destination: its elements are unpacked into place. Device memory goes through
    // host memory: the span the view reaches is read, updated and written back.
    std::vector<std::byte> values(packed.nbytes());
    packed.copy_to_host(values.data());
    if (host != nullptr) {
        scatter(values.data(), host + origin, shape_, strides_, item);
        return;
    }
    std::vector<std::byte> span(static_cast<std::size_t>(reach(shape_, strides_)) * item);
    storage_->copy_to_host(span.data(), origin, span.size());
    scatter(values.data(), span.data(), shape_, strides_, item);
    storage_->copy_from_host(origin, span.data(), span.size());
}

// ---- views ----------------------------------------------------------------------------------------------

Tensor Tensor::reshaped(std::int64_t offset, Shape shape, Strides strides) const {
    return Tensor(storage_, offset, std::move(shape), std::move(strides), dtype_);
}

Tensor Tensor::transpose(int d0, int d1) const {
    const auto a = static_cast<std::size_t>(normalize_dim(d0, dim()));
    const auto b = static_cast<std::size_t>(normalize_dim(d1, dim()));
    Shape shape = shape_;
    Strides strides = strides_;
    std::swap(shape[a], shape[b]);
    std::swap(strides[a], strides[b]);
    return reshaped(offset_, std::move(shape), std::move(strides));
}

Tensor Tensor::permute(const std::vector<int>& order) const {
    const int rank = dim();
    if (order.size() != static_cast<std::size_t>(rank)) {
        throw std::invalid_argument("permute: expected " + std::to_string(rank) +
                                    " dimensions, got " + std::to_string(order.size()));
    }
    Shape shape(order.size());
    Strides strides(order.size());
    std::vector<char> taken(order.size(), 0);
    for (std::size_t slot = 0; slot < order.size(); ++slot) {
        const int wanted = order[slot];
        const int source = wanted < 0 ? wanted + rank : wanted;
        if (source < 0 || source >= rank) {
            throw std::invalid_argument("permute: dimension " + std::to_string(wanted) +
                                        " is out of range for a " + std::to_string(rank) +
                                        "-d tensor");
        }
        if (taken[static_cast<std::size_t>(source)]++ != 0) {
            throw std::invalid_argument("permute: dimension " + std::to_string(wanted) +
                                        " appears more than once");
        }
        shape[slot] = shape_[static_cast<std::size_t>(source)];
        strides[slot] = strides_[static_cast<std::size_t>(source)];
    }
    return reshaped(offset_, std::move(shape), std::move(strides));
}

Tensor Tensor::slice(int d, std::int64_t start, std::int64_t end, std::int64_t step) const {
    const auto axis = static_cast<std::size_t>(normalize_dim(d, dim()));
    if (step < 1) {
        throw std::invalid_argument("slice: step must be >= 1");
    }
    // Python's rules: a negative bound counts from the end, then both are clamped to [0, n].
    const std::int64_t n = shape_[axis];
    const auto bound = [n](std::int64_t i) { return std::min(std::max(i < 0 ? i + n : i, std::int64_t{0}), n); };
    const std::int64_t first = bound(start);
    const std::int64_t stop = std::max(bound(end), first);
    Shape shape = shape_;
    Strides strides = strides_;
    shape[axis] = (stop - first + step - 1) / step;
    strides[axis] = strides_[axis] * step;
    return reshaped(offset_ + first * strides_[axis], std::move(shape), std::move(strides));
}

Tensor Tensor::expand(const Shape& shape) const {
    validate_shape(shape);
    return reshaped(offset_, shape, broadcast_strides(this->shape(), strides_, shape));
}

Tensor Tensor::unsqueeze(int d) const {
    // The new extent-1 dimension may also follow the last one: dim() + 1 positions.
    const int at = normalize_dim(d, dim() + 1);
    Shape shape = shape_;
    Strides strides = strides_;
    // Never stepped along; give it the stride a packed tensor would have there.
    const std::int64_t stride = at < dim() ? shape_[static_cast<std::size_t>(at)] *
                                                 strides_[static_cast<std::size_t>(at)]
                                           : 1;
    shape.insert(shape.begin() + at, 1);
    strides.insert(strides.begin() + at, stride);
    return reshaped(offset_, std::move(shape), std::move(strides));
}

Tensor Tensor::view(Shape shape) const {
    if (!is_contiguous()) {
        throw std::invalid_argument("view: tensor is not contiguous");
    }
    const auto holes = std::count(shape.begin(), shape.end(), std::int64_t{-1});
    if (holes > 1) {
        throw std::invalid_argument("view: only one dimension can be -1");
    }
    if (holes == 1) {
        std::int64_t known = 1;
        for (const std::int64_t extent : shape) {
            known *= extent == -1 ? 1 : extent;
        }
        if (known == 0 || numel() % known != 0) {
            throw std::invalid_argument("view: cannot infer -1 in " + to_string(shape) + " for " +
                                        std::to_string(numel()) + " elements");
        }
        *std::find(shape.begin(), shape.end(), std::int64_t{-1}) = numel() / known;
    }
    validate_shape(shape);
    if (mensurflow::numel(shape) != numel()) {
        throw std::invalid_argument("view: shape " + to_string(shape) + " does not match " +
                                    std::to_string(numel()) + " elements");
    }
    Strides strides = contiguous_strides(shape);
    return reshaped(offset_, std::move(shape), std::move(strides));
}

// ---- metadata -------------------------------------------------------------------------------------------

bool Tensor::shares_storage(const Tensor& other) const {
    return defined() && storage_ == other.storage_;
}

void Tensor::require_defined() const {
    if (storage_ == nullptr) {
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
