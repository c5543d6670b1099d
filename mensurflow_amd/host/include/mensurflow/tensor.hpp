// Tensor: an element type, a shape and strides over memory shared with other views. The public
// calls are mensurflow's (include/mensurflow/tensor.hpp:25-162) minus autograd, which is not on
// this backend's path. Copying a Tensor copies the view, not the memory.
#pragma once

#include "mensurflow/device.hpp"
#include "mensurflow/dtype.hpp"
#include "mensurflow/shape.hpp"

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace mensurflow {

namespace detail {
struct Storage;
struct TensorAccess;
} // namespace detail

class Tensor {
  public:
    Tensor() = default; // undefined; any use but defined() throws logic_error

    // New memory on `device` (the CPU unless given); runtime_error when it is not available.
    static Tensor empty(Shape shape, DType dtype = DType::F32, Device device = {});
    static Tensor constant(Shape shape, double value, DType dtype = DType::F32, Device device = {});
    static Tensor zeros(Shape shape, DType dtype = DType::F32, Device device = {});
    static Tensor ones(Shape shape, DType dtype = DType::F32, Device device = {});
    static Tensor full(Shape shape, double value, DType dtype = DType::F32, Device device = {});
    static Tensor eye(std::int64_t n, DType dtype = DType::F32, Device device = {});
    static Tensor zeros_like(const Tensor& other);
    static Tensor ones_like(const Tensor& other);
    static Tensor full_like(const Tensor& other, double value);

    // A new tensor holding numel(shape) elements read from contiguous host memory at `data`.
    static Tensor from_host(const void* data, Shape shape, DType dtype, Device device = {});

    template <typename T>
    static Tensor from_vector(const std::vector<T>& data, Shape shape, Device device = {}) {
        validate_shape(shape);
        if (static_cast<std::int64_t>(data.size()) != mensurflow::numel(shape)) {
            throw std::invalid_argument("from_vector: " + std::to_string(data.size()) +
                                        " values do not fill shape " + to_string(shape));
        }
        return from_host(data.data(), std::move(shape), dtype_of<T>, device);
    }

    // Views over the same memory.
    Tensor transpose(int d0, int d1) const;
    Tensor permute(const std::vector<int>& order) const;
    Tensor slice(int d, std::int64_t start, std::int64_t end, std::int64_t step = 1) const;
    Tensor expand(const Shape& shape) const;
    Tensor unsqueeze(int d) const;
    Tensor view(Shape shape) const; // of a contiguous tensor; at most one extent may be -1

    bool shares_storage(const Tensor& other) const;

    // A contiguous copy on `device`, or *this when the tensor already lives there.
    Tensor to(Device device) const;

    // *this when contiguous, else a packed copy on the same device. A device whose backend has a
    // strided-copy kernel (ROCm) packs there; others pack through host memory, as mensurflow does
    // (src/core/tensor.cpp:208-230).
    Tensor contiguous() const;

    // Overwrites this view's elements with `source`'s (same shape, dtype and device).
    void copy_from(const Tensor& source);

    // The elements in row-major order into `dst`; waits for queued device work.
    void copy_to_host(void* dst) const;

    template <typename T> T item() const {
        if (numel() != 1) {
            throw std::invalid_argument("item: tensor has " + std::to_string(numel()) +
                                        " elements, expected 1");
        }
        return to_vector<T>()[0];
    }

    template <typename T> std::vector<T> to_vector() const {
        if (dtype() != dtype_of<T>) {
            throw std::invalid_argument(std::string("to_vector: tensor is ") + dtype_name(dtype()) +
                                        ", requested " + dtype_name(dtype_of<T>));
        }
        std::vector<T> out(static_cast<std::size_t>(numel()));
        copy_to_host(out.data());
        return out;
    }

    bool defined() const { return storage_ != nullptr; }
    const Shape& shape() const;
    const Strides& strides() const;
    std::int64_t offset() const; // in elements, from the start of the memory
    DType dtype() const;
    Device device() const;
    int dim() const;
    std::int64_t size(int d) const; // d may count from the end (-1 = last)
    std::int64_t numel() const;
    std::size_t itemsize() const;
    std::size_t nbytes() const;
    bool is_contiguous() const;

  private:
    friend struct detail::TensorAccess;

    Tensor(std::shared_ptr<detail::Storage> storage, std::int64_t offset, Shape shape,
           Strides strides, DType dtype);

    void require_defined() const;
    Tensor reshaped(std::int64_t offset, Shape shape, Strides strides) const;

    std::shared_ptr<detail::Storage> storage_;
    std::int64_t offset_ = 0;
    Shape shape_;
    Strides strides_;
    DType dtype_ = DType::F32;
};

} // namespace mensurflow
