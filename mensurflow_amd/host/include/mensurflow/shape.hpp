// Shape and stride arithmetic (strides in elements, like the reference's shape.hpp).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace mensurflow {

using Shape = std::vector<std::int64_t>;
using Strides = std::vector<std::int64_t>;

// Throws invalid_argument for a negative dimension or an element count that overflows int64.
void validate_shape(const Shape& shape);

std::int64_t numel(const Shape& shape); // 1 for a scalar

Strides contiguous_strides(const Shape& shape);

// Row-major with no gaps; size-1 dimensions may have any stride; an empty tensor is contiguous.
bool is_contiguous(const Shape& shape, const Strides& strides);

// NumPy broadcasting; throws invalid_argument when the shapes do not broadcast.
Shape broadcast_shapes(const Shape& a, const Shape& b);

// Strides that show `shape` as the larger `target` (broadcast dimensions get stride 0).
Strides broadcast_strides(const Shape& shape, const Strides& strides, const Shape& target);

// A possibly negative dimension mapped into [0, ndim); throws out_of_range.
int normalize_dim(int dim, int ndim);

std::string to_string(const Shape& shape);

} // namespace mensurflow
