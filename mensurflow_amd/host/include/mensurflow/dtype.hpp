// Element types. Kernels are registered per dtype; the hot path is F32 (with I64 indices from
// argmax and Bool masks for where/attention). Mirrors include/mensurflow/dtype.hpp of the
// reference (same enumerators and helpers).
#pragma once

#include <cstddef>
#include <cstdint>

namespace mensurflow {

enum class DType { F32, F16, BF16, I32, I64, U8, Bool };

// Bytes per element.
std::size_t dtype_size(DType dtype);

// "f32", "bf16", ...; throws invalid_argument for a value outside the enumeration.
const char* dtype_name(DType dtype);

bool is_floating_point(DType dtype);

template <typename T> struct DTypeOf;
template <> struct DTypeOf<float> { static constexpr DType value = DType::F32; };
template <> struct DTypeOf<std::int32_t> { static constexpr DType value = DType::I32; };
template <> struct DTypeOf<std::int64_t> { static constexpr DType value = DType::I64; };
template <> struct DTypeOf<std::uint8_t> { static constexpr DType value = DType::U8; };

template <typename T> inline constexpr DType dtype_of = DTypeOf<T>::value;

} // namespace mensurflow
