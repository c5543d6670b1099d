// Seeded factories (the reference's include/mensurflow/ops/random.hpp:20-26): Philox4x32-10,
// offset counts output elements. The result is a CPU tensor.
#pragma once

#include "mensurflow/execution.hpp"
#include "mensurflow/tensor.hpp"

#include <cstdint>

namespace mensurflow {

Tensor uniform(Shape shape, float low = 0.0f, float high = 1.0f, std::uint64_t seed = 0,
               std::uint64_t offset = 0, Execution execution = Execution::Auto);

Tensor normal(Shape shape, float mean = 0.0f, float stddev = 1.0f, std::uint64_t seed = 0,
              std::uint64_t offset = 0, Execution execution = Execution::Auto);

} // namespace mensurflow
