// argmax along one axis (the reference's include/mensurflow/ops/reduction.hpp:45): the first
// index of the maximum; the first NaN wins. The result is I64 with the axis removed.
#pragma once

#include "mensurflow/execution.hpp"
#include "mensurflow/tensor.hpp"

namespace mensurflow {

Tensor argmax(const Tensor& x, int axis = -1, Execution execution = Execution::Auto);

} // namespace mensurflow
