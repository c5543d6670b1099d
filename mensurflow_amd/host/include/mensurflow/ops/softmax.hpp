// softmax along one axis (the reference's include/mensurflow/ops/softmax.hpp:20). A line whose
// elements are all -inf gives zeros; a NaN poisons its line.
#pragma once

#include "mensurflow/execution.hpp"
#include "mensurflow/tensor.hpp"

namespace mensurflow {

Tensor softmax(const Tensor& x, int axis = -1, Execution execution = Execution::Auto);

} // namespace mensurflow
