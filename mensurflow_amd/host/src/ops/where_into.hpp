// where() into a given output: the op's checks and operand handling, with `out` supplied by the
// caller (it may be x or y itself). Used by where(), which allocates out, and by attention's
// composition, which masks its own temporary scores in place.
#pragma once

#include "mensurflow/tensor.hpp"

namespace mensurflow::detail {

// out: F32, on x's device, of the shape cond, x and y broadcast to.
void where_into(const Tensor& condition, const Tensor& x, const Tensor& y, const Tensor& out,
                Execution execution);

} // namespace mensurflow::detail
