// Elementwise ops of the hot path (the reference's include/mensurflow/ops/elementwise.hpp:43,
// 62,141 and the binary ops gemm's composition uses).
#pragma once

#include "mensurflow/execution.hpp"
#include "mensurflow/tensor.hpp"

namespace mensurflow {

// NumPy-broadcast a + b, a - b and a * b.
Tensor add(const Tensor& a, const Tensor& b, Execution execution = Execution::Auto);
Tensor sub(const Tensor& a, const Tensor& b, Execution execution = Execution::Auto);
Tensor mul(const Tensor& a, const Tensor& b, Execution execution = Execution::Auto);

// x[batch, features] + bias[features].
Tensor bias_add(const Tensor& x, const Tensor& bias, Execution execution = Execution::Auto);

// GELU; approximate = the tanh form.
Tensor gelu(const Tensor& x, bool approximate = false, Execution execution = Execution::Auto);

// condition ? x : y with NumPy broadcasting; condition is Bool.
Tensor where(const Tensor& condition, const Tensor& x, const Tensor& y,
             Execution execution = Execution::Auto);

} // namespace mensurflow
