// BLAS operations of the hot path (the reference's include/mensurflow/ops/blas.hpp:17-77), plus
// one fused entry point. The last argument chooses where the op runs; results live on the
// inputs' device; a GPU call may return before the device finishes.
#pragma once

#include "mensurflow/execution.hpp"
#include "mensurflow/tensor.hpp"

namespace mensurflow {

// y[M] = a[M,K] x[K]. K == 0 gives zeros. Float32.
Tensor matvec(const Tensor& a, const Tensor& x, Execution execution = Execution::Auto);

// alpha * op(a) * x + beta * y; y optional (beta needs it).
Tensor gemv(const Tensor& a, const Tensor& x, float alpha = 1.0f, const Tensor* y = nullptr,
            float beta = 0.0f, bool transpose_a = false, Execution execution = Execution::Auto);

// c[M,N] = a[M,K] b[K,N]; strided views are accepted. K == 0 gives zeros.
Tensor matmul(const Tensor& a, const Tensor& b, Execution execution = Execution::Auto);

// alpha * op(a) * op(b) + beta * c. One fused dispatch (OpId::Gemm) on a device that has it;
// otherwise the reference's composition matmul -> mul(alpha) -> scal(beta) -> add.
Tensor gemm(const Tensor& a, const Tensor& b, float alpha = 1.0f, const Tensor* c = nullptr,
            float beta = 0.0f, bool transpose_a = false, bool transpose_b = false,
            Execution execution = Execution::Auto);

// Activation applied by gemm_epilogue after the bias.
enum class Activation { None, GeluTanh, Gelu };

// act(alpha * op(a) * op(b) + beta * c + bias), bias [N] broadcast over rows. The same result as
// the chain gelu(bias_add(gemm(...), bias), approximate) of the reference's ops, computed in one
// dispatch where the device has the fused kernel (ROCm), and as that chain elsewhere.
Tensor gemm_epilogue(const Tensor& a, const Tensor& b, const Tensor* bias,
                     Activation activation = Activation::None, float alpha = 1.0f,
                     const Tensor* c = nullptr, float beta = 0.0f, bool transpose_a = false,
                     bool transpose_b = false, Execution execution = Execution::Auto);

// alpha * op(a[i]) * op(b[i]) + beta * c[i] over NumPy-broadcast leading batch dimensions.
Tensor gemm_strided_batched(const Tensor& a, const Tensor& b, float alpha = 1.0f,
                            const Tensor* c = nullptr, float beta = 0.0f, bool transpose_a = false,
                            bool transpose_b = false, Execution execution = Execution::Auto);

// alpha * x for a vector x (a new contiguous tensor).
Tensor scal(float alpha, const Tensor& x, Execution execution = Execution::Auto);

// The 0-d sum of a[i] * b[i] over two vectors of one length (0 for empty ones).
Tensor dot(const Tensor& a, const Tensor& b, Execution execution = Execution::Auto);

} // namespace mensurflow
