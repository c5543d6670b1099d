// Naive scaled dot-product attention (the reference's include/mensurflow/ops/attention.hpp:21):
// softmax(q k^T * scale, masked) v from gemm_strided_batched, where and softmax. q [..., Lq, D],
// k [..., Lk, D], v [..., Lk, Dv]; mask is an optional Bool tensor broadcast to [..., Lq, Lk]
// (true keeps); causal keeps keys 0..i for query i; scale 0 means 1/sqrt(D). A query with every
// key removed gets zeros.
#pragma once

#include "mensurflow/execution.hpp"
#include "mensurflow/tensor.hpp"

namespace mensurflow {

Tensor attention(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor* mask = nullptr,
                 bool causal = false, float scale = 0.0f, Execution execution = Execution::Auto);

} // namespace mensurflow
