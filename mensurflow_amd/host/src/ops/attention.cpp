// Scaled dot-product attention (the reference's src/ops/attention.cpp:48-98). Where the execution
// device has a fused kernel (OpId::Attention) the op is one dispatch; a layout that kernel does
// not take (it throws NotImplemented), or a device without one, gets the reference's
// composition: a batched GEMM for the scaled scores, where() with -inf for masked positions,
// softmax over the keys, a batched GEMM with v.
#include "mensurflow/ops/attention.hpp"

#include "core/dispatcher.hpp"
#include "mensurflow/ops/blas.hpp"
#include "mensurflow/ops/elementwise.hpp"
#include "mensurflow/ops/softmax.hpp"

#include <cmath>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

namespace mensurflow {

namespace {

void require_operand(const Tensor& t, const char* name, const Tensor& q) {
    if (!t.defined()) {
        throw std::invalid_argument(std::string("attention: undefined ") + name);
    }
    if (t.dtype() != DType::F32) {
        throw std::invalid_argument(std::string("attention: ") + name + " must be F32, got " +
                                    dtype_name(t.dtype()));
    }
    if (t.dim() < 2) {
        throw std::invalid_argument(std::string("attention: ") + name +
                                    " needs at least 2 dimensions, got " + to_string(t.shape()));
    }
    if (t.device() != q.device()) {
        throw std::invalid_argument("attention: q, k and v must be on the same device");
    }
}

Shape batch_of(const Tensor& t) { return Shape(t.shape().begin(), t.shape().end() - 2); }

Shape with_matrix(Shape batch, std::int64_t rows, std::int64_t cols) {
    batch.push_back(rows);
    batch.push_back(cols);
    return batch;
}

// The fused kernel: q, k, v (and the mask) as views with the common batch shape. Returns an
// undefined tensor when the kernel does not take this layout.
Tensor fused_attention(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor* mask,
                       bool causal, float scale, Execution execution) {
    const Shape batch = broadcast_shapes(broadcast_shapes(batch_of(q), batch_of(k)), batch_of(v));
    const std::int64_t lq = q.size(-2), lk = k.size(-2), d = q.size(-1), dv = v.size(-1);
    detail::OpArgs args;
    args.inputs = {q.expand(with_matrix(batch, lq, d)), k.expand(with_matrix(batch, lk, d)),
                   v.expand(with_matrix(batch, lk, dv))};
    if (mask != nullptr) {
        args.inputs.push_back(mask->expand(with_matrix(batch, lq, lk)));
        args.has_mask = true;
    }
    args.outputs = {Tensor::empty(with_matrix(batch, lq, dv), DType::F32, q.device())};
    args.alpha = scale;
    args.causal = causal;
    try {
        detail::dispatch(detail::OpId::Attention, args, execution);
    } catch (const detail::NotImplemented&) {
        return Tensor();
    }
    return args.outputs[0];
}

Tensor masked(const Tensor& scores, const Tensor& keep, Execution execution) {
    const Tensor minus_infinity =
        Tensor::full({}, -std::numeric_limits<double>::infinity(), DType::F32, scores.device());
    return where(keep, scores, minus_infinity, execution);
}

} // namespace

Tensor attention(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor* mask, bool causal,
                 float scale, Execution execution) {
    require_operand(q, "q", q);
    require_operand(k, "k", q);
    require_operand(v, "v", q);
    const std::int64_t depth = q.size(-1);
    const std::int64_t queries = q.size(-2);
    const std::int64_t keys = k.size(-2);
    if (k.size(-1) != depth) {
        throw std::invalid_argument("attention: q " + to_string(q.shape()) + " and k " +
                                    to_string(k.shape()) + " differ in the last dimension");
    }
    if (v.size(-2) != keys) {
        throw std::invalid_argument("attention: k " + to_string(k.shape()) + " and v " +
                                    to_string(v.shape()) + " differ in the number of keys");
    }
    if (scale == 0.0f) {
        scale = depth > 0 ? static_cast<float>(1.0 / std::sqrt(static_cast<double>(depth))) : 1.0f;
    }
    Shape score_batch;
    try {
        score_batch = broadcast_shapes(batch_of(q), batch_of(k));
    } catch (const std::invalid_argument&) {
        throw std::invalid_argument("attention: batch shapes of q " + to_string(q.shape()) +
                                    " and k " + to_string(k.shape()) + " do not broadcast");
    }
    const Shape score_shape = with_matrix(score_batch, queries, keys);
    if (mask != nullptr) {
        if (!mask->defined() || mask->dtype() != DType::Bool) {
            throw std::invalid_argument("attention: mask must be a defined Bool tensor");
        }
        if (mask->device() != q.device()) {
            throw std::invalid_argument("attention: mask must be on the inputs' device");
        }
        bool fits = mask->dim() <= static_cast<int>(score_shape.size());
        if (fits) {
            try {
                fits = broadcast_shapes(mask->shape(), score_shape) == score_shape;
            } catch (const std::invalid_argument&) {
                fits = false;
            }
        }
        if (!fits) {
            throw std::invalid_argument("attention: mask " + to_string(mask->shape()) +
                                        " does not broadcast to the scores " +
                                        to_string(score_shape));
        }
    }
    if (detail::has_kernel_for(detail::OpId::Attention, execution, q.device())) {
        Tensor out = fused_attention(q, k, v, mask, causal, scale, execution);
        if (out.defined()) {
            return out;
        }
    }

    Tensor scores = gemm_strided_batched(q, k, scale, nullptr, 0.0f, false, true, execution);
    if (mask != nullptr) {
        scores = masked(scores, *mask, execution);
    }
    if (causal) {
        std::vector<std::uint8_t> keep(static_cast<std::size_t>(queries * keys));
        for (std::int64_t i = 0; i < queries; ++i) {
            for (std::int64_t j = 0; j < keys; ++j) {
                keep[static_cast<std::size_t>(i * keys + j)] = j <= i ? 1 : 0;
            }
        }
        const Tensor lower = Tensor::from_host(keep.data(), {queries, keys}, DType::Bool, q.device());
        scores = masked(scores, lower, execution);
    }
    const Tensor weights = softmax(scores, -1, execution);
    return gemm_strided_batched(weights, v, 1.0f, nullptr, 0.0f, false, false, execution);
}

} // namespace mensurflow
