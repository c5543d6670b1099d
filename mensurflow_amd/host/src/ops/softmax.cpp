// softmax: validation and dispatch (the reference's src/ops/softmax.cpp:35-69, forward only).
// argmax: last axis only (src/ops/reduction.cpp:164-190). uniform/normal: CPU factories
// (src/ops/random.cpp).
#include "mensurflow/ops/random.hpp"
#include "mensurflow/ops/reduction.hpp"
#include "mensurflow/ops/softmax.hpp"

#include "core/dispatcher.hpp"

#include <cmath>
#include <limits>
#include <stdexcept>
#include <string>

namespace mensurflow {

Tensor softmax(const Tensor& x, int axis, Execution execution) {
    if (!x.defined()) {
        throw std::invalid_argument("softmax: undefined input");
    }
    if (x.dtype() != DType::F32) {
        throw std::invalid_argument(std::string("softmax: input must be F32, got ") +
                                    dtype_name(x.dtype()));
    }
    const int extent = x.dim() == 0 ? 1 : x.dim();
    const int dim = axis < 0 ? axis + extent : axis;
    if (dim < 0 || dim >= extent) {
        throw std::invalid_argument("softmax: axis " + std::to_string(axis) +
                                    " is out of range for a " + std::to_string(x.dim()) +
                                    "-d tensor");
    }
    Tensor out = Tensor::empty(x.shape(), x.dtype(), x.device());
    detail::OpArgs args{{x.contiguous()}, {out}};
    args.axis = dim;
    detail::dispatch(detail::OpId::Softmax, args, execution);
    return out;
}

Tensor argmax(const Tensor& x, int axis, Execution execution) {
    if (!x.defined()) {
        throw std::invalid_argument("argmax: undefined tensor");
    }
    if (x.dim() == 0) {
        throw std::invalid_argument("argmax: input must have at least one dimension");
    }
    const int normalized = axis < 0 ? axis + x.dim() : axis;
    if (normalized != x.dim() - 1) {
        throw std::invalid_argument("argmax: only the last axis is supported");
    }
    if (x.size(-1) == 0) {
        throw std::invalid_argument("argmax: empty axis");
    }
    Shape shape(x.shape().begin(), x.shape().end() - 1);
    Tensor out = Tensor::empty(std::move(shape), DType::I64, x.device());
    detail::dispatch(detail::OpId::Argmax, {{x.contiguous()}, {out}}, execution);
    return out;
}

namespace {

Tensor random_op(detail::OpId op, Shape shape, float alpha, float beta, std::uint64_t seed,
                 std::uint64_t offset, Execution execution) {
    validate_shape(shape);
    const std::int64_t count = numel(shape);
    if (count > 0 &&
        static_cast<std::uint64_t>(count - 1) > std::numeric_limits<std::uint64_t>::max() - offset) {
        throw std::invalid_argument(std::string(detail::op_name(op)) +
                                    ": sample offset overflows uint64_t");
    }
    Tensor out = Tensor::empty(std::move(shape), DType::F32);
    detail::OpArgs args{{}, {out}};
    args.alpha = alpha;
    args.beta = beta;
    args.seed = seed;
    args.offset = offset;
    detail::dispatch(op, args, execution);
    return out;
}

} // namespace

Tensor uniform(Shape shape, float low, float high, std::uint64_t seed, std::uint64_t offset,
               Execution execution) {
    if (!std::isfinite(low) || !std::isfinite(high) || low > high) {
        throw std::invalid_argument("uniform: bounds must be finite and low <= high");
    }
    return random_op(detail::OpId::Uniform, std::move(shape), low, high, seed, offset, execution);
}

Tensor normal(Shape shape, float mean, float stddev, std::uint64_t seed, std::uint64_t offset,
              Execution execution) {
    if (!std::isfinite(mean) || !std::isfinite(stddev) || stddev < 0.0f) {
        throw std::invalid_argument("normal: mean and stddev must be finite, stddev >= 0");
    }
    return random_op(detail::OpId::Normal, std::move(shape), mean, stddev, seed, offset, execution);
}

} // namespace mensurflow
