// Elementwise ops of the hot path: validation, broadcasting by packing, dispatch (the
// reference's src/ops/elementwise.cpp:18,158,251,307,454 for unary_op, binary_op, bias_add,
// gelu and where).
#include "mensurflow/ops/elementwise.hpp"

#include "core/dispatcher.hpp"

#include <stdexcept>
#include <string>

namespace mensurflow {

namespace {

void require_compatible(const Tensor& a, const Tensor& b, const std::string& op) {
    if (!a.defined() || !b.defined()) {
        throw std::invalid_argument(op + ": undefined tensor");
    }
    if (a.dtype() != b.dtype()) {
        throw std::invalid_argument(op + ": dtypes differ (" + dtype_name(a.dtype()) + " and " +
                                    dtype_name(b.dtype()) + ")");
    }
    if (a.device() != b.device()) {
        throw std::invalid_argument(op + ": tensors are on " + to_string(a.device()) + " and " +
                                    to_string(b.device()) + "; move one with Tensor::to()");
    }
}

// An input smaller than the output, or not packed, becomes a contiguous tensor of `shape`.
Tensor packed(const Tensor& t, const Shape& shape) {
    return t.shape() == shape && t.is_contiguous() ? t : t.expand(shape).contiguous();
}

Tensor binary_op(detail::OpId op, const Tensor& a, const Tensor& b, Execution execution) {
    const std::string name = detail::op_name(op);
    require_compatible(a, b, name);
    Shape shape;
    try {
        shape = broadcast_shapes(a.shape(), b.shape());
    } catch (const std::invalid_argument& e) {
        throw std::invalid_argument(name + ": " + e.what());
    }
    Tensor out = Tensor::empty(shape, a.dtype(), a.device());
    if (numel(shape) == 0) {
        return out;
    }
    detail::dispatch(op, {{packed(a, shape), packed(b, shape)}, {out}}, execution);
    return out;
}

} // namespace

Tensor add(const Tensor& a, const Tensor& b, Execution execution) {
    return binary_op(detail::OpId::Add, a, b, execution);
}

Tensor mul(const Tensor& a, const Tensor& b, Execution execution) {
    return binary_op(detail::OpId::Mul, a, b, execution);
}

Tensor bias_add(const Tensor& x, const Tensor& bias, Execution execution) {
    require_compatible(x, bias, "bias_add");
    if (x.dim() != 2 || bias.dim() != 1) {
        throw std::invalid_argument("bias_add: expected [batch, features] and [features], got " +
                                    to_string(x.shape()) + " and " + to_string(bias.shape()));
    }
    if (x.size(1) != bias.size(0)) {
        throw std::invalid_argument("bias_add: bias length must match the matrix's feature count");
    }
    Tensor out = Tensor::empty(x.shape(), x.dtype(), x.device());
    detail::dispatch(detail::OpId::BiasAdd, {{x.contiguous(), bias.contiguous()}, {out}},
                     execution);
    return out;
}

Tensor gelu(const Tensor& x, bool approximate, Execution execution) {
    if (!x.defined()) {
        throw std::invalid_argument("gelu: undefined tensor");
    }
    Tensor out = Tensor::empty(x.shape(), x.dtype(), x.device());
    detail::OpArgs args{{x.contiguous()}, {out}};
    args.approximate = approximate;
    detail::dispatch(detail::OpId::Gelu, args, execution);
    return out;
}

Tensor where(const Tensor& condition, const Tensor& x, const Tensor& y, Execution execution) {
    require_compatible(x, y, "where");
    if (!condition.defined()) {
        throw std::invalid_argument("where: undefined condition tensor");
    }
    if (condition.dtype() != DType::Bool) {
        throw std::invalid_argument("where: condition must have Bool dtype");
    }
    if (condition.device() != x.device()) {
        throw std::invalid_argument("where: condition and values must be on the same device");
    }
    Shape shape;
    try {
        shape = broadcast_shapes(broadcast_shapes(x.shape(), y.shape()), condition.shape());
    } catch (const std::invalid_argument& e) {
        throw std::invalid_argument(std::string("where: ") + e.what());
    }
    Tensor out = Tensor::empty(shape, x.dtype(), x.device());
    // Values first, so the dispatch key is the values' dtype.
    detail::dispatch(detail::OpId::Where,
                     {{packed(x, shape), packed(y, shape), packed(condition, shape)}, {out}},
                     execution);
    return out;
}

} // namespace mensurflow
