// Elementwise ops of the hot path: add and mul (used by gemm's unfused composition), sub (the
// third binary op the reference's CUDA backend serves), bias_add, gelu and where. Checks, messages and broadcasting rules are mensurflow's
// (src/ops/elementwise.cpp:18,140-201,251-309,454-481). Operands that broadcast, or are not
// packed, become packed tensors of the output's shape before the kernel sees them, except where a
// device's where kernel reads broadcast views itself (ROCm), which saves materializing them.
#include "mensurflow/ops/elementwise.hpp"

#include "core/dispatcher.hpp"
#include "ops/checks.hpp"
#include "ops/where_into.hpp"

#include <string>

namespace mensurflow {

namespace {

using detail::OpArgs;
using detail::OpCheck;
using detail::OpId;

// `t` as a packed tensor of `shape` (itself when it already is one).
Tensor packed_as(const Tensor& t, const Shape& shape) {
    return t.shape() == shape && t.is_contiguous() ? t : t.expand(shape).contiguous();
}

Tensor pairwise(OpId op, const Tensor& a, const Tensor& b, Execution execution) {
    const OpCheck check(detail::op_name(op));
    check.compatible(a, b);
    const Shape shape = detail::broadcast_for(check, a.shape(), b.shape());
    Tensor out = Tensor::empty(shape, a.dtype(), a.device());
    if (out.numel() > 0) {
        detail::dispatch(op, {{packed_as(a, shape), packed_as(b, shape)}, {out}}, execution);
    }
    return out;
}

// Devices whose where kernel reads its operands through strides (stride 0 for a broadcast
// dimension), so broadcast operands need no packed copy.
bool where_reads_views(Device device) { return device.type == DeviceType::ROCm; }

} // namespace

Tensor add(const Tensor& a, const Tensor& b, Execution execution) {
    return pairwise(OpId::Add, a, b, execution);
}

Tensor sub(const Tensor& a, const Tensor& b, Execution execution) {
    return pairwise(OpId::Sub, a, b, execution);
}

Tensor mul(const Tensor& a, const Tensor& b, Execution execution) {
    return pairwise(OpId::Mul, a, b, execution);
}

Tensor bias_add(const Tensor& x, const Tensor& bias, Execution execution) {
    const OpCheck check("bias_add");
    check.compatible(x, bias);
    if (x.dim() != 2 || bias.dim() != 1) {
        check.fail("expected [batch, features] and [features], got " + to_string(x.shape()) +
                   " and " + to_string(bias.shape()));
    }
    if (x.size(1) != bias.size(0)) {
        check.fail("bias length must match the matrix's feature count");
    }
    Tensor out = Tensor::empty(x.shape(), x.dtype(), x.device());
    detail::dispatch(OpId::BiasAdd, {{x.contiguous(), bias.contiguous()}, {out}}, execution);
    return out;
}

Tensor gelu(const Tensor& x, bool approximate, Execution execution) {
    if (!x.defined()) {
        OpCheck("gelu").fail("undefined tensor");
    }
    Tensor out = Tensor::empty(x.shape(), x.dtype(), x.device());
    OpArgs args{{x.contiguous()}, {out}};
    args.approximate = approximate;
    detail::dispatch(OpId::Gelu, args, execution);
    return out;
}

namespace {

// where()'s checks; the shape its operands broadcast to.
Shape where_shape(const Tensor& condition, const Tensor& x, const Tensor& y) {
    const OpCheck check("where");
    check.compatible(x, y);
    if (!condition.defined()) {
        check.fail("undefined condition tensor");
    }
    if (condition.dtype() != DType::Bool) {
        check.fail("condition must have Bool dtype");
    }
    if (condition.device() != x.device()) {
        check.fail("condition and values must be on the same device");
    }
    return detail::broadcast_for(check, detail::broadcast_for(check, x.shape(), y.shape()),
                                 condition.shape());
}

} // namespace

namespace detail {

void where_into(const Tensor& condition, const Tensor& x, const Tensor& y, const Tensor& out,
                Execution execution) {
    const Shape shape = where_shape(condition, x, y);
    if (!out.defined() || out.shape() != shape || out.dtype() != x.dtype() ||
        out.device() != x.device() || !out.is_contiguous()) {
        OpCheck("where").fail("output must be a packed " + std::string(dtype_name(x.dtype())) +
                              " tensor of shape " + to_string(shape) + " on the inputs' device");
    }
    const bool as_views =
        where_reads_views(x.device()) && has_kernel_for(OpId::Where, execution, x.device());
    const auto operand = [&](const Tensor& t) {
        return as_views ? t.expand(shape) : packed_as(t, shape);
    };
    // The values come first: the kernel is keyed by their dtype, not the condition's.
    dispatch(OpId::Where, {{operand(x), operand(y), operand(condition)}, {out}}, execution);
}

} // namespace detail

Tensor where(const Tensor& condition, const Tensor& x, const Tensor& y, Execution execution) {
    const Shape shape = where_shape(condition, x, y);
    Tensor out = Tensor::empty(shape, x.dtype(), x.device());
    detail::where_into(condition, x, y, out, execution);
    return out;
}

} // namespace mensurflow
