// BLAS ops: validation, then dispatch (the reference's src/ops/blas.cpp:119-394, same checks and
// error types). Differences, all additive:
//   - matmul hands strided views to ROCm kernels as well as CPU ones (both read strides), so a
//     transposed device operand is never staged through the host;
//   - gemm issues one OpId::Gemm dispatch where the execution device has that kernel, and the
//     reference's matmul -> mul -> scal -> add composition elsewhere (same roundings);
//   - gemm_epilogue adds a bias and an activation to that fused dispatch.
#include "mensurflow/ops/blas.hpp"

#include "core/dispatcher.hpp"
#include "core/registry.hpp"
#include "mensurflow/ops/elementwise.hpp"

#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace mensurflow {

namespace {

void require_vector(const Tensor& t, const char* op, const char* name) {
    if (!t.defined()) {
        throw std::invalid_argument(std::string(op) + ": " + name + " is an undefined tensor");
    }
    if (t.dim() != 1) {
        throw std::invalid_argument(std::string(op) + ": " + name + " must be 1-D, got shape " +
                                    to_string(t.shape()));
    }
}

void require_matrix(const Tensor& t, const char* op, const char* name) {
    if (!t.defined()) {
        throw std::invalid_argument(std::string(op) + ": " + name + " is an undefined tensor");
    }
    if (t.dim() != 2) {
        throw std::invalid_argument(std::string(op) + ": " + name + " must be 2-D, got shape " +
                                    to_string(t.shape()));
    }
}

// Whether the kernels of `device` read arbitrary strides (a unit stride in one dimension).
bool reads_strides(Device device) {
    return device.type == DeviceType::CPU || device.type == DeviceType::ROCm;
}

int activation_code(Activation activation) {
    switch (activation) {
    case Activation::None: return 0;
    case Activation::GeluTanh: return 1;
    case Activation::Gelu: return 2;
    }
    throw std::invalid_argument("gemm_epilogue: invalid activation");
}

struct GemmOperands {
    Tensor left, right;
    std::int64_t m, n, k;
};

GemmOperands gemm_operands(const Tensor& a, const Tensor& b, const Tensor* c, float beta,
                           bool transpose_a, bool transpose_b, const char* name) {
    require_matrix(a, name, "a");
    require_matrix(b, name, "b");
    if (a.dtype() != b.dtype() || (c != nullptr && c->dtype() != a.dtype())) {
        throw std::invalid_argument(std::string(name) + ": dtypes differ");
    }
    if (a.device() != b.device() || (c != nullptr && c->device() != a.device())) {
        throw std::invalid_argument(std::string(name) + ": tensors are on different devices");
    }
    GemmOperands g;
    g.left = transpose_a ? a.transpose(0, 1) : a;
    g.right = transpose_b ? b.transpose(0, 1) : b;
    g.m = g.left.size(0);
    g.k = g.left.size(1);
    g.n = g.right.size(1);
    if (g.right.size(0) != g.k) {
        throw std::invalid_argument(std::string(name) + ": inner dimensions differ (" +
                                    to_string(g.left.shape()) + " times " +
                                    to_string(g.right.shape()) + ")");
    }
    if (c != nullptr && c->shape() != Shape{g.m, g.n}) {
        throw std::invalid_argument(std::string(name) + ": c shape does not match result");
    }
    if (c == nullptr && beta != 0.0f) {
        throw std::invalid_argument(std::string(name) + ": beta requires c");
    }
    return g;
}

// One fused dispatch: op(a), op(b) as views, then c (when beta != 0) and bias.
Tensor fused_gemm(const GemmOperands& g, const Tensor* bias, int activation, float alpha,
                  const Tensor* c, float beta, Execution execution) {
    Tensor out = Tensor::empty({g.m, g.n}, g.left.dtype(), g.left.device());
    if (g.m == 0 || g.n == 0) {
        return out;
    }
    detail::OpArgs args{{g.left, g.right}, {out}};
    args.alpha = alpha;
    args.beta = 0.0f;
    if (c != nullptr && beta != 0.0f) {
        args.inputs.push_back(c->contiguous());
        args.beta = beta;
    }
    if (bias != nullptr) {
        args.inputs.push_back(bias->contiguous());
        args.has_bias = true;
    }
    args.activation = activation;
    detail::dispatch(detail::OpId::Gemm, args, execution);
    return out;
}

} // namespace

Tensor scal(float alpha, const Tensor& x, Execution execution) {
    require_vector(x, "scal", "x");
    Tensor out = Tensor::empty(x.shape(), x.dtype(), x.device());
    if (x.size(0) == 0) {
        return out;
    }
    const Tensor input = x.strides()[0] == 1 ? x : x.contiguous();
    detail::OpArgs args{{input}, {out}};
    args.alpha = alpha;
    detail::dispatch(detail::OpId::Scal, args, execution);
    return out;
}

Tensor matvec(const Tensor& a, const Tensor& x, Execution execution) {
    require_matrix(a, "matvec", "a");
    require_vector(x, "matvec", "x");
    if (a.dtype() != x.dtype()) {
        throw std::invalid_argument(std::string("matvec: dtypes differ (") + dtype_name(a.dtype()) +
                                    " and " + dtype_name(x.dtype()) + ")");
    }
    if (a.device() != x.device()) {
        throw std::invalid_argument("matvec: tensors are on " + to_string(a.device()) + " and " +
                                    to_string(x.device()) + "; move one with Tensor::to()");
    }
    const std::int64_t m = a.size(0), k = a.size(1);
    if (x.size(0) != k) {
        throw std::invalid_argument("matvec: inner dimensions differ (" + to_string(a.shape()) +
                                    " times " + to_string(x.shape()) + ")");
    }
    Tensor out = Tensor::empty({m}, a.dtype(), a.device());
    if (m == 0) {
        return out;
    }
    if (k == 0) {
        return Tensor::zeros({m}, a.dtype(), a.device());
    }
    const Tensor matrix = a.is_contiguous() ? a : a.contiguous();
    const Tensor vector = x.strides()[0] == 1 ? x : x.contiguous();
    detail::dispatch(detail::OpId::Matvec, {{matrix, vector}, {out}}, execution);
    return out;
}

Tensor gemv(const Tensor& a, const Tensor& x, float alpha, const Tensor* y, float beta,
            bool transpose_a, Execution execution) {
    require_matrix(a, "gemv", "a");
    require_vector(x, "gemv", "x");
    if (y == nullptr && beta != 0.0f) {
        throw std::invalid_argument("gemv: beta requires an output vector");
    }
    if (a.dtype() != x.dtype() || (y != nullptr && a.dtype() != y->dtype())) {
        throw std::invalid_argument("gemv: dtypes differ");
    }
    if (a.device() != x.device() || (y != nullptr && a.device() != y->device())) {
        throw std::invalid_argument("gemv: tensors must share a device");
    }
    const std::int64_t rows = a.size(0), cols = a.size(1);
    const std::int64_t input = transpose_a ? rows : cols;
    const std::int64_t output = transpose_a ? cols : rows;
    if (x.size(0) != input) {
        throw std::invalid_argument("gemv: input length does not match matrix dimensions");
    }
    if (y != nullptr && y->size(0) != output) {
        throw std::invalid_argument("gemv: output length does not match matrix dimensions");
    }
    Tensor out = Tensor::empty({output}, a.dtype(), a.device());
    detail::OpArgs args{{a.contiguous(), x.contiguous()}, {out}};
    if (y != nullptr) {
        args.inputs.push_back(y->contiguous());
    }
    args.alpha = alpha;
    args.beta = beta;
    args.transpose = transpose_a;
    detail::dispatch(detail::OpId::Gemv, args, execution);
    return out;
}

Tensor matmul(const Tensor& a, const Tensor& b, Execution execution) {
    require_matrix(a, "matmul", "a");
    require_matrix(b, "matmul", "b");
    if (a.dtype() != b.dtype()) {
        throw std::invalid_argument(std::string("matmul: dtypes differ (") + dtype_name(a.dtype()) +
                                    " and " + dtype_name(b.dtype()) + ")");
    }
    if (a.device() != b.device()) {
        throw std::invalid_argument("matmul: tensors are on " + to_string(a.device()) + " and " +
                                    to_string(b.device()) + "; move one with Tensor::to()");
    }
    const std::int64_t m = a.size(0), k = a.size(1), n = b.size(1);
    if (b.size(0) != k) {
        throw std::invalid_argument("matmul: inner dimensions differ (" + to_string(a.shape()) +
                                    " times " + to_string(b.shape()) + ")");
    }
    Tensor out = Tensor::empty({m, n}, a.dtype(), a.device());
    if (m == 0 || n == 0) {
        return out;
    }
    if (k == 0) {
        return Tensor::zeros({m, n}, a.dtype(), a.device());
    }
    const bool strided_ok = reads_strides(a.device());
    const Tensor x = strided_ok || a.is_contiguous() ? a : a.contiguous();
    const Tensor y = strided_ok || b.is_contiguous() ? b : b.contiguous();
    detail::dispatch(detail::OpId::Matmul, {{x, y}, {out}}, execution);
    return out;
}

Tensor gemm(const Tensor& a, const Tensor& b, float alpha, const Tensor* c, float beta,
            bool transpose_a, bool transpose_b, Execution execution) {
    const GemmOperands g = gemm_operands(a, b, c, beta, transpose_a, transpose_b, "gemm");
    if (detail::has_kernel_for(detail::OpId::Gemm, execution, a.device())) {
        return fused_gemm(g, nullptr, 0, alpha, c, beta, execution);
    }
    // The reference's composition (src/ops/blas.cpp:244-261).
    Tensor result = matmul(g.left, g.right, execution);
    if (alpha != 1.0f) {
        result = mul(result, Tensor::full({}, alpha, DType::F32, result.device()), execution);
    }
    if (c != nullptr && beta != 0.0f) {
        result = add(result, scal(beta, c->contiguous().view({c->numel()}), execution)
                                 .view(c->shape()),
                     execution);
    }
    return result;
}

Tensor gemm_epilogue(const Tensor& a, const Tensor& b, const Tensor* bias, Activation activation,
                     float alpha, const Tensor* c, float beta, bool transpose_a, bool transpose_b,
                     Execution execution) {
    const GemmOperands g =
        gemm_operands(a, b, c, beta, transpose_a, transpose_b, "gemm_epilogue");
    const int act = activation_code(activation);
    if (bias != nullptr) {
        if (!bias->defined() || bias->dim() != 1 || bias->size(0) != g.n) {
            throw std::invalid_argument("gemm_epilogue: bias must be [n]");
        }
        if (bias->dtype() != a.dtype() || bias->device() != a.device()) {
            throw std::invalid_argument("gemm_epilogue: bias dtype or device differs");
        }
    }
    if (detail::has_kernel_for(detail::OpId::Gemm, execution, a.device())) {
        return fused_gemm(g, bias, act, alpha, c, beta, execution);
    }
    Tensor result = gemm(a, b, alpha, c, beta, transpose_a, transpose_b, execution);
    if (bias != nullptr) {
        result = bias_add(result, *bias, execution);
    }
    if (activation != Activation::None) {
        result = gelu(result, activation == Activation::GeluTanh, execution);
    }
    return result;
}

Tensor gemm_strided_batched(const Tensor& a, const Tensor& b, float alpha, const Tensor* c,
                            float beta, bool transpose_a, bool transpose_b, Execution execution) {
    for (const auto& [t, name] : {std::pair<const Tensor*, const char*>{&a, "a"}, {&b, "b"}}) {
        if (!t->defined()) {
            throw std::invalid_argument(std::string("gemm_strided_batched: ") + name +
                                        " is an undefined tensor");
        }
        if (t->dim() < 2) {
            throw std::invalid_argument(std::string("gemm_strided_batched: ") + name +
                                        " must be at least 2-D, got shape " +
                                        to_string(t->shape()));
        }
    }
    if (a.dtype() != b.dtype() || (c != nullptr && c->dtype() != a.dtype())) {
        throw std::invalid_argument("gemm_strided_batched: dtypes differ");
    }
    if (a.device() != b.device() || (c != nullptr && c->device() != a.device())) {
        throw std::invalid_argument("gemm_strided_batched: tensors are on different devices; move "
                                    "one with Tensor::to()");
    }
    if (c == nullptr && beta != 0.0f) {
        throw std::invalid_argument("gemm_strided_batched: beta requires c");
    }
    const Tensor left = transpose_a ? a.transpose(-2, -1) : a;
    const Tensor right = transpose_b ? b.transpose(-2, -1) : b;
    const std::int64_t m = left.size(-2), k = left.size(-1), n = right.size(-1);
    if (right.size(-2) != k) {
        throw std::invalid_argument("gemm_strided_batched: inner dimensions differ (" +
                                    to_string(left.shape()) + " times " + to_string(right.shape()) +
                                    ")");
    }
    const Shape left_batch(left.shape().begin(), left.shape().end() - 2);
    const Shape right_batch(right.shape().begin(), right.shape().end() - 2);
    Shape batch;
    try {
        batch = broadcast_shapes(left_batch, right_batch);
    } catch (const std::invalid_argument&) {
        throw std::invalid_argument("gemm_strided_batched: batch shapes " + to_string(left_batch) +
                                    " and " + to_string(right_batch) + " do not broadcast");
    }
    Shape out_shape = batch;
    out_shape.push_back(m);
    out_shape.push_back(n);
    Tensor initial;
    if (c != nullptr) {
        bool broadcasts = c->dim() <= static_cast<int>(out_shape.size());
        if (broadcasts) {
            try {
                broadcasts = broadcast_shapes(c->shape(), out_shape) == out_shape;
            } catch (const std::invalid_argument&) {
                broadcasts = false;
            }
        }
        if (!broadcasts) {
            throw std::invalid_argument("gemm_strided_batched: c has shape " +
                                        to_string(c->shape()) + ", which does not broadcast to " +
                                        to_string(out_shape));
        }
        if (beta != 0.0f) {
            initial = c->expand(out_shape).contiguous();
        }
    }
    Tensor out = Tensor::empty(out_shape, a.dtype(), a.device());
    if (out.numel() == 0) {
        return out;
    }
    if (k == 0) {
        if (initial.defined()) {
            return scal(beta, initial.view({initial.numel()}), execution).view(out_shape);
        }
        return Tensor::zeros(out_shape, a.dtype(), a.device());
    }
    Shape left_shape = batch;
    left_shape.push_back(m);
    left_shape.push_back(k);
    Shape right_shape = batch;
    right_shape.push_back(k);
    right_shape.push_back(n);
    detail::OpArgs args{{left.expand(left_shape), right.expand(right_shape)}, {out}};
    if (initial.defined()) {
        args.inputs.push_back(initial);
    }
    args.alpha = alpha;
    args.beta = initial.defined() ? beta : 0.0f;
    detail::dispatch(detail::OpId::GemmBatched, args, execution);
    return out;
}

} // namespace mensurflow
