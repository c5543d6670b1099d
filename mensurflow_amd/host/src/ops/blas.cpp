// BLAS ops of the hot path: checks, then one dispatch (mensurflow's src/ops/blas.cpp:119-394 for
// the checks, their order, the messages and the empty/zero-depth results). What this build adds:
//   - matmul passes strided views to ROCm kernels as it does to CPU ones (both read strides),
//     so a transposed device operand never goes through host memory;
//   - gemm is one OpId::Gemm dispatch where the execution device has that kernel, and
//     mensurflow's composition (matmul, mul by alpha, scal of c by beta, add) elsewhere, with the
//     same roundings either way;
//   - gemm_epilogue adds a bias and an activation to that one dispatch.
#include "mensurflow/ops/blas.hpp"

#include "core/dispatcher.hpp"
#include "mensurflow/ops/elementwise.hpp"
#include "ops/checks.hpp"

#include <stdexcept>
#include <string>

namespace mensurflow {

namespace {

using detail::OpArgs;
using detail::OpCheck;
using detail::OpId;

// Kernels of these devices read any strides with a unit step in one of the two matrix dimensions.
bool reads_views(Device device) {
    return device.type == DeviceType::CPU || device.type == DeviceType::ROCm;
}

// A vector as the kernels take it: unit stride.
Tensor unit_stride(const Tensor& v) { return v.strides()[0] == 1 ? v : v.contiguous(); }

// op(a) [m, k] and op(b) [k, n] as views, after the checks gemm and gemm_epilogue share.
struct Product {
    Tensor left, right;
    std::int64_t m = 0, n = 0, k = 0;
};

Product checked_product(const OpCheck& check, const Tensor& a, const Tensor& b, const Tensor* c,
                        float beta, bool transpose_a, bool transpose_b) {
    check.operand(a, "a", 2).operand(b, "b", 2);
    if (a.dtype() != b.dtype() || (c != nullptr && c->dtype() != a.dtype())) {
        check.fail("dtypes differ");
    }
    if (a.device() != b.device() || (c != nullptr && c->device() != a.device())) {
        check.fail("tensors are on different devices");
    }
    Product p;
    p.left = transpose_a ? a.transpose(0, 1) : a;
    p.right = transpose_b ? b.transpose(0, 1) : b;
    p.m = p.left.size(0);
    p.k = p.left.size(1);
    p.n = p.right.size(1);
    if (p.right.size(0) != p.k) {
        // mensurflow's gemm reports this from its inner matmul call.
        OpCheck("matmul").fail("inner dimensions differ (" + to_string(p.left.shape()) + " times " +
                               to_string(p.right.shape()) + ")");
    }
    if (c != nullptr && c->shape() != Shape{p.m, p.n}) {
        check.fail("c shape does not match result");
    }
    if (c == nullptr && beta != 0.0f) {
        check.fail("beta requires c");
    }
    return p;
}

// The single fused dispatch: inputs op(a), op(b), then c when beta != 0, then the bias.
Tensor fused(const Product& p, float alpha, const Tensor* c, float beta, const Tensor* bias,
             int activation, Execution execution) {
    Tensor out = Tensor::empty({p.m, p.n}, p.left.dtype(), p.left.device());
    if (out.numel() == 0) {
        return out;
    }
    OpArgs args{{p.left, p.right}, {out}};
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
    detail::dispatch(OpId::Gemm, args, execution);
    return out;
}

// mensurflow's gemm after the product: result * alpha (alpha != 1), + scal(beta, c) (beta != 0).
Tensor compose_alpha_beta(Tensor product, float alpha, const Tensor* c, float beta,
                          Execution execution) {
    if (alpha != 1.0f) {
        product = mul(product, Tensor::full({}, alpha, DType::F32, product.device()), execution);
    }
    if (c != nullptr && beta != 0.0f) {
        const Tensor scaled = scal(beta, c->contiguous().view({c->numel()}), execution);
        product = add(product, scaled.view(c->shape()), execution);
    }
    return product;
}

int activation_id(Activation activation) {
    switch (activation) {
    case Activation::None: return 0;
    case Activation::GeluTanh: return 1;
    case Activation::Gelu: return 2;
    }
    throw std::invalid_argument("gemm_epilogue: invalid activation");
}

} // namespace

Tensor scal(float alpha, const Tensor& x, Execution execution) {
    OpCheck("scal").operand(x, "x", 1);
    Tensor out = Tensor::empty(x.shape(), x.dtype(), x.device());
    if (x.size(0) > 0) {
        OpArgs args{{unit_stride(x)}, {out}};
        args.alpha = alpha;
        detail::dispatch(OpId::Scal, args, execution);
    }
    return out;
}

Tensor dot(const Tensor& a, const Tensor& b, Execution execution) {
    // The checks and messages of src/ops/blas.cpp:41-68.
    const OpCheck check("dot");
    check.operand(a, "a", 1).operand(b, "b", 1).same_dtype(a, b).same_device(a, b);
    if (a.size(0) != b.size(0)) {
        check.fail("lengths differ (" + std::to_string(a.size(0)) + " and " +
                   std::to_string(b.size(0)) + ")");
    }
    if (a.size(0) == 0) {
        return Tensor::zeros({}, a.dtype(), a.device()); // the sum of no products
    }
    Tensor out = Tensor::empty({}, a.dtype(), a.device());
    detail::dispatch(OpId::Dot, {{unit_stride(a), unit_stride(b)}, {out}}, execution);
    return out;
}

Tensor matvec(const Tensor& a, const Tensor& x, Execution execution) {
    const OpCheck check("matvec");
    check.operand(a, "a", 2).operand(x, "x", 1).same_dtype(a, x).same_device(a, x);
    const std::int64_t m = a.size(0), k = a.size(1);
    if (x.size(0) != k) {
        check.fail("inner dimensions differ (" + to_string(a.shape()) + " times " +
                   to_string(x.shape()) + ")");
    }
    if (m == 0) {
        return Tensor::empty({m}, a.dtype(), a.device());
    }
    if (k == 0) {
        return Tensor::zeros({m}, a.dtype(), a.device()); // an empty sum
    }
    Tensor out = Tensor::empty({m}, a.dtype(), a.device());
    detail::dispatch(OpId::Matvec, {{a.contiguous(), unit_stride(x)}, {out}}, execution);
    return out;
}

Tensor gemv(const Tensor& a, const Tensor& x, float alpha, const Tensor* y, float beta,
            bool transpose_a, Execution execution) {
    const OpCheck check("gemv");
    check.operand(a, "a", 2).operand(x, "x", 1);
    if (y == nullptr && beta != 0.0f) {
        check.fail("beta requires an output vector");
    }
    const bool dtypes_agree = a.dtype() == x.dtype() && (y == nullptr || y->dtype() == a.dtype());
    if (!dtypes_agree) {
        check.fail("dtypes differ");
    }
    const bool one_device = a.device() == x.device() && (y == nullptr || y->device() == a.device());
    if (!one_device) {
        check.fail("tensors must share a device");
    }
    const std::int64_t inputs = transpose_a ? a.size(0) : a.size(1);
    const std::int64_t outputs = transpose_a ? a.size(1) : a.size(0);
    if (x.size(0) != inputs) {
        check.fail("input length does not match matrix dimensions");
    }
    if (y != nullptr && y->size(0) != outputs) {
        check.fail("output length does not match matrix dimensions");
    }
    Tensor out = Tensor::empty({outputs}, a.dtype(), a.device());
    OpArgs args{{a.contiguous(), x.contiguous()}, {out}};
    if (y != nullptr) {
        args.inputs.push_back(y->contiguous());
    }
    args.alpha = alpha;
    args.beta = beta;
    args.transpose = transpose_a;
    detail::dispatch(OpId::Gemv, args, execution);
    return out;
}

Tensor matmul(const Tensor& a, const Tensor& b, Execution execution) {
    const OpCheck check("matmul");
    check.operand(a, "a", 2).operand(b, "b", 2).same_dtype(a, b).same_device(a, b);
    const std::int64_t m = a.size(0), k = a.size(1), n = b.size(1);
    if (b.size(0) != k) {
        check.fail("inner dimensions differ (" + to_string(a.shape()) + " times " +
                   to_string(b.shape()) + ")");
    }
    if (m == 0 || n == 0) {
        return Tensor::empty({m, n}, a.dtype(), a.device());
    }
    if (k == 0) {
        return Tensor::zeros({m, n}, a.dtype(), a.device());
    }
    const bool as_views = reads_views(a.device());
    const auto operand = [as_views](const Tensor& t) {
        return as_views || t.is_contiguous() ? t : t.contiguous();
    };
    Tensor out = Tensor::empty({m, n}, a.dtype(), a.device());
    detail::dispatch(OpId::Matmul, {{operand(a), operand(b)}, {out}}, execution);
    return out;
}

Tensor gemm(const Tensor& a, const Tensor& b, float alpha, const Tensor* c, float beta,
            bool transpose_a, bool transpose_b, Execution execution) {
    const Product p =
        checked_product(OpCheck("gemm"), a, b, c, beta, transpose_a, transpose_b);
    if (detail::has_kernel_for(OpId::Gemm, execution, a.device())) {
        return fused(p, alpha, c, beta, nullptr, 0, execution);
    }
    return compose_alpha_beta(matmul(p.left, p.right, execution), alpha, c, beta, execution);
}

Tensor gemm_epilogue(const Tensor& a, const Tensor& b, const Tensor* bias, Activation activation,
                     float alpha, const Tensor* c, float beta, bool transpose_a, bool transpose_b,
                     Execution execution) {
    const OpCheck check("gemm_epilogue");
    const Product p = checked_product(check, a, b, c, beta, transpose_a, transpose_b);
    const int act = activation_id(activation);
    if (bias != nullptr) {
        if (!bias->defined() || bias->dim() != 1 || bias->size(0) != p.n) {
            check.fail("bias must be [n]");
        }
        if (bias->dtype() != a.dtype() || bias->device() != a.device()) {
            check.fail("bias dtype or device differs");
        }
    }
    if (detail::has_kernel_for(OpId::Gemm, execution, a.device())) {
        return fused(p, alpha, c, beta, bias, act, execution);
    }
    // Elsewhere: the chain of mensurflow ops the fused call stands for.
    Tensor result =
        compose_alpha_beta(matmul(p.left, p.right, execution), alpha, c, beta, execution);
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
    const OpCheck check("gemm_strided_batched");
    check.operand(a, "a", 2, true).operand(b, "b", 2, true);
    if (a.dtype() != b.dtype() || (c != nullptr && c->dtype() != a.dtype())) {
        check.fail("dtypes differ");
    }
    if (a.device() != b.device() || (c != nullptr && c->device() != a.device())) {
        check.fail("tensors are on different devices; move one with Tensor::to()");
    }
    if (c == nullptr && beta != 0.0f) {
        check.fail("beta requires c");
    }
    // op() only swaps the last two extents and strides.
    const Tensor left = transpose_a ? a.transpose(-2, -1) : a;
    const Tensor right = transpose_b ? b.transpose(-2, -1) : b;
    const std::int64_t m = left.size(-2), k = left.size(-1), n = right.size(-1);
    if (right.size(-2) != k) {
        check.fail("inner dimensions differ (" + to_string(left.shape()) + " times " +
                   to_string(right.shape()) + ")");
    }
    const auto batch_of = [](const Tensor& t) { return Shape(t.shape().begin(), t.shape().end() - 2); };
    const auto with_matrix = [](Shape shape, std::int64_t rows, std::int64_t cols) {
        shape.push_back(rows);
        shape.push_back(cols);
        return shape;
    };
    Shape batch;
    try {
        batch = broadcast_shapes(batch_of(left), batch_of(right));
    } catch (const std::invalid_argument&) {
        check.fail("batch shapes " + to_string(batch_of(left)) + " and " +
                   to_string(batch_of(right)) + " do not broadcast");
    }
    const Shape out_shape = with_matrix(batch, m, n);
    // c broadcasts to the result (one C0 shared by the batch costs no copy of its own) and is
    // packed in the result's layout when it is read at all.
    Tensor initial;
    if (c != nullptr) {
        if (!detail::broadcasts_to(c->shape(), out_shape)) {
            check.fail("c has shape " + to_string(c->shape()) + ", which does not broadcast to " +
                       to_string(out_shape));
        }
        if (beta != 0.0f) {
            initial = c->expand(out_shape).contiguous();
        }
    }
    if (numel(out_shape) == 0) {
        return Tensor::empty(out_shape, a.dtype(), a.device());
    }
    if (k == 0) {
        // No products: beta * c, or zeros.
        return initial.defined()
                   ? scal(beta, initial.view({initial.numel()}), execution).view(out_shape)
                   : Tensor::zeros(out_shape, a.dtype(), a.device());
    }
    // Every matrix as a view with the full batch shape: broadcast dimensions get stride 0.
    Tensor out = Tensor::empty(out_shape, a.dtype(), a.device());
    OpArgs args{{left.expand(with_matrix(batch, m, k)), right.expand(with_matrix(batch, k, n))},
                {out}};
    if (initial.defined()) {
        args.inputs.push_back(initial);
    }
    args.alpha = alpha;
    args.beta = initial.defined() ? beta : 0.0f;
    detail::dispatch(OpId::GemmBatched, args, execution);
    return out;
}

} // namespace mensurflow
