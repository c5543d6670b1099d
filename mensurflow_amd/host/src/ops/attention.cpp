// Scaled dot-product attention (mensurflow's src/ops/attention.cpp:48-98: checks, messages, the
// default scale, top-left causal masking, zeros for a query that keeps no key). Where the
// execution device has a fused kernel (OpId::Attention) the op is that one dispatch; a layout the
// kernel does not take (it throws NotImplemented), or a device without one, runs mensurflow's
// composition: a batched GEMM for the scaled scores, where() with -inf for removed keys, softmax
// over the keys, and a batched GEMM with v. On ROCm the causal -inf comes from the scores GEMM
// itself where it takes it (the same bits, without a pass over the scores).
#include "mensurflow/ops/attention.hpp"

#include "core/dispatcher.hpp"
#include "mensurflow/ops/blas.hpp"
#include "mensurflow/ops/elementwise.hpp"
#include "mensurflow/ops/softmax.hpp"
#include "ops/checks.hpp"
#include "ops/where_into.hpp"

#include <algorithm>
#include <cmath>
#include <limits>
#include <string>
#include <vector>

namespace mensurflow {

namespace {

using detail::OpArgs;
using detail::OpCheck;
using detail::OpId;

const OpCheck kCheck("attention");

void check_operand(const Tensor& t, const char* name, const Tensor& q) {
    if (!t.defined()) {
        kCheck.fail(std::string("undefined ") + name);
    }
    if (t.dtype() != DType::F32) {
        kCheck.fail(std::string(name) + " must be F32, got " + dtype_name(t.dtype()));
    }
    if (t.dim() < 2) {
        kCheck.fail(std::string(name) + " needs at least 2 dimensions, got " +
                    to_string(t.shape()));
    }
    if (t.device() != q.device()) {
        kCheck.fail("q, k and v must be on the same device");
    }
}

Shape leading(const Tensor& t) { return Shape(t.shape().begin(), t.shape().end() - 2); }

Shape matrix_shape(Shape batch, std::int64_t rows, std::int64_t cols) {
    batch.insert(batch.end(), {rows, cols});
    return batch;
}

// The fused kernel, with q, k, v (and the mask) as views of one common batch shape; an undefined
// tensor when the kernel does not take this layout.
Tensor fused_call(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor* mask, bool causal,
                  float scale, Execution execution) {
    Shape batch;
    try {
        batch = broadcast_shapes(broadcast_shapes(leading(q), leading(k)), leading(v));
    } catch (const std::invalid_argument&) {
        return Tensor(); // the composition reports it, as mensurflow's second GEMM does
    }
    const std::int64_t lq = q.size(-2), lk = k.size(-2), d = q.size(-1), dv = v.size(-1);
    OpArgs args;
    args.inputs = {q.expand(matrix_shape(batch, lq, d)), k.expand(matrix_shape(batch, lk, d)),
                   v.expand(matrix_shape(batch, lk, dv))};
    if (mask != nullptr) {
        args.inputs.push_back(mask->expand(matrix_shape(batch, lq, lk)));
        args.has_mask = true;
    }
    args.outputs = {Tensor::empty(matrix_shape(batch, lq, dv), DType::F32, q.device())};
    args.alpha = scale;
    args.causal = causal;
    try {
        detail::dispatch(OpId::Attention, args, execution);
    } catch (const detail::NotImplemented&) {
        return Tensor();
    }
    return args.outputs.front();
}

// -inf wherever `keep` is false, so softmax gives those keys no weight: where(keep, scores, -inf)
// written into the scores themselves. They are this call's own temporary, so the values are
// where()'s without a second scores-sized buffer, and a device whose where kernel reads views
// (ROCm) writes only the removed keys.
void drop_where_not(const Tensor& keep, const Tensor& scores, Execution execution) {
    const Tensor minus_infinity =
        Tensor::full({}, -std::numeric_limits<double>::infinity(), DType::F32, scores.device());
    detail::where_into(keep, scores, minus_infinity, scores, execution);
}

// The [lq, lk] Bool lower triangle: query i keeps keys 0..i.
Tensor causal_keep(std::int64_t lq, std::int64_t lk, Device device) {
    std::vector<std::uint8_t> keep(static_cast<std::size_t>(lq * lk), 0);
    for (std::int64_t i = 0; i < lq; ++i) {
        const std::int64_t kept = std::min(i + 1, lk);
        std::fill_n(keep.begin() + i * lk, kept, std::uint8_t{1});
    }
    return Tensor::from_host(keep.data(), {lq, lk}, DType::Bool, device);
}

// The scaled scores q k^T with -inf above the diagonal, written by the ROCm batched GEMM's
// causal epilogue (OpArgs::causal), when the scores GEMM runs on ROCm; undefined when it runs
// elsewhere or the kernel does not take the layout (the composition then masks with where()).
Tensor causal_scores(const Tensor& q, const Tensor& k, const Shape& batch, float scale,
                     Execution execution) {
    Device target;
    try {
        target = detail::execution_device(execution, q.device());
    } catch (const std::exception&) {
        return Tensor();
    }
    if (target.type != DeviceType::ROCm || target != q.device()) {
        return Tensor();
    }
    const std::int64_t lq = q.size(-2), lk = k.size(-2), d = q.size(-1);
    OpArgs args;
    args.inputs = {q.expand(matrix_shape(batch, lq, d)),
                   k.transpose(-2, -1).expand(matrix_shape(batch, d, lk))};
    args.outputs = {Tensor::empty(matrix_shape(batch, lq, lk), DType::F32, q.device())};
    args.alpha = scale;
    args.beta = 0.0f;
    args.causal = true;
    try {
        detail::dispatch(OpId::GemmBatched, args, execution);
    } catch (const detail::NotImplemented&) {
        return Tensor();
    }
    return args.outputs.front();
}

} // namespace

Tensor attention(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor* mask, bool causal,
                 float scale, Execution execution) {
    check_operand(q, "q", q);
    check_operand(k, "k", q);
    check_operand(v, "v", q);
    const std::int64_t depth = q.size(-1), lq = q.size(-2), lk = k.size(-2);
    if (k.size(-1) != depth) {
        kCheck.fail("q " + to_string(q.shape()) + " and k " + to_string(k.shape()) +
                    " differ in the last dimension");
    }
    if (v.size(-2) != lk) {
        kCheck.fail("k " + to_string(k.shape()) + " and v " + to_string(v.shape()) +
                    " differ in the number of keys");
    }
    if (scale == 0.0f) {
        scale = depth > 0 ? static_cast<float>(1.0 / std::sqrt(static_cast<double>(depth))) : 1.0f;
    }
    // The scores' shape, with the message mensurflow's first batched GEMM gives when the batch
    // dimensions do not broadcast.
    Shape score_batch;
    try {
        score_batch = broadcast_shapes(leading(q), leading(k));
    } catch (const std::invalid_argument&) {
        OpCheck("gemm_strided_batched")
            .fail("batch shapes " + to_string(leading(q)) + " and " + to_string(leading(k)) +
                  " do not broadcast");
    }
    const Shape scores_shape = matrix_shape(score_batch, lq, lk);
    if (mask != nullptr) {
        if (!mask->defined() || mask->dtype() != DType::Bool) {
            kCheck.fail("mask must be a defined Bool tensor");
        }
        if (mask->device() != q.device()) {
            kCheck.fail("mask must be on the inputs' device");
        }
        if (broadcast_shapes(mask->shape(), scores_shape) != scores_shape) {
            kCheck.fail("mask " + to_string(mask->shape()) + " does not broadcast to the scores " +
                        to_string(scores_shape));
        }
    }
    if (detail::has_kernel_for(OpId::Attention, execution, q.device())) {
        const Tensor out = fused_call(q, k, v, mask, causal, scale, execution);
        if (out.defined()) {
            return out;
        }
    }
    // The composition: the scaled scores come from the GEMM's alpha.
    Tensor scores;
    if (causal && numel(scores_shape) > 0 && depth > 0) {
        scores = causal_scores(q, k, score_batch, scale, execution);
    }
    const bool causal_done = scores.defined();
    if (!causal_done) {
        scores = gemm_strided_batched(q, k, scale, nullptr, 0.0f, false, true, execution);
    }
    if (mask != nullptr) {
        drop_where_not(*mask, scores, execution);
    }
    if (causal && !causal_done) {
        drop_where_not(causal_keep(lq, lk, q.device()), scores, execution);
    }
    const Tensor weights = softmax(scores, -1, execution);
    return gemm_strided_batched(weights, v, 1.0f, nullptr, 0.0f, false, false, execution);
}

} // namespace mensurflow
