// Test-only CPU kernels backed by the C oracle (see oracle_cpu.hpp). The adapters mirror how the
// reference's CPU backend hands tensors to its kernels (src/backends/cpu/backend.cpp:115-291).
#include "oracle_cpu.hpp"

#include "core/dispatcher.hpp"
#include "core/registry.hpp"
#include "core/tensor_access.hpp"
#include "oracle.h"

#include <cstdint>
#include <vector>

namespace test {

namespace {

using mensurflow::DType;
using mensurflow::DeviceType;
using mensurflow::Tensor;
using mensurflow::detail::OpArgs;
using mensurflow::detail::OpId;
using mensurflow::detail::Stream;
using mensurflow::detail::TensorAccess;

// The packed GEMM's depth block for a CPU with a large L2 (gemm_packed.cpp:227-276).
constexpr std::int64_t kDepthBlock = 768;

template <typename T> T* ptr(const Tensor& t) { return TensorAccess::data<T>(t); }

void matmul(const OpArgs& args, Stream&) {
    const Tensor& a = args.inputs[0];
    const Tensor& b = args.inputs[1];
    const Tensor& c = args.outputs[0];
    orc_sgemm_packed(a.size(0), b.size(1), a.size(1), ptr<float>(a), a.strides()[0],
                     a.strides()[1], ptr<float>(b), b.strides()[0], b.strides()[1], ptr<float>(c),
                     c.size(1), kDepthBlock);
}

// Per-matrix offsets by walking the batch index, then the packed GEMM and the alpha/beta finish
// pass for each matrix (src/backends/cpu/backend.cpp:239-291, gemm_batched.cpp:12-28).
void gemm_batched(const OpArgs& args, Stream&) {
    const Tensor& a = args.inputs[0];
    const Tensor& b = args.inputs[1];
    const Tensor& out = args.outputs[0];
    const bool with_c0 = args.inputs.size() > 2;
    const int batch_dims = out.dim() - 2;
    std::int64_t batch = 1;
    for (int d = 0; d < batch_dims; ++d) {
        batch *= out.size(d);
    }
    const std::int64_t m = out.size(-2), n = out.size(-1), k = a.size(-1);
    const auto bd = static_cast<std::size_t>(batch_dims);
    std::vector<std::int64_t> index(bd, 0);
    for (std::int64_t i = 0; i < batch; ++i) {
        std::int64_t oa = 0, ob = 0, rest = i;
        for (int d = batch_dims - 1; d >= 0; --d) {
            const auto du = static_cast<std::size_t>(d);
            const std::int64_t idx = rest % out.size(d);
            rest /= out.size(d);
            oa += idx * a.strides()[du];
            ob += idx * b.strides()[du];
        }
        float* c = ptr<float>(out) + i * m * n;
        orc_sgemm_packed(m, n, k, ptr<float>(a) + oa, a.strides()[bd], a.strides()[bd + 1],
                         ptr<float>(b) + ob, b.strides()[bd], b.strides()[bd + 1], c, n,
                         kDepthBlock);
        if (args.alpha != 1.0f || (with_c0 && args.beta != 0.0f)) {
            const float* c0 = with_c0 ? ptr<float>(args.inputs[2]) + i * m * n : nullptr;
            orc_axpby_f32(c, c, args.alpha, c0, with_c0 ? args.beta : 0.0f, m * n);
        }
    }
}

void gemv(const OpArgs& args, Stream&) {
    const Tensor& a = args.inputs[0];
    const float* y0 = args.inputs.size() > 2 ? ptr<float>(args.inputs[2]) : nullptr;
    orc_gemv_f32(ptr<float>(a), ptr<float>(args.inputs[1]), ptr<float>(args.outputs[0]),
                 a.size(0), a.size(1), args.alpha, args.beta, y0, args.transpose ? 1 : 0);
}

void matvec(const OpArgs& args, Stream&) {
    const Tensor& a = args.inputs[0];
    orc_matvec_f32(ptr<float>(a), ptr<float>(args.inputs[1]), ptr<float>(args.outputs[0]),
                   a.size(0), a.size(1));
}

void bias_add(const OpArgs& args, Stream&) {
    const Tensor& out = args.outputs[0];
    orc_bias_add_f32(ptr<float>(args.inputs[0]), ptr<float>(args.inputs[1]), ptr<float>(out),
                     out.numel(), out.size(1));
}

void gelu(const OpArgs& args, Stream&) {
    const Tensor& out = args.outputs[0];
    orc_gelu_f32(ptr<float>(args.inputs[0]), ptr<float>(out), out.numel(),
                 args.approximate ? 1 : 0);
}

void where(const OpArgs& args, Stream&) {
    const Tensor& out = args.outputs[0];
    orc_where_f32(ptr<std::uint8_t>(args.inputs[2]), ptr<float>(args.inputs[0]),
                  ptr<float>(args.inputs[1]), ptr<float>(out), out.numel());
}

void softmax(const OpArgs& args, Stream&) {
    const Tensor& x = args.inputs[0];
    std::int64_t outer = 1, length = 1, inner = 1;
    for (int d = 0; d < x.dim(); ++d) {
        if (d < args.axis) {
            outer *= x.size(d);
        } else if (d == args.axis) {
            length = x.size(d);
        } else {
            inner *= x.size(d);
        }
    }
    orc_softmax_f32(ptr<float>(x), ptr<float>(args.outputs[0]), outer, length, inner);
}

void argmax(const OpArgs& args, Stream&) {
    const Tensor& x = args.inputs[0];
    const std::int64_t width = x.size(x.dim() - 1);
    orc_argmax_f32(ptr<float>(x), ptr<std::int64_t>(args.outputs[0]), x.numel() / width, width);
}

void add(const OpArgs& args, Stream&) {
    const Tensor& out = args.outputs[0];
    orc_add_f32(ptr<float>(args.inputs[0]), ptr<float>(args.inputs[1]), ptr<float>(out),
                out.numel());
}

void sub(const OpArgs& args, Stream&) {
    const Tensor& out = args.outputs[0];
    orc_sub_f32(ptr<float>(args.inputs[0]), ptr<float>(args.inputs[1]), ptr<float>(out),
                out.numel());
}

// The reference's Dot adapter (src/backends/cpu/backend.cpp) writes dot_f32's float into the
// 0-d output.
void dot(const OpArgs& args, Stream&) {
    const Tensor& x = args.inputs[0];
    *ptr<float>(args.outputs[0]) = orc_dot_f32(ptr<float>(x), ptr<float>(args.inputs[1]),
                                               x.numel());
}

void mul(const OpArgs& args, Stream&) {
    const Tensor& out = args.outputs[0];
    orc_mul_f32(ptr<float>(args.inputs[0]), ptr<float>(args.inputs[1]), ptr<float>(out),
                out.numel());
}

void scal(const OpArgs& args, Stream&) {
    const Tensor& out = args.outputs[0];
    orc_axpby_f32(ptr<float>(out), ptr<float>(args.inputs[0]), args.alpha, nullptr, 0.0f,
                  out.numel());
}

void uniform(const OpArgs& args, Stream&) {
    const Tensor& out = args.outputs[0];
    orc_uniform_f32(ptr<float>(out), out.numel(), args.alpha, args.beta, args.seed, args.offset);
}

void normal(const OpArgs& args, Stream&) {
    const Tensor& out = args.outputs[0];
    orc_normal_f32(ptr<float>(out), out.numel(), args.alpha, args.beta, args.seed, args.offset);
}

} // namespace

void register_oracle_cpu_kernels() {
    auto& dispatcher = mensurflow::detail::Registry::instance().dispatcher();
    auto add_kernel = [&dispatcher](OpId op, mensurflow::detail::KernelFn fn) {
        dispatcher.register_kernel({op, DeviceType::CPU, DType::F32}, fn);
    };
    add_kernel(OpId::Matmul, matmul);
    add_kernel(OpId::GemmBatched, gemm_batched);
    add_kernel(OpId::Gemv, gemv);
    add_kernel(OpId::Matvec, matvec);
    add_kernel(OpId::BiasAdd, bias_add);
    add_kernel(OpId::Gelu, gelu);
    add_kernel(OpId::Where, where);
    add_kernel(OpId::Softmax, softmax);
    add_kernel(OpId::Argmax, argmax);
    add_kernel(OpId::Add, add);
    add_kernel(OpId::Mul, mul);
    add_kernel(OpId::Sub, sub);
    add_kernel(OpId::Dot, dot);
    add_kernel(OpId::Scal, scal);
    add_kernel(OpId::Uniform, uniform);
    add_kernel(OpId::Normal, normal);
}

} // namespace test
