// The op table and dispatch (semantics of the reference's src/core/dispatcher.cpp:228-353).
#include "core/dispatcher.hpp"

#include "core/registry.hpp"

#include <stdexcept>

namespace mensurflow::detail {

const char* op_name(OpId op) {
    switch (op) {
    case OpId::Scal: return "scal";
    case OpId::Copy: return "copy";
    case OpId::Add: return "add";
    case OpId::Mul: return "mul";
    case OpId::Matvec: return "matvec";
    case OpId::Gemv: return "gemv";
    case OpId::Matmul: return "matmul";
    case OpId::Gelu: return "gelu";
    case OpId::Where: return "where";
    case OpId::BiasAdd: return "bias_add";
    case OpId::Argmax: return "argmax";
    case OpId::GemmBatched: return "gemm_strided_batched";
    case OpId::Uniform: return "uniform";
    case OpId::Normal: return "normal";
    case OpId::Softmax: return "softmax";
    case OpId::Gemm: return "gemm";
    case OpId::StridedCopy: return "strided_copy";
    case OpId::Attention: return "attention";
    }
    throw std::invalid_argument("invalid OpId");
}

void Dispatcher::register_kernel(KernelKey key, KernelFn kernel) {
    if (kernel == nullptr) {
        throw std::invalid_argument("register_kernel: null kernel");
    }
    if (!kernels_.emplace(key, kernel).second) {
        throw std::logic_error(std::string("kernel registered twice: ") + op_name(key.op) + " on " +
                               device_type_name(key.device) + " for " + dtype_name(key.dtype));
    }
}

KernelFn Dispatcher::find(KernelKey key) const {
    const auto it = kernels_.find(key);
    return it == kernels_.end() ? nullptr : it->second;
}

KernelFn Dispatcher::lookup(KernelKey key) const {
    if (KernelFn kernel = find(key)) {
        return kernel;
    }
    throw NotImplemented(std::string(op_name(key.op)) + " is not implemented on " +
                         device_type_name(key.device) + " for " + dtype_name(key.dtype));
}

void Dispatcher::register_tunable(KernelKey key, TunableKernel tunable) {
    if (tunable.key == nullptr || tunable.defaults == nullptr || tunable.space == nullptr ||
        tunable.allowed == nullptr) {
        throw std::invalid_argument("register_tunable: " + tunable.name + " is missing a function");
    }
    if (tunable.params.size() > static_cast<std::size_t>(TuningConfig::capacity)) {
        throw std::invalid_argument("register_tunable: " + tunable.name + " has more than " +
                                    std::to_string(TuningConfig::capacity) + " parameters");
    }
    const std::string name = tunable.name;
    if (!tunables_.emplace(key, std::move(tunable)).second) {
        throw std::logic_error("tunable kernel registered twice: " + name);
    }
}

const TunableKernel* Dispatcher::tunable(KernelKey key) const {
    const auto it = tunables_.find(key);
    return it == tunables_.end() ? nullptr : &it->second;
}

Device execution_device(Execution execution, Device data_device) {
    switch (execution) {
    case Execution::Auto:
    case Execution::CPU:
        return {DeviceType::CPU, 0};
    case Execution::GPU:
        if (data_device.type != DeviceType::CPU) {
            return data_device;
        }
        for (DeviceType type : {DeviceType::CUDA, DeviceType::Metal, DeviceType::ROCm}) {
            if (Registry::instance().find(type) != nullptr) {
                return {type, 0};
            }
        }
        throw std::runtime_error("Execution::GPU requested, but no GPU is available");
    }
    throw std::invalid_argument("invalid Execution value");
}

namespace {

// Runs the kernel on `target`. When the data lives elsewhere, the inputs are copied over, the
// kernel fills fresh outputs there, and those are copied back into the caller's outputs.
void run_on(OpId op, const OpArgs& args, Device target, Device data_device) {
    const Tensor& source = args.inputs.empty() ? args.outputs[0] : args.inputs[0];
    Registry& registry = Registry::instance();
    Backend& backend = registry.get(target);
    const KernelFn kernel = registry.dispatcher().lookup({op, target.type, source.dtype()});
    if (target == data_device) {
        kernel(args, backend.stream(target.index));
        return;
    }
    OpArgs moved = args;
    for (Tensor& input : moved.inputs) {
        input = input.to(target);
    }
    for (Tensor& output : moved.outputs) {
        output = Tensor::empty(output.shape(), output.dtype(), target);
    }
    kernel(moved, backend.stream(target.index));
    for (std::size_t i = 0; i < args.outputs.size(); ++i) {
        Tensor destination = args.outputs[i]; // shares the caller's storage
        destination.copy_from(moved.outputs[i].to(data_device));
    }
}

} // namespace

void dispatch(OpId op, const OpArgs& args, Execution execution) {
    const bool factory = op == OpId::Uniform || op == OpId::Normal;
    if (args.inputs.empty() && (!factory || args.outputs.empty())) {
        throw std::invalid_argument(std::string(op_name(op)) + ": no input tensors");
    }
    const Tensor& source = args.inputs.empty() ? args.outputs[0] : args.inputs[0];
    const Device data_device = source.device();
    for (const auto* group : {&args.inputs, &args.outputs}) {
        for (const Tensor& t : *group) {
            if (t.device() != data_device) {
                throw std::invalid_argument(std::string(op_name(op)) + ": tensors are on " +
                                            to_string(data_device) + " and " +
                                            to_string(t.device()) + "; move one with Tensor::to()");
            }
        }
    }
    run_on(op, args, execution_device(execution, data_device), data_device);
}

bool has_kernel_for(OpId op, Execution execution, Device data_device) {
    try {
        const Device target = execution_device(execution, data_device);
        return Registry::instance().dispatcher().find({op, target.type, DType::F32}) != nullptr;
    } catch (const std::exception&) {
        return false;
    }
}

} // namespace mensurflow::detail
