// The op table and dispatch (the contract of mensurflow's src/core/dispatcher.cpp:228-353). The
// kernels sit in a dense table indexed by (op, device type, dtype); a call's device comes from
// execution_device(), or from the active tuning scope (core/tuning.hpp), and a call whose data
// lives on another device is moved there and back by a Relocation.
#include "core/dispatcher.hpp"

#include "core/registry.hpp"
#include "core/tensor_access.hpp"
#include "core/tuning.hpp"
#include "mensurflow/trace.hpp"

#include <stdexcept>
#include <string>

namespace mensurflow::detail {

namespace {

constexpr const char* kOpNames[] = {
    "scal",    "copy",     "add",         "mul",     "matvec",  "gemv",
    "matmul",  "gelu",     "where",       "bias_add", "argmax", "gemm_strided_batched",
    "uniform", "normal",   "softmax",     "gemm",    "strided_copy", "attention",
    "dot",     "sub",
};
constexpr std::size_t kOpCount = sizeof(kOpNames) / sizeof(kOpNames[0]);
static_assert(kOpCount == static_cast<std::size_t>(OpId::Sub) + 1, "a name for every op");

constexpr std::size_t kDeviceTypeCount = static_cast<std::size_t>(DeviceType::ROCm) + 1;
constexpr std::size_t kDTypeCount = static_cast<std::size_t>(DType::Bool) + 1;

// The table slot of `key`, or kOpCount * ... (out of range) for values outside the enums.
std::size_t slot_of(KernelKey key) {
    const auto op = static_cast<std::size_t>(key.op);
    const auto device = static_cast<std::size_t>(key.device);
    const auto dtype = static_cast<std::size_t>(key.dtype);
    if (op >= kOpCount || device >= kDeviceTypeCount || dtype >= kDTypeCount) {
        throw std::invalid_argument("invalid kernel key");
    }
    return (op * kDeviceTypeCount + device) * kDTypeCount + dtype;
}

std::string describe(KernelKey key) {
    return std::string(op_name(key.op)) + " on " + device_type_name(key.device) + " for " +
           dtype_name(key.dtype);
}

// The tensor a call is keyed and placed by: its first input, or for a factory (no inputs) its
// first output.
const Tensor& anchor_of(OpId op, const OpArgs& args) {
    const bool factory = op == OpId::Uniform || op == OpId::Normal;
    if (!args.inputs.empty()) {
        return args.inputs.front();
    }
    if (factory && !args.outputs.empty()) {
        return args.outputs.front();
    }
    throw std::invalid_argument(std::string(op_name(op)) + ": no input tensors");
}

void require_single_device(OpId op, const OpArgs& args, Device home) {
    auto check = [&](const Tensor& t) {
        if (t.device() != home) {
            throw std::invalid_argument(std::string(op_name(op)) + ": tensors are on " +
                                        to_string(home) + " and " + to_string(t.device()) +
                                        "; move one with Tensor::to()");
        }
    };
    for (const Tensor& t : args.inputs) {
        check(t);
    }
    for (const Tensor& t : args.outputs) {
        check(t);
    }
}

// A call run away from its data: the inputs copied to the target, the outputs computed into
// temporaries there, then copied into the caller's tensors.
class Relocation {
  public:
    Relocation(const OpArgs& original, Device target) : original_(original), moved_(original) {
        for (Tensor& input : moved_.inputs) {
            input = input.to(target);
        }
        for (Tensor& output : moved_.outputs) {
            output = Tensor::empty(output.shape(), output.dtype(), target);
        }
    }
    const OpArgs& args() const { return moved_; }
    void write_back(Device home) const {
        for (std::size_t i = 0; i < moved_.outputs.size(); ++i) {
            Tensor destination = original_.outputs[i]; // shares the caller's storage
            std::byte* host = TensorAccess::storage(destination).host_data();
            if (host != nullptr && destination.is_contiguous()) {
                // Straight into the caller's host memory: no host temporary and no second copy.
                moved_.outputs[i].copy_to_host(host + static_cast<std::size_t>(destination.offset()) *
                                                          destination.itemsize());
            } else {
                destination.copy_from(moved_.outputs[i].to(home));
            }
        }
    }

  private:
    const OpArgs& original_;
    OpArgs moved_;
};

// The backend call inside its "kernel" span; under MENSURFLOW_TRACE_SYNC the span also covers
// the device's work (trace.hpp).
void run_kernel(KernelFn kernel, const OpArgs& args, Stream& stream, Device target) {
    MENSURFLOW_TRACE("kernel", target, args.inputs, args.outputs);
    kernel(args, stream);
#ifdef MENSURFLOW_ENABLE_TRACING
    if (trace::detail::waits_for_device()) {
        stream.synchronize();
    }
#endif
}

void run_where(OpId op, const OpArgs& args, Device target, Device home) {
    MENSURFLOW_TRACE(op_name(op), target, args.inputs, args.outputs);
    Registry& registry = Registry::instance();
    Backend& backend = registry.get(target);
    const KernelFn kernel =
        registry.dispatcher().lookup({op, target.type, anchor_of(op, args).dtype()});
    Stream& stream = backend.stream(target.index);
    if (target == home) {
        run_kernel(kernel, args, stream, target);
        return;
    }
    const Relocation relocation(args, target);
    run_kernel(kernel, relocation.args(), stream, target);
    relocation.write_back(home);
}

} // namespace

const char* op_name(OpId op) {
    const auto index = static_cast<std::size_t>(op);
    if (index >= kOpCount) {
        throw std::invalid_argument("invalid OpId");
    }
    return kOpNames[index];
}

Dispatcher::Dispatcher() : table_(kOpCount * kDeviceTypeCount * kDTypeCount, nullptr) {}

void Dispatcher::register_kernel(KernelKey key, KernelFn kernel) {
    if (kernel == nullptr) {
        throw std::invalid_argument("register_kernel: null kernel");
    }
    KernelFn& slot = table_[slot_of(key)];
    if (slot != nullptr) {
        throw std::logic_error("kernel registered twice: " + describe(key));
    }
    slot = kernel;
}

KernelFn Dispatcher::find(KernelKey key) const { return table_[slot_of(key)]; }

KernelFn Dispatcher::lookup(KernelKey key) const {
    const KernelFn kernel = find(key);
    if (kernel == nullptr) {
        throw NotImplemented(std::string(op_name(key.op)) + " is not implemented on " +
                             device_type_name(key.device) + " for " + dtype_name(key.dtype));
    }
    return kernel;
}

void Dispatcher::register_tunable(KernelKey key, TunableKernel tunable) {
    const bool complete = tunable.key && tunable.defaults && tunable.space && tunable.allowed;
    if (!complete) {
        throw std::invalid_argument("register_tunable: " + tunable.name + " is missing a function");
    }
    if (tunable.params.size() > static_cast<std::size_t>(TuningConfig::capacity)) {
        throw std::invalid_argument("register_tunable: " + tunable.name + " has more than " +
                                    std::to_string(TuningConfig::capacity) + " parameters");
    }
    if (tunables_.count(key) != 0) {
        throw std::logic_error("tunable kernel registered twice: " + tunable.name);
    }
    tunables_.emplace(key, std::move(tunable));
}

const TunableKernel* Dispatcher::tunable(KernelKey key) const {
    const auto found = tunables_.find(key);
    return found != tunables_.end() ? &found->second : nullptr;
}

Device execution_device(Execution execution, Device data_device) {
    if (execution == Execution::Auto || execution == Execution::CPU) {
        return Device{DeviceType::CPU, 0};
    }
    if (execution != Execution::GPU) {
        throw std::invalid_argument("invalid Execution value");
    }
    if (data_device.type != DeviceType::CPU) {
        return data_device; // data already on a GPU stays there
    }
    constexpr DeviceType kGpuOrder[] = {DeviceType::CUDA, DeviceType::Metal, DeviceType::ROCm};
    for (const DeviceType type : kGpuOrder) {
        if (Registry::instance().find(type) != nullptr) {
            return Device{type, 0};
        }
    }
    throw std::runtime_error("Execution::GPU requested, but no GPU is available");
}

void dispatch(OpId op, const OpArgs& args, Execution execution) {
    const Device home = anchor_of(op, args).device();
    require_single_device(op, args, home);
    if (!tuning_active()) {
        run_where(op, args, execution_device(execution, home), home);
        return;
    }
    // A tuning scope may pick the device of an Auto call and the kernel's settings.
    OpArgs tuned = args;
    const Device target = apply_tuning(op, execution, home, tuned);
    run_where(op, tuned, target, home);
}

bool has_kernel_for(OpId op, Execution execution, Device data_device) {
    Device target;
    try {
        target = execution_device(execution, data_device);
    } catch (const std::exception&) {
        return false;
    }
    return Registry::instance().dispatcher().find({op, target.type, DType::F32}) != nullptr;
}

} // namespace mensurflow::detail
