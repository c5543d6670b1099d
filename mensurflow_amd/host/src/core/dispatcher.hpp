// The op table: (op, device type, dtype) -> kernel, and dispatch(), which runs an op where the
// caller's Execution says (the reference's src/core/dispatcher.hpp:21-285, same types and
// semantics). A missing kernel is an error (NotImplemented), never a silent move to another
// device.
//
// This build carries the ops of the BLAS hot path only. Two ops are new: Gemm (one fused
// alpha/beta/bias/activation GEMM, so mensurflow::gemm is one dispatch on devices that have it)
// and StridedCopy (device-side packing of a strided view for Tensor::contiguous()).
#pragma once

#include "backends/backend.hpp"
#include "mensurflow/dtype.hpp"
#include "mensurflow/execution.hpp"
#include "mensurflow/tensor.hpp"

#include <array>
#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

namespace mensurflow::detail {

enum class OpId {
    Scal,
    Copy,
    Add,
    Mul,
    Matvec,
    Gemv,
    Matmul,
    Gelu,
    Where,
    BiasAdd,
    Argmax,
    GemmBatched,
    Uniform,
    Normal,
    Softmax,
    Gemm,        // new: fused gemm (alpha, beta, bias, activation)
    StridedCopy, // new: pack a strided view on its own device
    Attention    // new: fused scaled dot-product attention (mask, causal)
};

const char* op_name(OpId op);

struct KernelKey {
    OpId op;
    DeviceType device;
    DType dtype;
};

inline bool operator<(const KernelKey& a, const KernelKey& b) {
    return std::tie(a.op, a.device, a.dtype) < std::tie(b.op, b.device, b.dtype);
}

// Settings a tuner chose for one call of a tunable kernel (values of its registered parameters,
// in order); size 0 = the kernel's defaults.
struct TuningConfig {
    static constexpr int capacity = 8;
    std::array<std::int64_t, capacity> values{};
    int size = 0;
};

// Everything a kernel needs. Ops validate first, so kernels may assume shapes agree and all
// tensors are on one device.
struct OpArgs {
    std::vector<Tensor> inputs;
    std::vector<Tensor> outputs;
    float alpha = 1.0f;
    float beta = 1.0f; // note: 1 by default, as in the reference
    int axis = -1;
    bool transpose = false;
    bool approximate = false;
    std::uint64_t seed = 0;
    std::uint64_t offset = 0;
    // Gemm only: activation after the bias (0 none, 1 gelu-tanh, 2 gelu) and whether the last
    // input is a bias vector.
    int activation = 0;
    bool has_bias = false;
    // Attention only: causal masking, and whether the last input is a Bool mask.
    bool causal = false;
    bool has_mask = false;
    TuningConfig tuning{};
};

using KernelFn = void (*)(const OpArgs& args, Stream& stream);

// A parameter axis of a tunable kernel's search space (the reference's SearchAxis).
struct SearchAxis {
    int param = 0;
    std::vector<std::int64_t> values;
};

struct SearchRegion {
    std::string name;
    TuningConfig start;
    std::vector<SearchAxis> axes;
};

// What a backend registers for a kernel whose settings a tuner may choose.
struct TunableKernel {
    std::string name;
    int version = 1;
    std::vector<std::string> key_names;
    std::vector<std::int64_t> (*key)(const OpArgs& args) = nullptr;
    std::vector<std::string> params;
    TuningConfig (*defaults)() = nullptr;
    std::vector<SearchRegion> (*space)(const OpArgs& args) = nullptr;
    bool (*allowed)(const OpArgs& args, const TuningConfig& config) = nullptr;
};

// No kernel for the requested (op, device, dtype).
class NotImplemented : public std::runtime_error {
  public:
    using std::runtime_error::runtime_error;
};

class Dispatcher {
  public:
    // Throws invalid_argument for a null kernel, logic_error for a second registration.
    void register_kernel(KernelKey key, KernelFn kernel);
    KernelFn find(KernelKey key) const; // nullptr when absent
    KernelFn lookup(KernelKey key) const; // throws NotImplemented naming op, device and dtype
    void register_tunable(KernelKey key, TunableKernel tunable);
    const TunableKernel* tunable(KernelKey key) const;
    const std::map<KernelKey, TunableKernel>& tunables() const { return tunables_; }

  private:
    std::map<KernelKey, KernelFn> kernels_;
    std::map<KernelKey, TunableKernel> tunables_;
};

// CPU -> cpu:0; GPU -> the data's device if it is a GPU, else the first available CUDA, Metal
// or ROCm device (runtime_error if none); Auto -> cpu:0.
Device execution_device(Execution execution, Device data_device);

// Runs `op` where `execution` says, copying inputs there and outputs back when the data lives
// elsewhere. Throws invalid_argument for mixed devices, runtime_error for an unavailable device,
// NotImplemented for a missing kernel.
void dispatch(OpId op, const OpArgs& args, Execution execution);

// True when `op` has an F32 kernel on the device a call with these settings would run on (false
// when that device cannot be resolved: the caller's unfused path then reports the error).
bool has_kernel_for(OpId op, Execution execution, Device data_device);

} // namespace mensurflow::detail
