// The op table and dispatch(): the plugin surface a backend registers against. Types, fields and
// calls are the ones mensurflow's core defines (src/core/dispatcher.hpp:21-285), so a backend
// written against this header compiles against mensurflow's. This build lists only the hot
// path's ops, plus three that its integration adds:
//   Gemm         one fused GEMM (alpha, beta * C0, bias, activation): mensurflow::gemm is one
//                dispatch where a device has it;
//   StridedCopy  packs a strided view on its own device, for Tensor::contiguous();
//   Attention    fused scaled dot-product attention (mask, causal).
// A missing kernel is reported (NotImplemented); dispatch never moves an op to another device on
// its own.
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
    Gemm,
    StridedCopy,
    Attention,
    Dot,
    Sub
};

// "gemm_strided_batched", "bias_add", ...: the name errors and tuning results use.
const char* op_name(OpId op);

struct KernelKey {
    OpId op;
    DeviceType device;
    DType dtype;
};

inline bool operator<(const KernelKey& a, const KernelKey& b) {
    return std::tie(a.op, a.device, a.dtype) < std::tie(b.op, b.device, b.dtype);
}

// A tunable kernel's settings for one call: the values of its parameters in registration order.
// size 0 = none chosen, the kernel picks its own.
struct TuningConfig {
    static constexpr int capacity = 8;
    std::array<std::int64_t, capacity> values{};
    int size = 0;
};

inline bool operator<(const TuningConfig& a, const TuningConfig& b) {
    return std::tie(a.size, a.values) < std::tie(b.size, b.values);
}
inline bool operator==(const TuningConfig& a, const TuningConfig& b) {
    return a.size == b.size && a.values == b.values;
}
inline bool operator!=(const TuningConfig& a, const TuningConfig& b) { return !(a == b); }

// One call's operands and scalars. Ops validate before they dispatch, so a kernel may take the
// shapes as agreeing and every tensor as living on its device.
struct OpArgs {
    std::vector<Tensor> inputs;
    std::vector<Tensor> outputs;
    float alpha = 1.0f;
    float beta = 1.0f; // 1 unless an op sets it (gemv's beta, the batched GEMM's beta)
    int axis = -1;
    bool transpose = false;
    bool approximate = false; // gelu: the tanh form
    std::uint64_t seed = 0;
    std::uint64_t offset = 0;
    // Gemm: the activation applied after the bias (0 none, 1 gelu-tanh, 2 gelu), and whether the
    // last input is the bias vector.
    int activation = 0;
    bool has_bias = false;
    // Attention: causal masking, and whether the last input is a Bool mask. GemmBatched (the
    // ROCm kernel only, which attention's composition alone sends it to): out(..., i, j) = -inf
    // wherever j > i; a layout the kernel cannot mask throws NotImplemented.
    bool causal = false;
    bool has_mask = false;
    TuningConfig tuning{}; // filled by dispatch() from an active tuning scope
};

using KernelFn = void (*)(const OpArgs& args, Stream& stream);

// An ordered axis of a tunable kernel's settings: parameter `param` takes `values`.
struct SearchAxis {
    int param = 0;
    std::vector<std::int64_t> values;
};

// A region of settings searched as a whole: parameters off the axes keep their `start` value.
struct SearchRegion {
    std::string name;
    TuningConfig start;
    std::vector<SearchAxis> axes;
};

// A kernel whose settings a tuner may choose: how a call is keyed, its parameters and defaults,
// the space to search for a call, and which points of it can run.
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

// No kernel for the (op, device, dtype) asked for, or a layout a kernel does not take.
class NotImplemented : public std::runtime_error {
  public:
    using std::runtime_error::runtime_error;
};

class Dispatcher {
  public:
    Dispatcher();
    // invalid_argument for a null kernel; logic_error when the key already has one.
    void register_kernel(KernelKey key, KernelFn kernel);
    KernelFn find(KernelKey key) const;   // nullptr when the key has no kernel
    KernelFn lookup(KernelKey key) const; // NotImplemented naming op, device and dtype
    // invalid_argument for a missing function or too many params; logic_error when repeated.
    void register_tunable(KernelKey key, TunableKernel tunable);
    const TunableKernel* tunable(KernelKey key) const; // nullptr when not tunable
    const std::map<KernelKey, TunableKernel>& tunables() const { return tunables_; }

  private:
    std::vector<KernelFn> table_; // dense: one slot per (op, device type, dtype)
    std::map<KernelKey, TunableKernel> tunables_;
};

// Where a call runs: CPU -> cpu:0; GPU -> the data's device when that is a GPU, else device 0 of
// the first available of CUDA, Metal, ROCm (runtime_error when none is); Auto -> cpu:0, unless
// an active tuning scope holds a device choice for the call (core/tuning.hpp).
Device execution_device(Execution execution, Device data_device);

// Runs `op` where `execution` says. Every input and output must be on one device; when the op
// runs on another, its inputs are copied there, the kernel fills temporaries, and those are
// copied back into `outputs`. Throws invalid_argument for mixed devices, runtime_error for an
// unavailable device and NotImplemented for a missing kernel.
void dispatch(OpId op, const OpArgs& args, Execution execution);

// Whether the device a call with this execution would run on has an F32 kernel for `op` (false
// when that device cannot be resolved; the caller's unfused path then reports why).
bool has_kernel_for(OpId op, Execution execution, Device data_device);

} // namespace mensurflow::detail
