// Algorithm and Tuner: record an algorithm's calls, measure each one's device choice and kernel
// settings, store the winners (public side: include/mensurflow/tuning.hpp).
#include "mensurflow/tuning.hpp"

#include "core/registry.hpp"
#include "core/tuning.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <functional>
#include <iostream>
#include <limits>
#include <numeric>
#include <sstream>
#include <stdexcept>

namespace mensurflow {

namespace {

using detail::KernelFn;
using detail::OpArgs;
using detail::RecordedCall;
using detail::Registry;
using detail::TunableKernel;
using detail::TuningConfig;
using detail::TuningEntry;

using Clock = std::chrono::steady_clock;

// A measuring copy of a recorded call: every input resident on `device` (moved there when it lives
// elsewhere) and fresh outputs there, so a measurement never writes the algorithm's own tensors.
OpArgs measuring_copy(const OpArgs& args, Device device) {
    OpArgs copy = args;
    std::transform(copy.inputs.begin(), copy.inputs.end(), copy.inputs.begin(),
                   [device](const Tensor& t) { return t.device() == device ? t : t.to(device); });
    std::transform(copy.outputs.begin(), copy.outputs.end(), copy.outputs.begin(),
                   [device](const Tensor& t) { return Tensor::empty(t.shape(), t.dtype(), device); });
    return copy;
}

// A call's fp32 outputs as host vectors (empty for outputs of other types): what the result of a
// tuned point is compared by.
using Readback = std::vector<std::vector<float>>;

Readback read_back(const OpArgs& args) {
    Readback values(args.outputs.size());
    std::transform(args.outputs.begin(), args.outputs.end(), values.begin(), [](const Tensor& t) {
        return t.dtype() == DType::F32 ? t.to_vector<float>() : std::vector<float>{};
    });
    return values;
}

// Whether `got` is `want` up to the summation-order differences between kernel settings: per
// output, every element within 1e-3 of that output's largest magnitude (plus 1e-6), and NaN
// exactly where `want` has NaN.
bool within_rounding(const Readback& want, const Readback& got) {
    const auto same_output = [](const std::vector<float>& w, const std::vector<float>& g) {
        if (w.size() != g.size()) {
            return false;
        }
        const double largest = std::accumulate(
            w.begin(), w.end(), 0.0,
            [](double most, float v) { return std::max(most, std::fabs(static_cast<double>(v))); });
        const double slack = 1e-3 * largest + 1e-6;
        return std::equal(w.begin(), w.end(), g.begin(), [slack](float a, float b) {
            return std::isnan(a) ? std::isnan(b)
                                 : std::fabs(static_cast<double>(b) - static_cast<double>(a)) <=
                                       slack;
        });
    };
    return want.size() == got.size() &&
           std::equal(want.begin(), want.end(), got.begin(), same_output);
}

// Median milliseconds per call of `run`, which waits for its own work. Calls are timed in
// batches. The batch doubles from one call until it lasts at least a millisecond, so that short
// calls stay above the clock's resolution, and that calibrating batch is the first sample. More
// batches follow until there are options.min_samples of them and options.min_time_s has passed,
// 500 at most.
double median_ms(const std::function<void()>& run, const TuneOptions& options) {
    const auto batch_seconds = [&run](int calls) {
        const auto t0 = Clock::now();
        for (int i = 0; i < calls; ++i) {
            run();
        }
        return std::chrono::duration<double>(Clock::now() - t0).count();
    };
    run(); // the first call carries one-time costs (plans, caches)
    int batch = 1;
    double seconds = batch_seconds(batch);
    while (seconds < 1e-3 && batch < (1 << 20)) {
        batch *= 2;
        seconds = batch_seconds(batch);
    }
    std::vector<double> per_call{seconds / batch};
    const auto sampling = Clock::now();
    const auto enough = [&] {
        const double spent = std::chrono::duration<double>(Clock::now() - sampling).count();
        return static_cast<int>(per_call.size()) >= options.min_samples &&
               spent >= options.min_time_s;
    };
    while (per_call.size() < 500 && !enough()) {
        per_call.push_back(batch_seconds(batch) / batch);
    }
    const auto middle = per_call.begin() + static_cast<std::ptrdiff_t>(per_call.size() / 2);
    std::nth_element(per_call.begin(), middle, per_call.end());
    return *middle * 1e3;
}

// Every point of `region` (the product of its axes, the last axis fastest) that the kernel allows
// for this call.
std::vector<TuningConfig> points_of(const TunableKernel& tunable, const detail::SearchRegion& region,
                                    const OpArgs& args) {
    std::vector<TuningConfig> points;
    for (const detail::SearchAxis& axis : region.axes) {
        if (axis.values.empty()) {
            return points;
        }
    }
    std::vector<std::size_t> at(region.axes.size(), 0);
    for (;;) {
        TuningConfig point = region.start;
        for (std::size_t a = 0; a < region.axes.size(); ++a) {
            point.values[static_cast<std::size_t>(region.axes[a].param)] = region.axes[a].values[at[a]];
        }
        if (tunable.allowed(args, point)) {
            points.push_back(point);
        }
        std::size_t a = region.axes.size();
        while (a > 0) {
            --a;
            if (++at[a] < region.axes[a].values.size()) {
                break;
            }
            at[a] = 0;
            if (a == 0) {
                return points;
            }
        }
        if (region.axes.empty()) {
            return points;
        }
    }
}

} // namespace

Algorithm::Algorithm(Function function) : function_(std::move(function)) {
    if (!function_) {
        throw std::invalid_argument("Algorithm: empty function");
    }
}

std::vector<Tensor> Algorithm::run(const std::vector<Tensor>& inputs) const {
    return function_(inputs);
}

std::vector<Tensor> Algorithm::run(const std::vector<Tensor>& inputs, const Tuner& tuner) const {
    const detail::TuningScope scope({tuner.cache_.get(), nullptr});
    return function_(inputs);
}

Tuner::Tuner(std::string path)
    : path_(std::move(path)), cache_(std::make_shared<detail::TuningCache>()) {
    cache_->load(path_);
}

void Tuner::save() const { cache_->save(path_); }

std::size_t Tuner::size() const {
    const std::string& here = detail::machine_name();
    return static_cast<std::size_t>(std::count_if(
        cache_->entries().begin(), cache_->entries().end(),
        [&](const TuningEntry& e) { return e.machine == here; }));
}

std::string Tuner::describe() const {
    detail::TuningCache here;
    for (const TuningEntry& e : cache_->entries()) {
        if (e.machine == detail::machine_name()) {
            here.store(e);
        }
    }
    std::ostringstream text;
    here.write(text);
    return text.str();
}

TuneReport Tuner::tune(const Algorithm& algorithm, const std::vector<Tensor>& inputs,
                       const TuneOptions& options) {
    Registry& registry = Registry::instance();
    const std::string& machine = detail::machine_name();
    TuneReport report;

    // 1. The calls the algorithm makes, seen with nothing applied.
    std::vector<RecordedCall> calls;
    {
        const detail::TuningScope scope({nullptr, &calls});
        algorithm.run(inputs);
    }

    const auto store = [&](TunedCall result, const std::string& op, const std::string& device,
                           int version) {
        TuningEntry entry;
        entry.machine = machine;
        entry.op = op;
        entry.device = device;
        entry.version = version;
        entry.key = result.key;
        entry.config = result.best_settings;
        entry.best_ms = result.best_ms;
        entry.default_ms = result.default_ms;
        entry.mode = "tested";
        cache_->store(entry);
        if (options.verbose) {
            std::cout << "  " << result.op << " on " << result.device << " " << result.key << ": "
                      << to_string(result.best_settings) << " " << result.best_ms
                      << " ms (default " << result.default_ms << " ms)\n";
        }
        report.calls.push_back(std::move(result));
    };
    const auto stored = [&](TunedCall& result, const std::string& op, const std::string& device,
                            int version) {
        const TuningEntry* held = cache_->find(machine, op, device, version, result.key);
        if (held == nullptr || options.retune) {
            return false;
        }
        result.reused = true;
        result.best_settings = held->config;
        result.best_ms = held->best_ms;
        result.default_ms = held->default_ms;
        report.calls.push_back(result);
        return true;
    };

    for (const RecordedCall& call : calls) {
        const detail::OpId op = call.op;
        const DType dtype = (call.args.inputs.empty() ? call.args.outputs.at(0)
                                                      : call.args.inputs[0]).dtype();
        Device target = call.device;

        // 2. The device of an Auto call: the CPU (the default) against every GPU with a kernel,
        //    each timed with its copies in and out.
        if (call.execution == Execution::Auto && !call.args.inputs.empty()) {
            TunedCall result;
            result.op = detail::op_name(op);
            result.device = detail::kAutoDevice;
            result.key = detail::placement_key(call.args, call.data_device);
            result.default_settings = {{"gpu", 0}};
            if (!stored(result, result.op, detail::kAutoDevice, 1)) {
                double best = std::numeric_limits<double>::infinity();
                for (const Device device : registry.devices()) {
                    if (device.index != 0 ||
                        registry.dispatcher().find({op, device.type, dtype}) == nullptr) {
                        continue;
                    }
                    const KernelFn kernel = registry.dispatcher().find({op, device.type, dtype});
                    detail::Stream& stream = registry.get(device).stream(device.index);
                    const double ms = median_ms(
                        [&] {
                            OpArgs moved = measuring_copy(call.args, device);
                            kernel(moved, stream);
                            for (Tensor& out : moved.outputs) {
                                out = out.to(call.data_device);
                            }
                            if (!moved.outputs.empty()) {
                                (void)read_back(moved);
                            }
                        },
                        options);
                    ++result.space_size;
                    if (device.type == DeviceType::CPU) {
                        result.default_ms = ms;
                    }
                    if (ms < best) {
                        best = ms;
                        result.best_ms = ms;
                        result.best_settings = {{"gpu", device.type == DeviceType::CPU ? 0 : 1}};
                        target = device;
                    }
                }
                if (result.space_size > 0) {
                    store(result, result.op, detail::kAutoDevice, 1);
                }
            } else {
                for (const auto& [name, value] : result.best_settings) {
                    if (name == "gpu") {
                        target = detail::execution_device(value != 0 ? Execution::GPU
                                                                     : Execution::CPU,
                                                          call.data_device);
                    }
                }
            }
        }

        // 3. The settings of the kernel on the device the call runs on.
        const TunableKernel* tunable = registry.dispatcher().tunable({op, target.type, dtype});
        if (tunable == nullptr) {
            continue;
        }
        const OpArgs base = measuring_copy(call.args, target);
        TunedCall result;
        result.op = tunable->name;
        result.device = to_string(target);
        result.key = detail::call_key(*tunable, base, target);
        result.default_settings = detail::from_config(*tunable, tunable->defaults());
        if (stored(result, tunable->name, device_type_name(target.type), tunable->version)) {
            continue;
        }
        const KernelFn kernel = registry.dispatcher().lookup({op, target.type, dtype});
        detail::Stream& stream = registry.get(target).stream(target.index);
        const auto timed = [&](const TuningConfig& config, Readback* out) {
            OpArgs args = measuring_copy(base, target);
            args.tuning = config;
            kernel(args, stream);
            if (out != nullptr) {
                *out = read_back(args);
            }
            return median_ms(
                [&] {
                    kernel(args, stream);
                    stream.synchronize();
                },
                options);
        };
        Readback reference;
        result.default_ms = timed(tunable->defaults(), &reference);
        result.best_ms = result.default_ms;
        result.best_settings = result.default_settings;
        for (const detail::SearchRegion& region : tunable->space(base)) {
            for (const TuningConfig& point : points_of(*tunable, region, base)) {
                Readback outputs;
                double ms = std::numeric_limits<double>::infinity();
                try {
                    ms = timed(point, &outputs);
                } catch (const std::exception&) {
                    continue; // a point the kernel refuses at run time
                }
                ++result.space_size;
                if (ms < result.best_ms && within_rounding(reference, outputs)) {
                    result.best_ms = ms;
                    result.best_settings = detail::from_config(*tunable, point);
                }
            }
        }
        store(result, tunable->name, device_type_name(target.type), tunable->version);
    }
    if (options.save) {
        save();
    }
    return report;
}

} // namespace mensurflow
