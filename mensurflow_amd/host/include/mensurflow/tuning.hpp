// Tuning: measuring, on this machine, the settings of the tunable kernels an algorithm calls and
// the device of its Execution::Auto calls, keeping the winners in a text file, and running the
// algorithm with them. The names follow mensurflow's include/mensurflow/tuning.hpp; the results
// file is the same format (src/core/tuning.hpp:1-19), so either library reads the other's.
//
//   mf::Algorithm step([](const std::vector<mf::Tensor>& in) {
//       return std::vector<mf::Tensor>{mf::matmul(in[0], in[1])}; // Execution::Auto
//   });
//   mf::Tuner tuner("mensurflow_tuning.txt"); // earlier results, if the file exists
//   tuner.tune(step, {a, b});                 // device choice + kernel settings, then saved
//   auto out = step.run({a, b}, tuner);       // the stored choices applied
//
// This build searches every allowed point of a kernel's space (the ROCm GEMM's is at most 72
// points); a point is kept only when its result agrees with the default's within 1e-3 of the
// output's largest magnitude. Without a stored choice an Auto call runs on the CPU.
#pragma once

#include "mensurflow/tensor.hpp"

#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace mensurflow {

namespace detail {
class TuningCache;
}

class Tuner;

// A function from input tensors to output tensors, run once per run() and several times while it
// is tuned, so it should have no effect beyond its outputs.
class Algorithm {
  public:
    using Function = std::function<std::vector<Tensor>(const std::vector<Tensor>& inputs)>;

    explicit Algorithm(Function function);

    std::vector<Tensor> run(const std::vector<Tensor>& inputs) const;
    // With the settings `tuner` holds for this machine; calls it has nothing for run as usual.
    std::vector<Tensor> run(const std::vector<Tensor>& inputs, const Tuner& tuner) const;

  private:
    Function function_;
};

// name = value, in order. to_string gives "name=value name=value".
using TuningValues = std::vector<std::pair<std::string, std::int64_t>>;
std::string to_string(const TuningValues& values);

struct TuneOptions {
    bool retune = false;      // measure calls that already have a stored result again
    bool save = true;         // write the file when tune() ends
    double min_time_s = 0.02; // per point: sample until this much time has passed ...
    int min_samples = 3;      // ... and at least this many samples (the median is kept)
    bool verbose = false;     // print each call's result
};

// What tuning found for one call.
struct TunedCall {
    std::string op;     // "matmul", or the tunable kernel's name
    std::string device; // "rocm:0", or "auto" for a device choice
    std::string key;
    TuningValues default_settings;
    TuningValues best_settings;
    double default_ms = 0;
    double best_ms = 0;
    bool reused = false;        // already stored, not measured again
    std::size_t space_size = 0; // points measured
};

struct TuneReport {
    std::vector<TunedCall> calls;
};

class Tuner {
  public:
    // Reads the results stored at `path` (a missing file is fine); runtime_error naming the line
    // of a malformed file.
    explicit Tuner(std::string path = "mensurflow_tuning.txt");

    // Runs `algorithm` on `inputs` once to see its calls, then measures, for each: the device of
    // an Auto call (every available device, copies included; the CPU is the default), and the
    // settings of a tunable kernel on the device it runs on. Saves the file (options.save).
    TuneReport tune(const Algorithm& algorithm, const std::vector<Tensor>& inputs,
                    const TuneOptions& options = {});

    void save() const;
    const std::string& path() const { return path_; }
    std::size_t size() const;     // results stored for this machine
    std::string describe() const; // those results, as the file holds them

  private:
    friend class Algorithm;
    std::string path_;
    std::shared_ptr<detail::TuningCache> cache_;
};

} // namespace mensurflow
