// Tuned placement: the results file, the keys calls are stored under, and the hook dispatch()
// consults while a tuning scope is active. The file format, the keys and the hook's contract are
// mensurflow's (src/core/tuning.hpp:1-19, src/core/tuning.cpp:290-320,506-541), so a results
// file written by either is read by the other:
//
//   # comment
//   machine <cpu model> | <first GPU name>
//   <op> <device> v<version> <key> -> <name>=<value> ... | <best> ms (default <ms> ms) <mode>
//
// A kernel-settings line has the device type the kernel ran on and the kernel's key ("m=4096
// n=4096 k=4096"); a device-choice line has device "auto", a key naming where the data lives, its
// dtype and the input shapes ("data=cpu f32 256x1024 1024x4096"), and one setting, gpu=0 or 1.
// A line applies only to a call with exactly its machine, op, device, version and key.
#pragma once

#include "core/dispatcher.hpp"
#include "mensurflow/tuning.hpp"

#include <ostream>
#include <string>
#include <vector>

namespace mensurflow::detail {

inline const char* const kAutoDevice = "auto";

struct TuningEntry {
    std::string machine;
    std::string op;     // TunableKernel::name, or op_name() for a device choice
    std::string device; // device type name, or "auto"
    int version = 1;
    std::string key;
    TuningValues config;
    double best_ms = 0;
    double default_ms = 0;
    std::string mode; // "tested": measured on exactly this call
};

class TuningCache {
  public:
    // A missing file is an empty cache; a malformed one is runtime_error("<path>:<line>: ...").
    void load(const std::string& path);
    void save(const std::string& path) const; // runtime_error when it cannot be written
    void write(std::ostream& out) const;
    const TuningEntry* find(const std::string& machine, const std::string& op,
                            const std::string& device, int version, const std::string& key) const;
    void store(TuningEntry entry); // replaces the entry for the same call
    const std::vector<TuningEntry>& entries() const { return entries_; }

  private:
    std::vector<TuningEntry> entries_;
};

// "<cpu model> | <name of the first non-CPU device>": results are stored per machine.
const std::string& machine_name();

// A kernel call's key: the kernel's key values by name, plus threads=<n> on the CPU.
std::string call_key(const TunableKernel& tunable, const OpArgs& args, Device device);

// A device choice's key: "data=<device type> <dtype> <shape>..." over the inputs.
std::string placement_key(const OpArgs& args, Device data_device);

// Named settings as the kernel's TuningConfig (defaults for names it lacks), and back.
TuningConfig to_config(const TunableKernel& tunable, const TuningValues& settings);
TuningValues from_config(const TunableKernel& tunable, const TuningConfig& config);

// A call seen while a scope was recording: where its data was, where it ran, with what.
struct RecordedCall {
    OpId op;
    Execution execution;
    Device data_device;
    Device device;
    OpArgs args;
};

struct TuningContext {
    const TuningCache* cache = nullptr;          // results to apply
    std::vector<RecordedCall>* record = nullptr; // calls are appended here
};

// Makes `context` the calling thread's tuning context until the scope ends. Scopes nest: each
// thread keeps a stack of the contexts of its open scopes, and the innermost one applies.
class TuningScope {
  public:
    explicit TuningScope(TuningContext context);
    ~TuningScope();
    TuningScope(const TuningScope&) = delete;
    TuningScope& operator=(const TuningScope&) = delete;
};

bool tuning_active();

// dispatch()'s hook while a scope is active: the device the call runs on (the stored choice for
// an Auto call, else execution_device()), after recording the call and setting args.tuning to
// the stored settings of the kernel that will run, if any.
Device apply_tuning(OpId op, Execution execution, Device data_device, OpArgs& args);

} // namespace mensurflow::detail
