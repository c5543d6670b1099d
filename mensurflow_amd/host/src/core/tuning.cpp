// The results file, call keys, tuning scopes and dispatch()'s tuning hook (format and contract
// in core/tuning.hpp).
#include "core/tuning.hpp"

#include "core/registry.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <iterator>
#include <optional>
#include <regex>
#include <sstream>
#include <stdexcept>
#include <string_view>
#include <thread>

#if defined(__x86_64__) || defined(__i386__)
#include <cpuid.h>
#endif

namespace mensurflow::detail {

namespace {

// The contexts of the calling thread's open scopes, innermost last.
thread_local std::vector<TuningContext> t_scopes;

std::string_view strip(std::string_view text) {
    const char* const blanks = " \t\r\n";
    const std::size_t first = text.find_first_not_of(blanks);
    if (first == std::string_view::npos) {
        return {};
    }
    return text.substr(first, text.find_last_not_of(blanks) - first + 1);
}

// Whitespace-separated words of `text`.
std::vector<std::string> words(std::string_view text) {
    std::vector<std::string> out;
    std::istringstream in{std::string(text)};
    for (std::string word; in >> word;) {
        out.push_back(word);
    }
    return out;
}

std::string joined(const std::vector<std::string>& parts, std::size_t from) {
    std::string text;
    for (std::size_t i = from; i < parts.size(); ++i) {
        text += (i > from ? " " : "") + parts[i];
    }
    return text;
}

// "a=1 b=-2" -> {{"a", 1}, {"b", -2}}; invalid_argument for anything else.
TuningValues parse_settings(std::string_view text) {
    TuningValues values;
    for (const std::string& pair : words(text)) {
        const std::size_t eq = pair.find('=');
        if (eq == std::string::npos || eq == 0 || eq + 1 == pair.size()) {
            throw std::invalid_argument("expected name=value, got '" + pair + "'");
        }
        const std::string digits = pair.substr(eq + 1);
        std::size_t used = 0;
        const long long value = std::stoll(digits, &used);
        if (used != digits.size()) {
            throw std::invalid_argument("not an integer: '" + digits + "'");
        }
        values.emplace_back(pair.substr(0, eq), static_cast<std::int64_t>(value));
    }
    return values;
}

// The processor's brand string (CPUID leaves 0x80000002-4 on x86, /proc/cpuinfo elsewhere).
std::string processor_name() {
    std::string name;
#if defined(__x86_64__) || defined(__i386__)
    unsigned top = 0, b = 0, c = 0, d = 0;
    if (__get_cpuid(0x80000000u, &top, &b, &c, &d) && top >= 0x80000004u) {
        char brand[49] = {};
        for (unsigned leaf = 0; leaf < 3; ++leaf) {
            unsigned regs[4] = {};
            __get_cpuid(0x80000002u + leaf, &regs[0], &regs[1], &regs[2], &regs[3]);
            std::memcpy(brand + 16 * leaf, regs, sizeof regs);
        }
        name = brand;
    }
#else
    std::ifstream info("/proc/cpuinfo");
    for (std::string line; name.empty() && std::getline(info, line);) {
        if (line.rfind("model name", 0) == 0 || line.rfind("Model", 0) == 0) {
            const std::size_t colon = line.find(':');
            if (colon != std::string::npos) {
                name = line.substr(colon + 1);
            }
        }
    }
#endif
    name = std::string(strip(name));
    return name.empty() ? "unknown CPU" : name;
}

std::string shape_words(const Shape& shape) {
    if (shape.empty()) {
        return "scalar";
    }
    std::string text;
    for (const std::int64_t extent : shape) {
        text += (text.empty() ? "" : "x") + std::to_string(extent);
    }
    return text;
}

// The CPU kernels' thread count as OpenMP reports it by default: OMP_NUM_THREADS when set,
// else every hardware thread.
std::int64_t cpu_threads() {
    if (const char* env = std::getenv("OMP_NUM_THREADS")) {
        const long value = std::strtol(env, nullptr, 10);
        if (value > 0) {
            return value;
        }
    }
    const unsigned hardware = std::thread::hardware_concurrency();
    return hardware > 0 ? hardware : 1;
}

std::int64_t setting(const TuningValues& values, const std::string& name, std::int64_t absent) {
    const auto found = std::find_if(values.begin(), values.end(),
                                    [&](const auto& pair) { return pair.first == name; });
    return found != values.end() ? found->second : absent;
}

} // namespace

// ---- the results file --------------------------------------------------------------------------

namespace {

// One result line, "<op> <device> v<version> <key words> -> <settings> | <best> ms (default <ms>
// ms) <mode>", taken apart by one pattern; the key is every word between the version and the
// arrow. The error texts name the part that did not match, as the file format's readers expect.
// As lenient as the format's first reader: the version is the number at the start of what follows
// 'v' (so "v1x" is version 1), the mode is the first word after the timings (63 characters at
// most) and anything after it is ignored.
TuningEntry parse_result(const std::string& line, const std::string& machine) {
    static const std::regex whole(
        R"(^(\S+)\s+(\S+)\s+(\S+)((?:\s+\S+)*?)\s+->\s*(.*?)\s*\|\s*(.*)$)");
    static const std::regex times(R"(^(\S+)\s+ms\s+\(default\s+(\S+)\s+ms\)\s+(\S+).*$)");
    std::smatch part;
    if (!std::regex_match(line, part, whole)) {
        throw std::invalid_argument("expected '<op> <device> v<version> <key> -> <settings> | "
                                    "<ms> ms (default <ms> ms) <mode>'");
    }
    const std::string version = part[3].str();
    if (version.size() < 2 || version[0] != 'v') {
        throw std::invalid_argument("expected '<op> <device> v<version>' at the start");
    }
    TuningEntry entry;
    entry.machine = machine;
    entry.op = part[1].str();
    entry.device = part[2].str();
    entry.version = std::stoi(version.substr(1));
    entry.key = joined(words(part[4].str()), 0); // runs of blanks in the key count as one
    entry.config = parse_settings(part[5].str());
    const std::string tail = part[6].str();
    std::smatch timing;
    if (!std::regex_match(tail, timing, times)) {
        throw std::invalid_argument("expected '<ms> ms (default <ms> ms) <mode>' after '|'");
    }
    entry.best_ms = std::stod(timing[1].str());
    entry.default_ms = std::stod(timing[2].str());
    entry.mode = timing[3].str().substr(0, 63);
    return entry;
}

} // namespace

void TuningCache::load(const std::string& path) {
    std::ifstream file(path);
    if (!file) {
        return; // no results stored yet
    }
    std::vector<TuningEntry> parsed;
    std::string machine;
    std::string raw;
    for (int number = 1; std::getline(file, raw); ++number) {
        const std::string line(strip(raw));
        try {
            if (line.empty() || line.front() == '#') {
                continue;
            }
            if (line.compare(0, 8, "machine ") == 0) {
                machine = std::string(strip(std::string_view(line).substr(8)));
            } else if (machine.empty()) {
                throw std::invalid_argument("a result before any 'machine' line");
            } else if (line.compare(0, 6, "place ") != 0) {
                // ("place" lines are the older device-choice form: skipped, measured again
                // when tuned.)
                parsed.push_back(parse_result(line, machine));
            }
        } catch (const std::out_of_range& e) {
            throw std::runtime_error(path + ":" + std::to_string(number) +
                                     ": number out of range: " + e.what());
        } catch (const std::invalid_argument& e) {
            throw std::runtime_error(path + ":" + std::to_string(number) + ": " + e.what());
        }
    }
    entries_.swap(parsed);
}

void TuningCache::write(std::ostream& out) const {
    // The entries grouped by machine, machines in the order they first appear.
    std::vector<std::pair<std::string, std::vector<const TuningEntry*>>> groups;
    for (const TuningEntry& entry : entries_) {
        auto group = std::find_if(groups.begin(), groups.end(),
                                  [&](const auto& g) { return g.first == entry.machine; });
        if (group == groups.end()) {
            group = groups.insert(groups.end(), {entry.machine, {}});
        }
        group->second.push_back(&entry);
    }
    std::ostringstream text;
    text << "# mensurflow tuning results (format: src/core/tuning.hpp)\n"
         << "# <op> <device> v<version> <key> -> <settings> | <best> ms (default <ms> ms) <mode>\n"
         << "# device 'auto': the device for Execution::Auto, gpu=0 or gpu=1 (times include the "
            "copies)\n";
    text << std::fixed << std::setprecision(4);
    for (const auto& [machine, members] : groups) {
        text << "\nmachine " << machine << '\n';
        for (const TuningEntry* e : members) {
            text << e->op << ' ' << e->device << " v" << e->version << ' ' << e->key << " -> "
                 << mensurflow::to_string(e->config) << " | " << e->best_ms << " ms (default "
                 << e->default_ms << " ms) " << e->mode << '\n';
        }
    }
    out << text.str();
}

void TuningCache::save(const std::string& path) const {
    std::ofstream file(path);
    if (file) {
        write(file);
    }
    if (!file) {
        throw std::runtime_error("cannot write tuning results to " + path);
    }
}

const TuningEntry* TuningCache::find(const std::string& machine, const std::string& op,
                                     const std::string& device, int version,
                                     const std::string& key) const {
    const auto found = std::find_if(entries_.begin(), entries_.end(), [&](const TuningEntry& e) {
        return e.version == version && e.op == op && e.device == device && e.key == key &&
               e.machine == machine;
    });
    return found != entries_.end() ? &*found : nullptr;
}

void TuningCache::store(TuningEntry entry) {
    for (TuningEntry& held : entries_) {
        if (held.machine == entry.machine && held.op == entry.op && held.device == entry.device &&
            held.key == entry.key) {
            held = std::move(entry);
            return;
        }
    }
    entries_.push_back(std::move(entry));
}

// ---- keys ----------------------------------------------------------------------------------------

namespace {

// The name of the first registered device that is not the CPU, "" when there is none.
std::string first_accelerator_name() {
    const Registry& registry = Registry::instance();
    const std::vector<Device> devices = registry.devices();
    const auto found = std::find_if(devices.begin(), devices.end(),
                                    [](const Device& d) { return d.type != DeviceType::CPU; });
    return found == devices.end() ? std::string() : registry.get(*found).info(found->index).name;
}

// "name=value" words joined by single spaces: the key and settings text of the results file.
class KeyWriter {
  public:
    void add(const std::string& name, std::int64_t value) {
        text_ += text_.empty() ? "" : " ";
        text_ += name;
        text_ += '=';
        text_ += std::to_string(value);
    }
    std::string take() { return std::move(text_); }

  private:
    std::string text_;
};

} // namespace

// The CPU model, then " | " and the first accelerator's name where there is one; worked out
// once per process.
const std::string& machine_name() {
    static const std::string name = [] {
        const std::string accelerator = first_accelerator_name();
        return accelerator.empty() ? processor_name() : processor_name() + " | " + accelerator;
    }();
    return name;
}

// The tunable's key values under their names; on the CPU also the thread count, which its
// kernels' best settings depend on.
std::string call_key(const TunableKernel& tunable, const OpArgs& args, Device device) {
    const std::vector<std::int64_t> values = tunable.key(args);
    const std::size_t named = std::min(values.size(), tunable.key_names.size());
    KeyWriter key;
    for (std::size_t i = 0; i < named; ++i) {
        key.add(tunable.key_names[i], values[i]);
    }
    if (device.type == DeviceType::CPU) {
        key.add("threads", cpu_threads());
    }
    return key.take();
}

// "data=<device type> <dtype of the first input> <shape of each input>".
std::string placement_key(const OpArgs& args, Device data_device) {
    std::vector<std::string> parts{std::string("data=") + device_type_name(data_device.type),
                                   dtype_name(args.inputs.at(0).dtype())};
    std::transform(args.inputs.begin(), args.inputs.end(), std::back_inserter(parts),
                   [](const Tensor& input) { return shape_words(input.shape()); });
    return joined(parts, 0);
}

TuningConfig to_config(const TunableKernel& tunable, const TuningValues& settings) {
    TuningConfig config = tunable.defaults();
    config.size = static_cast<int>(tunable.params.size());
    for (std::size_t p = 0; p < tunable.params.size(); ++p) {
        config.values[p] = setting(settings, tunable.params[p], config.values[p]);
    }
    return config;
}

TuningValues from_config(const TunableKernel& tunable, const TuningConfig& config) {
    TuningValues named;
    const auto count = std::min<std::size_t>(static_cast<std::size_t>(config.size),
                                             tunable.params.size());
    for (std::size_t p = 0; p < count; ++p) {
        named.emplace_back(tunable.params[p], config.values[p]);
    }
    return named;
}

// ---- scopes and the hook -------------------------------------------------------------------------

TuningScope::TuningScope(TuningContext context) { t_scopes.push_back(context); }

TuningScope::~TuningScope() { t_scopes.pop_back(); }

bool tuning_active() { return !t_scopes.empty(); }

namespace {

// Where an Auto call with a stored placement runs (GPU when its "gpu" setting is nonzero); the
// requested execution when there is no stored placement or the call is not Auto.
Execution stored_placement(const TuningCache* results, OpId op, Execution execution,
                           Device data_device, const OpArgs& args) {
    if (results == nullptr || execution != Execution::Auto || args.inputs.empty()) {
        return execution;
    }
    const TuningEntry* placed = results->find(machine_name(), op_name(op), kAutoDevice, 1,
                                              placement_key(args, data_device));
    if (placed == nullptr) {
        return execution;
    }
    return setting(placed->config, "gpu", 0) != 0 ? Execution::GPU : Execution::CPU;
}

// The stored settings of the kernel that runs `op` on `target`, if it is tunable and has any.
std::optional<TuningConfig> stored_settings(const TuningCache* results, OpId op, Device target,
                                            const OpArgs& args) {
    if (results == nullptr) {
        return std::nullopt;
    }
    const Tensor& first = args.inputs.empty() ? args.outputs.at(0) : args.inputs.front();
    const TunableKernel* tunable =
        Registry::instance().dispatcher().tunable({op, target.type, first.dtype()});
    if (tunable == nullptr) {
        return std::nullopt;
    }
    const TuningEntry* stored =
        results->find(machine_name(), tunable->name, device_type_name(target.type),
                      tunable->version, call_key(*tunable, args, target));
    if (stored == nullptr) {
        return std::nullopt;
    }
    return to_config(*tunable, stored->config);
}

} // namespace

Device apply_tuning(OpId op, Execution execution, Device data_device, OpArgs& args) {
    const TuningContext context = t_scopes.back();
    const Device target = execution_device(
        stored_placement(context.cache, op, execution, data_device, args), data_device);
    if (context.record != nullptr) {
        context.record->push_back(RecordedCall{op, execution, data_device, target, args});
    }
    if (const std::optional<TuningConfig> tuned = stored_settings(context.cache, op, target, args)) {
        args.tuning = *tuned;
    }
    return target;
}

} // namespace mensurflow::detail

namespace mensurflow {

std::string to_string(const TuningValues& values) {
    std::string text;
    for (const auto& [name, value] : values) {
        text += (text.empty() ? "" : " ") + name + "=" + std::to_string(value);
    }
    return text;
}

} // namespace mensurflow
