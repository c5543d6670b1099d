// The results file, call keys, tuning scopes and dispatch()'s tuning hook (format and contract
// in core/tuning.hpp).
#include "core/tuning.hpp"

#include "core/registry.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string_view>
#include <thread>

#if defined(__x86_64__) || defined(__i386__)
#include <cpuid.h>
#endif

namespace mensurflow::detail {

namespace {

thread_local TuningContext* t_context = nullptr;

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

void TuningCache::load(const std::string& path) {
    std::ifstream file(path);
    if (!file) {
        return;
    }
    std::vector<TuningEntry> read;
    std::string machine;
    int line_number = 0;
    for (std::string raw; std::getline(file, raw);) {
        ++line_number;
        const std::string_view line = strip(raw);
        const auto bad = [&](const std::string& why) {
            return std::runtime_error(path + ":" + std::to_string(line_number) + ": " + why);
        };
        if (line.empty() || line.front() == '#') {
            continue;
        }
        if (line.rfind("machine ", 0) == 0) {
            machine = std::string(strip(line.substr(8)));
            continue;
        }
        if (machine.empty()) {
            throw bad("a result before any 'machine' line");
        }
        if (line.rfind("place ", 0) == 0) {
            continue; // an older device-choice form: ignored, measured again when tuned
        }
        const std::size_t arrow = line.find(" -> ");
        const std::size_t bar = arrow == std::string_view::npos ? arrow : line.find(" | ", arrow);
        if (bar == std::string_view::npos) {
            throw bad("expected '<op> <device> v<version> <key> -> <settings> | <ms> ms (default "
                      "<ms> ms) <mode>'");
        }
        TuningEntry entry;
        entry.machine = machine;
        try {
            const std::vector<std::string> head = words(line.substr(0, arrow));
            if (head.size() < 3 || head[2].size() < 2 || head[2][0] != 'v') {
                throw bad("expected '<op> <device> v<version>' at the start");
            }
            entry.op = head[0];
            entry.device = head[1];
            entry.version = std::stoi(head[2].substr(1));
            entry.key = joined(head, 3);
            entry.config = parse_settings(line.substr(arrow + 4, bar - arrow - 4));
            const std::string tail(line.substr(bar + 3));
            char mode[64] = {};
            if (std::sscanf(tail.c_str(), "%lf ms (default %lf ms) %63s", &entry.best_ms,
                            &entry.default_ms, mode) != 3) {
                throw bad("expected '<ms> ms (default <ms> ms) <mode>' after '|'");
            }
            entry.mode = mode;
        } catch (const std::invalid_argument& e) {
            throw bad(e.what());
        } catch (const std::out_of_range& e) {
            throw bad(std::string("number out of range: ") + e.what());
        }
        read.push_back(std::move(entry));
    }
    entries_ = std::move(read);
}

void TuningCache::write(std::ostream& out) const {
    out << "# mensurflow tuning results (format: src/core/tuning.hpp)\n"
        << "# <op> <device> v<version> <key> -> <settings> | <best> ms (default <ms> ms) <mode>\n"
        << "# device 'auto': the device for Execution::Auto, gpu=0 or gpu=1 (times include the "
           "copies)\n";
    std::vector<std::string> machines;
    for (const TuningEntry& entry : entries_) {
        if (std::find(machines.begin(), machines.end(), entry.machine) == machines.end()) {
            machines.push_back(entry.machine);
        }
    }
    for (const std::string& machine : machines) {
        out << "\nmachine " << machine << '\n';
        for (const TuningEntry& e : entries_) {
            if (e.machine != machine) {
                continue;
            }
            char times[96];
            std::snprintf(times, sizeof times, "%.4f ms (default %.4f ms) ", e.best_ms,
                          e.default_ms);
            out << e.op << ' ' << e.device << " v" << e.version << ' ' << e.key << " -> "
                << mensurflow::to_string(e.config) << " | " << times << e.mode << '\n';
        }
    }
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

const std::string& machine_name() {
    static const std::string name = [] {
        std::string text = processor_name();
        const Registry& registry = Registry::instance();
        for (const Device& device : registry.devices()) {
            if (device.type != DeviceType::CPU) {
                text += " | " + registry.get(device).info(device.index).name;
                break;
            }
        }
        return text;
    }();
    return name;
}

std::string call_key(const TunableKernel& tunable, const OpArgs& args, Device device) {
    const std::vector<std::int64_t> values = tunable.key(args);
    TuningValues named;
    for (std::size_t i = 0; i < std::min(values.size(), tunable.key_names.size()); ++i) {
        named.emplace_back(tunable.key_names[i], values[i]);
    }
    if (device.type == DeviceType::CPU) {
        // The CPU's kernels split work over threads, so their best settings depend on the count.
        named.emplace_back("threads", cpu_threads());
    }
    return mensurflow::to_string(named);
}

std::string placement_key(const OpArgs& args, Device data_device) {
    std::string key = "data=";
    key += device_type_name(data_device.type);
    key += ' ';
    key += dtype_name(args.inputs.at(0).dtype());
    for (const Tensor& input : args.inputs) {
        key += ' ' + shape_words(input.shape());
    }
    return key;
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

TuningScope::TuningScope(TuningContext context) : context_(context), outer_(t_context) {
    t_context = &context_;
}

TuningScope::~TuningScope() { t_context = outer_; }

bool tuning_active() { return t_context != nullptr; }

Device apply_tuning(OpId op, Execution execution, Device data_device, OpArgs& args) {
    const TuningContext& context = *t_context;
    const TuningCache* results = context.cache;
    // 1. The device: a stored choice replaces Auto; everything else resolves as usual.
    Execution resolved = execution;
    if (results != nullptr && execution == Execution::Auto && !args.inputs.empty()) {
        const TuningEntry* choice = results->find(machine_name(), op_name(op), kAutoDevice, 1,
                                                  placement_key(args, data_device));
        if (choice != nullptr) {
            resolved = setting(choice->config, "gpu", 0) != 0 ? Execution::GPU : Execution::CPU;
        }
    }
    const Device target = execution_device(resolved, data_device);
    if (context.record != nullptr) {
        context.record->push_back(RecordedCall{op, execution, data_device, target, args});
    }
    // 2. The settings of the kernel that runs there, when it is tunable and a result is stored.
    if (results != nullptr) {
        const DType dtype = (args.inputs.empty() ? args.outputs.at(0) : args.inputs[0]).dtype();
        const TunableKernel* tunable =
            Registry::instance().dispatcher().tunable({op, target.type, dtype});
        if (tunable != nullptr) {
            const TuningEntry* stored =
                results->find(machine_name(), tunable->name, device_type_name(target.type),
                              tunable->version, call_key(*tunable, args, target));
            if (stored != nullptr) {
                args.tuning = to_config(*tunable, stored->config);
            }
        }
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
