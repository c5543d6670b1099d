// Minimal helpers for the C++ tests of the host layer: each test is an executable returning
// non-zero on failure (the reference's test style). Flags: --cpu-only skips GPU devices,
// --require-gpu fails when no rocm device is listed.
#pragma once

#include "mensurflow/mensurflow.hpp"

#include <cmath>
#include <cstring>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

namespace test {

struct Options {
    bool cpu_only = false;
    bool require_gpu = false;
};

inline Options& options() {
    static Options opts;
    return opts;
}

inline void parse(int argc, char** argv) {
    for (int i = 1; i < argc; ++i) {
        const std::string arg = argv[i];
        if (arg == "--cpu-only") {
            options().cpu_only = true;
        } else if (arg == "--require-gpu") {
            options().require_gpu = true;
        }
    }
}

// The devices a test loops over: CPU first, then rocm unless --cpu-only.
inline std::vector<mensurflow::Device> devices() {
    std::vector<mensurflow::Device> out;
    bool gpu = false;
    for (mensurflow::Device d : mensurflow::list_devices()) {
        if (d.type != mensurflow::DeviceType::CPU) {
            gpu = true;
            if (options().cpu_only) {
                continue;
            }
        }
        out.push_back(d);
    }
    if (options().require_gpu && !gpu) {
        throw std::runtime_error("--require-gpu: no rocm device is listed");
    }
    return out;
}

inline mensurflow::Execution execution_on(mensurflow::Device device) {
    return device.type == mensurflow::DeviceType::CPU ? mensurflow::Execution::CPU
                                                      : mensurflow::Execution::GPU;
}

inline void require(bool condition, const std::string& message) {
    if (!condition) {
        throw std::runtime_error(message);
    }
}

template <typename E, typename Fn> void require_throws(Fn&& fn, const std::string& message) {
    try {
        fn();
    } catch (const E&) {
        return;
    } catch (const std::exception& e) {
        throw std::runtime_error("expected a different exception (" + message + "), got: " +
                                 e.what());
    }
    throw std::runtime_error("expected exception: " + message);
}

inline bool same_bits(const std::vector<float>& a, const std::vector<float>& b) {
    return a.size() == b.size() &&
           (a.empty() || std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0);
}

// Multiples of 0.25 in [-4, 4] from an LCG (the reference tests' generator): fp32 sums of their
// products are exact in any order.
inline std::vector<float> quarter_input(std::int64_t n, std::uint32_t seed) {
    std::vector<float> v(static_cast<std::size_t>(n));
    std::uint32_t state = seed;
    for (auto& x : v) {
        state = state * 1664525u + 1013904223u;
        x = static_cast<float>(static_cast<int>(state >> 12) % 33 - 16) / 4;
    }
    return v;
}

template <typename Fn> int run(const char* name, int argc, char** argv, Fn&& body) {
    try {
        parse(argc, argv);
        body();
    } catch (const std::exception& e) {
        std::cerr << name << " FAILED: " << e.what() << '\n';
        return 1;
    }
    std::cout << name << " passed\n";
    return 0;
}

} // namespace test
