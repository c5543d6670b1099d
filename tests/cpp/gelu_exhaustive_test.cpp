// The tanh gelu the HIP kernels run (mensurflow_amd/csrc/gelu_tanh.hpp), compiled here for the
// CPU with the same double operations, against the oracle's restatement of the reference
// (orc_gelu_f32, src/backends/cpu/ops/elementwise/elementwise.cpp:24-27,173-194): the same float
// bits for every input bit pattern taken (every one with --stride 1; NaN for both counts as equal).
// The device's reciprocal instruction is stood in for by 1/d, 1/d (1 + 2^-20) and 1/d (1 - 2^-20):
// the result must not depend on how close the reciprocal's start is.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {
int g_rcp_mode = 0;
double host_rcp(double d) {
    const double q = 1.0 / d;
    return g_rcp_mode == 0 ? q : g_rcp_mode == 1 ? q * (1.0 + 0x1.0p-20) : q * (1.0 - 0x1.0p-20);
}
} // namespace

#define MFR_GELU_RCP(d) host_rcp(d)
#include "gelu_tanh.hpp"
#include "oracle.h"

int main(int argc, char** argv) {
    int64_t stride = 1;
    for (int i = 1; i + 1 < argc; ++i) {
        if (std::string(argv[i]) == "--stride") {
            stride = std::atoll(argv[i + 1]);
        }
    }
    if (stride < 1) {
        std::fprintf(stderr, "--stride must be >= 1\n");
        return 2;
    }
    const int64_t total = (int64_t{1} << 32);
    const int64_t count = (total + stride - 1) / stride;
    constexpr int64_t kChunk = int64_t{1} << 16;
    const int64_t chunks = (count + kChunk - 1) / kChunk;
    bool ok = true;
    for (g_rcp_mode = 0; g_rcp_mode < 3; ++g_rcp_mode) {
        long long mismatches = 0;
        uint32_t first_bad = 0;
        bool any_bad = false;
#pragma omp parallel for schedule(dynamic, 16) reduction(+ : mismatches)
        for (int64_t c = 0; c < chunks; ++c) {
            const int64_t begin = c * kChunk;
            const int64_t n = count - begin < kChunk ? count - begin : kChunk;
            std::vector<float> x(static_cast<size_t>(n)), want(static_cast<size_t>(n));
            for (int64_t i = 0; i < n; ++i) {
                const uint32_t bits = static_cast<uint32_t>((begin + i) * stride);
                std::memcpy(&x[static_cast<size_t>(i)], &bits, 4);
            }
            orc_gelu_f32(x.data(), want.data(), n, 1);
            for (int64_t i = 0; i < n; ++i) {
                const float got = mfr::gelu_math::gelu_tanh(x[static_cast<size_t>(i)]);
                const float ref = want[static_cast<size_t>(i)];
                uint32_t gb, rb;
                std::memcpy(&gb, &got, 4);
                std::memcpy(&rb, &ref, 4);
                const bool same = gb == rb || (std::isnan(got) && std::isnan(ref));
                if (!same) {
                    ++mismatches;
#pragma omp critical
                    if (!any_bad) {
                        any_bad = true;
                        std::memcpy(&first_bad, &x[static_cast<size_t>(i)], 4);
                    }
                }
            }
        }
        std::printf("  reciprocal start %s: %lld inputs, %lld mismatches%s\n",
                    g_rcp_mode == 0 ? "exact" : g_rcp_mode == 1 ? "2^-20 high" : "2^-20 low",
                    static_cast<long long>(count), mismatches,
                    any_bad ? (" (first at bits 0x" + std::to_string(first_bad) + ")").c_str()
                            : "");
        ok = ok && mismatches == 0;
    }
    if (!ok) {
        std::printf("gelu_exhaustive_test FAILED\n");
        return 1;
    }
    std::printf("gelu_exhaustive_test passed\n");
    return 0;
}
