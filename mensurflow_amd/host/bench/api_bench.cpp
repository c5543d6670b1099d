// Times the BASELINE workloads through the mensurflow C++ API on the rocm device: the calls a
// mensurflow user makes (mensurflow::gemm, gemv, gemm_epilogue, attention with Execution::GPU),
// each returning a new tensor, so the figures include the dispatcher, the backend's kernel
// adapters, the output allocation and the C ABI on top of the kernels. Host wall time over runs
// of calls ended by a read-back, which waits for the device's stream. Prints one JSON line.
//
// usage: mfr_api_bench [calls]
#include "mensurflow/mensurflow.hpp"

#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

using namespace mensurflow;

namespace {

std::vector<float> values(std::size_t count, std::uint32_t seed, float scale) {
    std::vector<float> out(count);
    std::uint32_t state = seed * 2654435761u + 1u;
    for (auto& v : out) {
        state = state * 1664525u + 1013904223u;
        v = scale * (static_cast<float>(state >> 8) * (1.0f / 16777216.0f) * 2.0f - 1.0f);
    }
    return out;
}

Tensor random(Shape shape, std::uint32_t seed, float scale, Device device) {
    std::size_t count = 1;
    for (auto s : shape) {
        count *= static_cast<std::size_t>(s);
    }
    return Tensor::from_vector(values(count, seed, scale), shape, device);
}

double elapsed_ms(std::chrono::steady_clock::time_point since) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - since)
        .count();
}

// Microseconds per call. Untimed calls first, for at least 50 ms: the clocks ramp up over the
// first ~10 ms of work after the GPU was idle. Then runs of `calls` calls, each ended by a
// read-back (which waits for the stream), until at least 50 ms have been timed.
template <typename Fn> double time_us(Fn&& fn, int calls, const Tensor& probe) {
    const auto warm = std::chrono::steady_clock::now();
    do {
        for (int i = 0; i < calls; ++i) {
            fn();
        }
        (void)probe.to_vector<float>();
    } while (elapsed_ms(warm) < 50.0);
    const auto start = std::chrono::steady_clock::now();
    long total = 0;
    do {
        for (int i = 0; i < calls; ++i) {
            fn();
        }
        (void)probe.to_vector<float>();
        total += calls;
    } while (elapsed_ms(start) < 50.0);
    return elapsed_ms(start) * 1e3 / static_cast<double>(total);
}

} // namespace

int main(int argc, char** argv) {
    const int calls = argc > 1 ? std::atoi(argv[1]) : 20;
    const Device gpu{DeviceType::ROCm, 0};
    if (!device_available(gpu)) {
        std::fprintf(stderr, "mfr_api_bench: no rocm device\n");
        return 2;
    }
    const auto on = Execution::GPU;
    const Tensor probe = Tensor::zeros({1}, DType::F32, gpu);

    // 4096^3, B transposed, alpha 1.5, beta 0.5.
    const std::int64_t n = 4096;
    const Tensor a = random({n, n}, 1, 1.0f, gpu);
    const Tensor b = random({n, n}, 2, 1.0f, gpu);
    const Tensor c0 = random({n, n}, 3, 1.0f, gpu);
    const double gemm_us =
        time_us([&] { (void)gemm(a, b, 1.5f, &c0, 0.5f, false, true, on); }, calls, probe);

    // gemv 16384^2, alpha 2, beta 0.5, A x and A^T x.
    const std::int64_t g = 16384;
    const Tensor ga = random({g, g}, 4, 1.0f, gpu);
    const Tensor gx = random({g}, 5, 1.0f, gpu);
    const Tensor gy = random({g}, 6, 1.0f, gpu);
    const double gemv_n_us =
        time_us([&] { (void)gemv(ga, gx, 2.0f, &gy, 0.5f, false, on); }, calls, probe);
    const double gemv_t_us =
        time_us([&] { (void)gemv(ga, gx, 2.0f, &gy, 0.5f, true, on); }, calls, probe);

    // X[4093,1023] W[1023,4099] + bias, tanh gelu.
    const Tensor x = random({4093, 1023}, 7, 1.0f, gpu);
    const Tensor w = random({1023, 4099}, 8, 0.03f, gpu);
    const Tensor bias = random({4099}, 9, 0.1f, gpu);
    const double mlp_us = time_us(
        [&] { (void)gemm_epilogue(x, w, &bias, Activation::GeluTanh, 1.0f, nullptr, 0.0f, false,
                                  false, on); },
        calls, probe);

    // attention [8, 16, 1024, 64], causal.
    const Tensor q = random({8, 16, 1024, 64}, 10, 1.0f, gpu);
    const Tensor k = random({8, 16, 1024, 64}, 11, 1.0f, gpu);
    const Tensor v = random({8, 16, 1024, 64}, 12, 1.0f, gpu);
    const double attention_us =
        time_us([&] { (void)attention(q, k, v, nullptr, true, 0.0f, on); }, calls, probe);

    // The same GEMM and gemv N with the operands in host memory: Execution::GPU copies them to
    // the device, runs the kernel and copies the result back (pageable, synchronous copies, as
    // the reference's GPU backends do), so these calls include the PCIe transfers. One call per
    // run; the result is a host tensor, so each call has finished when it returns.
    const Device cpu{DeviceType::CPU, 0};
    const Tensor ha = a.to(cpu), hb = b.to(cpu), hc0 = c0.to(cpu);
    const double host_gemm_us =
        time_us([&] { (void)gemm(ha, hb, 1.5f, &hc0, 0.5f, false, true, on); }, 1, probe);
    const Tensor hga = ga.to(cpu), hgx = gx.to(cpu), hgy = gy.to(cpu);
    const double host_gemv_us =
        time_us([&] { (void)gemv(hga, hgx, 2.0f, &hgy, 0.5f, false, on); }, 1, probe);

    const double gemm_tflops = 2.0 * n * n * n / (gemm_us * 1e-6) / 1e12;
    const double gemv_bytes = 4.0 * (static_cast<double>(g) * g + 3.0 * g);
    std::printf("{\"calls_per_run\": %d, \"gemm_4096_us\": %.1f, \"gemm_4096_tflops\": %.2f, "
                "\"gemv_n_us\": %.2f, \"gemv_n_gbs\": %.1f, \"gemv_t_us\": %.2f, "
                "\"gemv_t_gbs\": %.1f, \"mlp_us\": %.1f, \"attention_cfg5_us\": %.1f, "
                "\"host_resident_gemm_4096_ms\": %.2f, \"host_resident_gemm_4096_tflops\": %.2f, "
                "\"host_resident_gemv_n_ms\": %.2f, \"host_resident_gemv_n_gbs\": %.1f}\n",
                calls, gemm_us, gemm_tflops, gemv_n_us, gemv_bytes / (gemv_n_us * 1e-6) / 1e9,
                gemv_t_us, gemv_bytes / (gemv_t_us * 1e-6) / 1e9, mlp_us, attention_us,
                host_gemm_us * 1e-3, 2.0 * n * n * n / (host_gemm_us * 1e-6) / 1e12,
                host_gemv_us * 1e-3, gemv_bytes / (host_gemv_us * 1e-6) / 1e9);
    return 0;
}
