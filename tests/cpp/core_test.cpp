// Host-layer core: device naming, the op table, execution-device rules, registry, Tensor views
// and transfers on every device (the behaviours the reference's tests/core/dispatcher_test.cpp,
// transfer_test.cpp and device tests pin).
#include "core/dispatcher.hpp"
#include "core/registry.hpp"
#include "core/tensor_access.hpp"
#include "oracle_cpu.hpp"
#include "test_util.hpp"

#include <cstdint>
#include <cstdlib>
#include <numeric>
#include <string>
#include <vector>

using namespace mensurflow;
using detail::Dispatcher;
using detail::KernelKey;
using detail::OpArgs;
using detail::OpId;

namespace {

void noop_kernel(const OpArgs&, detail::Stream&) {}

void test_device_names() {
    test::require(to_string(Device{DeviceType::ROCm, 1}) == "rocm:1", "rocm:1 name");
    test::require(parse_device("ROCm") == (Device{DeviceType::ROCm, 0}), "parse rocm");
    test::require(parse_device("rocm:3") == (Device{DeviceType::ROCm, 3}), "parse rocm:3");
    test::require(parse_device("cpu") == (Device{DeviceType::CPU, 0}), "parse cpu");
    test::require_throws<std::invalid_argument>([] { parse_device("tpu:0"); }, "unknown type");
    test::require_throws<std::invalid_argument>([] { parse_device("rocm:-1"); }, "negative index");
    test::require_throws<std::invalid_argument>([] { parse_device("rocm:"); }, "empty index");
}

void test_dispatcher_table() {
    Dispatcher d;
    const KernelKey key{OpId::Matmul, DeviceType::ROCm, DType::F32};
    test::require(d.find(key) == nullptr, "empty table");
    d.register_kernel(key, noop_kernel);
    test::require(d.find(key) == noop_kernel, "registered kernel is found");
    test::require_throws<std::logic_error>([&] { d.register_kernel(key, noop_kernel); },
                                           "duplicate registration");
    test::require_throws<std::invalid_argument>(
        [&] { d.register_kernel({OpId::Gemv, DeviceType::ROCm, DType::F32}, nullptr); },
        "null kernel");
    try {
        d.lookup({OpId::Softmax, DeviceType::ROCm, DType::I32});
        throw std::runtime_error("lookup of a missing kernel did not throw");
    } catch (const detail::NotImplemented& e) {
        const std::string what = e.what();
        test::require(what.find("softmax") != std::string::npos &&
                          what.find("rocm") != std::string::npos &&
                          what.find("i32") != std::string::npos,
                      "NotImplemented names op, device and dtype: " + what);
    }
}

void test_execution_device() {
    test::require(detail::execution_device(Execution::CPU, {DeviceType::ROCm, 0}) ==
                      (Device{DeviceType::CPU, 0}),
                  "CPU runs on cpu:0");
    test::require(detail::execution_device(Execution::Auto, {DeviceType::CPU, 0}) ==
                      (Device{DeviceType::CPU, 0}),
                  "Auto runs on cpu:0");
    test::require(detail::execution_device(Execution::GPU, {DeviceType::ROCm, 0}) ==
                      (Device{DeviceType::ROCm, 0}),
                  "GPU keeps the data's GPU");
    const bool has_gpu = detail::Registry::instance().find(DeviceType::ROCm) != nullptr;
    if (has_gpu) {
        test::require(detail::execution_device(Execution::GPU, {DeviceType::CPU, 0}) ==
                          (Device{DeviceType::ROCm, 0}),
                      "GPU from CPU data picks rocm:0");
    } else {
        test::require_throws<std::runtime_error>(
            [] { detail::execution_device(Execution::GPU, {DeviceType::CPU, 0}); },
            "GPU with no GPU throws");
    }
}

void test_registry_and_default_device() {
    const auto devices = list_devices();
    test::require(!devices.empty() && devices[0] == (Device{DeviceType::CPU, 0}), "CPU first");
    test::require_throws<std::runtime_error>(
        [] { Tensor::empty({2}, DType::F32, {DeviceType::ROCm, 99}); }, "unavailable device");
    setenv("MENSURFLOW_DEVICE", "vulkan:0", 1);
    test::require_throws<std::runtime_error>([] { default_device(); },
                                             "MENSURFLOW_DEVICE names a missing device");
    setenv("MENSURFLOW_DEVICE", "cpu", 1);
    test::require(default_device() == (Device{DeviceType::CPU, 0}), "MENSURFLOW_DEVICE=cpu");
    unsetenv("MENSURFLOW_DEVICE");
    const bool has_gpu = device_available({DeviceType::ROCm, 0});
    test::require(default_device().type == (has_gpu ? DeviceType::ROCm : DeviceType::CPU),
                  "default device prefers a GPU");
}

std::vector<float> iota(std::int64_t n) {
    std::vector<float> v(static_cast<std::size_t>(n));
    std::iota(v.begin(), v.end(), 0.0f);
    return v;
}

void test_transfers(Device device) {
    const auto values = iota(2 * 3 * 4);
    const Tensor t = Tensor::from_vector(values, {2, 3, 4}, device);
    test::require(t.device() == device && t.is_contiguous(), "from_vector");
    test::require(t.to_vector<float>() == values, "round trip");
    // A transposed view read back follows strides; contiguous() packs it (on the device for rocm).
    const Tensor tt = t.transpose(0, 2);
    std::vector<float> want;
    for (int c = 0; c < 4; ++c) {
        for (int b = 0; b < 3; ++b) {
            for (int a = 0; a < 2; ++a) {
                want.push_back(values[static_cast<std::size_t>(a * 12 + b * 4 + c)]);
            }
        }
    }
    test::require(tt.to_vector<float>() == want, "strided read-back");
    const Tensor packed = tt.contiguous();
    test::require(packed.is_contiguous() && packed.device() == device &&
                      packed.to_vector<float>() == want,
                  "contiguous() on " + to_string(device));
    // Slices and broadcasts.
    test::require(t.slice(1, 1, 3).to_vector<float>().size() == 16, "slice");
    const Tensor row = Tensor::from_vector(std::vector<float>{1, 2, 3}, {3}, device);
    const auto expanded = row.expand({2, 3}).contiguous().to_vector<float>();
    test::require(expanded == (std::vector<float>{1, 2, 3, 1, 2, 3}), "expand + contiguous");
    // Bool and I64 tensors move too.
    const Tensor mask = Tensor::full({2, 2}, 1.0, DType::Bool, device);
    std::vector<std::uint8_t> bytes(4);
    mask.transpose(0, 1).copy_to_host(bytes.data());
    test::require(bytes == (std::vector<std::uint8_t>{1, 1, 1, 1}), "bool round trip");
    const Tensor idx = Tensor::from_vector(std::vector<std::int64_t>{7, -3}, {2}, device);
    test::require(idx.to_vector<std::int64_t>() == (std::vector<std::int64_t>{7, -3}), "i64");
    // copy_from into a contiguous destination stays on the device.
    Tensor dst = Tensor::zeros({4, 3, 2}, DType::F32, device);
    dst.copy_from(tt);
    test::require(dst.to_vector<float>() == want, "copy_from a view");
    // to() between devices.
    const Tensor back = t.to({DeviceType::CPU, 0});
    test::require(back.device() == (Device{DeviceType::CPU, 0}) && back.to_vector<float>() == values,
                  "to(cpu)");
    // to() from host views onto this device: a transposed view and a broadcast (their spans
    // move and the device packs them), a sparse slice (packed on the host), a view with an
    // offset; each arrives on another device contiguous, with the view's values.
    const Device cpu{DeviceType::CPU, 0};
    const auto big = iota(64 * 48);
    const Tensor host = Tensor::from_vector(big, {64, 48}, cpu);
    const Tensor host_row = Tensor::from_vector(std::vector<float>{5, -1, 2}, {1, 3}, cpu);
    const std::vector<Tensor> views = {host.transpose(0, 1), host_row.expand({40, 3}),
                                       host.slice(1, 0, 48, 16), host.slice(0, 3, 60).slice(1, 5, 41)};
    for (const Tensor& view : views) {
        const Tensor moved = view.to(device);
        // (On the CPU, to() returns the view itself.)
        test::require(moved.device() == device && (device == cpu || moved.is_contiguous()) &&
                          moved.shape() == view.shape() &&
                          moved.to_vector<float>() == view.to_vector<float>(),
                      "to(" + to_string(device) + ") of a host view " + to_string(view.shape()));
    }
    // A 9-dimensional transposed view: more dimensions than a device's strided copy takes
    // (MFR_MAX_COPY_DIMS on rocm), so to() gathers it on the host, and contiguous() and the
    // read-back of the device-resident view go through host memory.
    {
        const Shape shape9 = {2, 1, 3, 1, 2, 1, 2, 3, 2};
        const auto nine = iota(numel(shape9));
        const Tensor host9 = Tensor::from_vector(nine, shape9, cpu).transpose(0, 8);
        const std::vector<float> want9 = host9.to_vector<float>();
        const Tensor moved9 = host9.to(device);
        test::require(moved9.device() == device && moved9.shape() == host9.shape() &&
                          moved9.to_vector<float>() == want9,
                      "to(" + to_string(device) + ") of a 9-D transposed host view");
        const Tensor dev9 = Tensor::from_vector(nine, shape9, device).transpose(0, 8);
        test::require(dev9.to_vector<float>() == want9, "read-back of a 9-D device view");
        const Tensor packed9 = dev9.contiguous();
        test::require(packed9.is_contiguous() && packed9.device() == device &&
                          packed9.to_vector<float>() == want9,
                      "contiguous() of a 9-D view on " + to_string(device));
    }
    // Empty tensors.
    test::require(Tensor::empty({0, 5}, DType::F32, device).to_vector<float>().empty(), "empty");
}

// A dropped tensor's device memory serves the next allocation of its size at once, while a
// kernel that reads it may still be queued on the device's stream. Products whose inputs are
// released before the result is read, followed by fills of new tensors of those sizes, must read
// the inputs they were given. Quarter-integer values make every sum exact.
void test_released_memory_reuse(Device device) {
    const auto on = test::execution_on(device);
    for (int round = 0; round < 24; ++round) {
        const std::int64_t m = 64 + 8 * (round % 5), k = 96, n = 40 + round;
        std::vector<float> av(static_cast<std::size_t>(m * k)), bv(static_cast<std::size_t>(k * n));
        for (std::size_t i = 0; i < av.size(); ++i) {
            av[i] = static_cast<float>(static_cast<int>((i * 7 + round) % 13) - 6) / 4.0f;
        }
        for (std::size_t i = 0; i < bv.size(); ++i) {
            bv[i] = static_cast<float>(static_cast<int>((i * 5 + round) % 11) - 5) / 4.0f;
        }
        Tensor c;
        {
            const Tensor a = Tensor::from_vector(av, {m, k}, device);
            const Tensor b = Tensor::from_vector(bv, {k, n}, device);
            c = matmul(a, b, on);
        } // a and b are released before the product is read back
        const Tensor over_a = Tensor::full({m, k}, -1000.0, DType::F32, device);
        const Tensor over_b = Tensor::full({k, n}, 1000.0, DType::F32, device);
        std::vector<float> want(static_cast<std::size_t>(m * n));
        for (std::int64_t i = 0; i < m; ++i) {
            for (std::int64_t j = 0; j < n; ++j) {
                double sum = 0.0;
                for (std::int64_t p = 0; p < k; ++p) {
                    sum += static_cast<double>(av[static_cast<std::size_t>(i * k + p)]) *
                           bv[static_cast<std::size_t>(p * n + j)];
                }
                want[static_cast<std::size_t>(i * n + j)] = static_cast<float>(sum);
            }
        }
        test::require(c.to_vector<float>() == want,
                      "product after its inputs were released, round " + std::to_string(round));
        test::require(over_a.to_vector<float>()[0] == -1000.0f &&
                          over_b.to_vector<float>().back() == 1000.0f,
                      "fills of reused memory");
    }
}

void test_run_elsewhere() {
    // Data on the CPU, op on the GPU: inputs copied over, result written back into the CPU output.
    if (!device_available({DeviceType::ROCm, 0}) || test::options().cpu_only) {
        return;
    }
    const Tensor a = Tensor::from_vector(std::vector<float>{1, 2, 3, 4, 5, 6}, {2, 3});
    const Tensor b = Tensor::from_vector(std::vector<float>{7, 8, 9, 10, 11, 12}, {3, 2});
    const Tensor c = matmul(a, b, Execution::GPU);
    test::require(c.device() == (Device{DeviceType::CPU, 0}), "result stays on the data's device");
    test::require(c.to_vector<float>() == (std::vector<float>{58, 64, 139, 154}),
                  "GPU result written back");
    test::require_throws<std::invalid_argument>(
        [&] { matmul(a, b.to({DeviceType::ROCm, 0}), Execution::GPU); }, "mixed devices");
}

// ---- trace spans (mensurflow/trace.hpp) ------------------------------------------------------

std::vector<trace::Event>& recorded() {
    static std::vector<trace::Event> events;
    return events;
}

void record(const trace::Event& event) { recorded().push_back(event); }

const trace::Event* find_event(const std::vector<trace::Event>& events, const std::string& name) {
    for (const trace::Event& e : events) {
        if (name == e.name) {
            return &e;
        }
    }
    return nullptr;
}

// With a hook attached, a matmul on `device` reports its op span with the operands' shapes, a
// "kernel" span inside it, the allocation of its result, and the read-back; detached, nothing.
// main() sets MENSURFLOW_TRACE_SYNC before the first span, so on rocm a kernel span covers the
// kernel itself: a 2048^3 product (~130 us on one MI355X) cannot close in the few microseconds
// its launch takes.
void test_trace_spans(Device device) {
    const Execution on = test::execution_on(device);
    const Tensor a = Tensor::full({64, 32}, 1.0, DType::F32, device);
    const Tensor b = Tensor::full({32, 16}, 2.0, DType::F32, device);
    recorded().clear();
    trace::hook.store(&record);
    const Tensor c = matmul(a, b, on);
    const std::vector<float> values = c.to_vector<float>();
    trace::hook.store(nullptr);
    const std::vector<trace::Event> events = recorded();
    test::require(values.size() == 64 * 16 && values[0] == 64.0f, "traced matmul's values");
    const trace::Event* op = find_event(events, "matmul");
    test::require(op != nullptr && op->device == device && op->dtype == DType::F32 &&
                      op->inputs == (std::vector<Shape>{{64, 32}, {32, 16}}) &&
                      op->outputs == (std::vector<Shape>{{64, 16}}),
                  "matmul span: device, dtype, shapes");
    const trace::Event* kernel = find_event(events, "kernel");
    test::require(kernel != nullptr && kernel->device == device &&
                      kernel->start_ns >= op->start_ns && kernel->end_ns <= op->end_ns &&
                      kernel->start_ns <= kernel->end_ns,
                  "kernel span inside the op span");
    const trace::Event* alloc = find_event(events, "Tensor::empty");
    test::require(alloc != nullptr && alloc->outputs == (std::vector<Shape>{{64, 16}}),
                  "the result's allocation");
    test::require(find_event(events, "Tensor::copy_to_host") != nullptr, "the read-back");
    recorded().clear();
    (void)matmul(a, b, on);
    test::require(recorded().empty(), "no events without a hook");

    if (device.type == DeviceType::ROCm) {
        const Tensor x = Tensor::full({2048, 2048}, 0.5, DType::F32, device);
        (void)matmul(x, x, on).to_vector<float>(); // the plan and code loading, untraced
        recorded().clear();
        trace::hook.store(&record);
        const Tensor y = matmul(x, x, on);
        trace::hook.store(nullptr);
        const trace::Event* big = find_event(recorded(), "kernel");
        test::require(big != nullptr && big->end_ns - big->start_ns >= 60000,
                      "under MENSURFLOW_TRACE_SYNC the kernel span covers the device's work");
        test::require(y.to_vector<float>()[0] == 512.0f, "traced 2048^3 product");
    }
}

// Host tensors of 4 MiB or more start on a 2 MiB boundary (their memory asks for transparent huge
// pages, so a first write faults once per 2 MiB); smaller ones on a 64-byte line. A large one
// goes to every device and back unchanged.
void test_large_host_buffers() {
    const Device cpu{DeviceType::CPU, 0};
    const Tensor small = Tensor::zeros({1000}, DType::F32, cpu);
    const auto small_at = reinterpret_cast<std::uintptr_t>(detail::TensorAccess::data<float>(small));
    test::require(small_at % 64 == 0, "a small host buffer starts on a 64-byte line");
    const std::int64_t n = (std::int64_t{6} << 20) / 4 + 7; // a little over 6 MiB
    const auto values = iota(n);
    const Tensor big = Tensor::from_vector(values, {n}, cpu);
    const auto big_at = reinterpret_cast<std::uintptr_t>(detail::TensorAccess::data<float>(big));
    test::require(big_at % (std::uintptr_t{2} << 20) == 0,
                  "a host buffer of 4 MiB or more starts on a 2 MiB boundary");
    for (Device device : test::devices()) {
        const Tensor there = big.to(device);
        test::require(there.to(cpu).to_vector<float>() == values,
                      "a 6 MiB host tensor through " + to_string(device) + " and back");
    }
}

} // namespace

int main(int argc, char** argv) {
    // Read once, at the first span: the rocm kernel spans of test_trace_spans wait for the device.
    setenv("MENSURFLOW_TRACE_SYNC", "1", 1);
    return test::run("core_test", argc, argv, [] {
        test::register_oracle_cpu_kernels();
        test_device_names();
        test_dispatcher_table();
        test_execution_device();
        test_registry_and_default_device();
        for (Device device : test::devices()) {
            std::cout << "  transfers on " << to_string(device) << '\n';
            test_transfers(device);
            test_released_memory_reuse(device);
            test_trace_spans(device);
        }
        test_run_elsewhere();
        test_large_host_buffers();
    });
}
