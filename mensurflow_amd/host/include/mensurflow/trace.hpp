// Spans around the points where a call spends its time: the public contract of mensurflow's
// include/mensurflow/trace.hpp:1-104 (the Event a hook receives, the `hook` pointer, the
// MENSURFLOW_TRACE macro), so a collector written for mensurflow attaches here unchanged.
//
// With MENSURFLOW_ENABLE_TRACING defined (this repository's build defines it for libmensurflow.so
// and everything compiled against it), MENSURFLOW_TRACE(...) opens a span that closes at the end of
// the enclosing scope and then hands one Event to `hook`. Without a hook a span costs one relaxed
// atomic load. Without the definition the macro expands to nothing and its arguments are not
// evaluated.
//
// The library produces events and never stores or prints them. Spans sit in the dispatcher (one
// named after the op, one named "kernel" around the backend call) and in Tensor's allocation and
// copies (empty, from_host, to, contiguous, copy_from, copy_to_host).
//
// On a GPU a "kernel" span closes when the launch returns, while the kernel may still run. With
// MENSURFLOW_TRACE_SYNC set to anything but "" or "0" (read once, at the first span) and a hook
// attached, the dispatcher waits for the device's stream before closing each "kernel" span, so
// its duration covers the kernel itself. That serialises host and device: it is for profiling.
#pragma once

#ifdef MENSURFLOW_ENABLE_TRACING

#include "mensurflow/device.hpp"
#include "mensurflow/dtype.hpp"
#include "mensurflow/shape.hpp"
#include "mensurflow/tensor.hpp"

#include <atomic>
#include <chrono>
#include <cstdint>
#include <cstdlib>
#include <vector>

namespace mensurflow::trace {

struct Event {
    const char* name;           // the op ("matmul"), "kernel", or a Tensor step ("Tensor::to")
    Device device;              // where it ran
    DType dtype;                // the dtype its kernel was chosen for
    std::vector<Shape> inputs;  // input shapes
    std::vector<Shape> outputs; // output shapes
    std::int64_t start_ns;      // steady_clock
    std::int64_t end_ns;
};

using Hook = void (*)(const Event& event);

// The listener; null (the default) turns every span into a single load.
inline std::atomic<Hook> hook{nullptr};

namespace detail {

inline std::int64_t steady_ns() {
    const auto since = std::chrono::steady_clock::now().time_since_epoch();
    return std::chrono::duration_cast<std::chrono::nanoseconds>(since).count();
}

inline bool listening() { return hook.load(std::memory_order_relaxed) != nullptr; }

// Whether "kernel" spans wait for the device: MENSURFLOW_TRACE_SYNC, with a hook attached.
inline bool waits_for_device() {
    static const bool requested = [] {
        const char* value = std::getenv("MENSURFLOW_TRACE_SYNC");
        return value != nullptr && value[0] != '\0' && !(value[0] == '0' && value[1] == '\0');
    }();
    return requested && listening();
}

inline std::vector<Shape> shapes_of(const std::vector<Tensor>& tensors) {
    std::vector<Shape> shapes;
    shapes.reserve(tensors.size());
    for (const Tensor& t : tensors) {
        shapes.push_back(t.shape());
    }
    return shapes;
}

} // namespace detail

class Span {
  public:
    // An op or a kernel call: the dtype is that of the first input (a factory's first output).
    Span(const char* name, Device device, const std::vector<Tensor>& inputs,
         const std::vector<Tensor>& outputs)
        : live_(detail::listening()) {
        if (live_) {
            const std::vector<Tensor>& anchor = inputs.empty() ? outputs : inputs;
            event_ = Event{name,
                           device,
                           anchor.empty() ? DType::F32 : anchor.front().dtype(),
                           detail::shapes_of(inputs),
                           detail::shapes_of(outputs),
                           detail::steady_ns(),
                           0};
        }
    }

    // A step on one tensor (an allocation, a copy): its shape as the one output.
    Span(const char* name, Device device, const Shape& shape, DType dtype)
        : live_(detail::listening()) {
        if (live_) {
            event_ = Event{name, device, dtype, {}, {shape}, detail::steady_ns(), 0};
        }
    }

    Span(const Span&) = delete;
    Span& operator=(const Span&) = delete;

    ~Span() {
        if (!live_) {
            return;
        }
        event_.end_ns = detail::steady_ns();
        if (const Hook listener = hook.load(std::memory_order_relaxed)) {
            listener(event_);
        }
    }

  private:
    bool live_;
    Event event_{};
};

} // namespace mensurflow::trace

#define MENSURFLOW_TRACE_JOIN2(a, b) a##b
#define MENSURFLOW_TRACE_JOIN(a, b) MENSURFLOW_TRACE_JOIN2(a, b)
#define MENSURFLOW_TRACE(...)                                                                     \
    ::mensurflow::trace::Span MENSURFLOW_TRACE_JOIN(mensurflow_trace_span_, __LINE__)(__VA_ARGS__)

#else

#define MENSURFLOW_TRACE(...) ((void)0)

#endif
