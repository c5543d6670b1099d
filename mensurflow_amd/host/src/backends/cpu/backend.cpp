// The CPU device of this build: host memory and a queue that runs everything at once. It holds no
// compute kernels. In a mensurflow tree the CPU backend is mensurflow's own, with its kernels;
// this repository ships the ROCm backend, and its C++ tests install the CPU oracle's kernels here
// (tests/cpp/oracle_cpu.cpp).
#include "backends/backend.hpp"
#include "core/dispatcher.hpp"
#include "core/registry.hpp"

#include <sys/mman.h>

#include <cstdlib>
#include <cstring>
#include <new>

namespace mensurflow::detail {

namespace {

// Host allocations start on a cache line, which also suits the widest vector loads.
constexpr std::size_t kLine = 64;

// Allocations of at least kHugeFrom bytes start on a 2 MiB boundary, span whole 2 MiB pages and
// ask the kernel for transparent huge pages (where the system allows them on request), so their
// first write takes one fault per 2 MiB instead of one per 4 KiB: a new 64 MiB host tensor
// filled from the device measured 11-15 ms of 4 KiB faults on an MI355X box's host, 3-4.6 ms
// with huge pages. Where the request is refused the memory is ordinary memory.
constexpr std::size_t kHugePage = std::size_t{2} << 20;
constexpr std::size_t kHugeFrom = std::size_t{4} << 20;

struct FreeWithFree {
    void operator()(std::byte* p) const { std::free(p); }
};

class HostBuffer final : public Buffer {
  public:
    explicit HostBuffer(std::size_t bytes) : bytes_(bytes) {
        if (bytes == 0) {
            return; // a zero-byte buffer has no address
        }
        const std::size_t align = bytes >= kHugeFrom ? kHugePage : kLine;
        const std::size_t rounded = (bytes + align - 1) / align * align;
        memory_.reset(static_cast<std::byte*>(std::aligned_alloc(align, rounded)));
        if (!memory_) {
            throw std::bad_alloc();
        }
        if (align == kHugePage) {
            (void)madvise(memory_.get(), rounded, MADV_HUGEPAGE); // a hint; refusal is harmless
        }
    }
    std::size_t size() const override { return bytes_; }
    void* native() const override { return memory_.get(); }
    void* host_ptr() const override { return memory_.get(); }

  private:
    std::size_t bytes_;
    std::unique_ptr<std::byte, FreeWithFree> memory_;
};

std::byte* at(const Buffer& buffer, std::size_t offset) {
    return static_cast<std::byte*>(buffer.native()) + offset;
}

// Host work finishes before the call returns, so there is never anything to wait for.
class InlineQueue final : public Stream {
  public:
    void copy_h2d(Buffer& dst, std::size_t offset, const void* src, std::size_t bytes) override {
        std::memcpy(at(dst, offset), src, bytes);
    }
    void copy_d2h(void* dst, const Buffer& src, std::size_t offset, std::size_t bytes) override {
        std::memcpy(dst, at(src, offset), bytes);
    }
    void copy_d2d(Buffer& dst, std::size_t dst_offset, const Buffer& src, std::size_t src_offset,
                  std::size_t bytes) override {
        std::memmove(at(dst, dst_offset), at(src, src_offset), bytes); // ranges may overlap
    }
    void synchronize() override {}
};

class HostBackend final : public Backend {
  public:
    DeviceType type() const override { return DeviceType::CPU; }
    int device_count() const override { return 1; }
    DeviceInfo info(int) const override { return DeviceInfo{"cpu", 0}; }
    std::shared_ptr<Buffer> allocate(int, std::size_t bytes) override {
        return std::make_shared<HostBuffer>(bytes);
    }
    Stream& stream(int) override { return queue_; }
    void register_kernels(Dispatcher&) override {}

  private:
    InlineQueue queue_;
};

} // namespace

void register_cpu_backend(Registry& registry) { registry.add(std::make_unique<HostBackend>()); }

} // namespace mensurflow::detail
