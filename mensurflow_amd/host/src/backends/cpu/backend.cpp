// The CPU device: host memory and inline "streams" (the reference's CpuBuffer/CpuStream,
// src/backends/cpu/backend.cpp:43-83). This backend registers no compute kernels: in a
// mensurflow build the reference's own CPU kernels sit here; this repository is the ROCm
// backend, and its tests plug the CPU oracle in at this point.
#include "backends/backend.hpp"
#include "core/dispatcher.hpp"
#include "core/registry.hpp"

#include <cstring>
#include <new>

namespace mensurflow::detail {

namespace {

constexpr std::size_t kAlignment = 64;

class CpuBuffer final : public Buffer {
  public:
    explicit CpuBuffer(std::size_t bytes) : size_(bytes) {
        if (bytes > 0) {
            data_ = ::operator new(bytes, std::align_val_t{kAlignment});
        }
    }
    ~CpuBuffer() override {
        if (data_ != nullptr) {
            ::operator delete(data_, std::align_val_t{kAlignment});
        }
    }
    CpuBuffer(const CpuBuffer&) = delete;
    CpuBuffer& operator=(const CpuBuffer&) = delete;
    std::size_t size() const override { return size_; }
    void* native() const override { return data_; }
    void* host_ptr() const override { return data_; }

  private:
    std::size_t size_;
    void* data_ = nullptr;
};

class CpuStream final : public Stream {
  public:
    void copy_h2d(Buffer& dst, std::size_t offset, const void* src, std::size_t bytes) override {
        std::memcpy(static_cast<std::byte*>(dst.native()) + offset, src, bytes);
    }
    void copy_d2h(void* dst, const Buffer& src, std::size_t offset, std::size_t bytes) override {
        std::memcpy(dst, static_cast<const std::byte*>(src.native()) + offset, bytes);
    }
    void copy_d2d(Buffer& dst, std::size_t dst_offset, const Buffer& src, std::size_t src_offset,
                  std::size_t bytes) override {
        std::memmove(static_cast<std::byte*>(dst.native()) + dst_offset,
                     static_cast<const std::byte*>(src.native()) + src_offset, bytes);
    }
    void synchronize() override {}
};

class CpuBackend final : public Backend {
  public:
    DeviceType type() const override { return DeviceType::CPU; }
    int device_count() const override { return 1; }
    DeviceInfo info(int) const override { return {"cpu", 0}; }
    std::shared_ptr<Buffer> allocate(int, std::size_t bytes) override {
        return std::make_shared<CpuBuffer>(bytes);
    }
    Stream& stream(int) override { return stream_; }
    void register_kernels(Dispatcher&) override {}

  private:
    CpuStream stream_;
};

} // namespace

void register_cpu_backend(Registry& registry) { registry.add(std::make_unique<CpuBackend>()); }

} // namespace mensurflow::detail
