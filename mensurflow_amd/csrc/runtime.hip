// Devices, memory, streams, events and copies of the C ABI (include/mfr_rocm.h). These are the
// runtime half of the reference's Backend/Buffer/Stream interface (src/backends/backend.hpp).
#include "common.hpp"

#include <unistd.h>

#include <algorithm>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

namespace mfr {

namespace {
thread_local std::string g_last_error;

// HIP device ids of the usable devices, in order: mensurflow device index i is hip id ids[i].
// Only gfx950 (MI355X/MI350X) devices are usable: the kernels are compiled for it alone.
const std::vector<int>& usable_devices() {
    static std::vector<int> ids;
    static std::once_flag once;
    std::call_once(once, [] {
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess) {
            (void)hipGetLastError(); // no driver: no devices, not an error
            return;
        }
        for (int id = 0; id < count; ++id) {
            hipDeviceProp_t prop;
            if (hipGetDeviceProperties(&prop, id) != hipSuccess) {
                (void)hipGetLastError();
                continue;
            }
            if (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) {
                ids.push_back(id);
            }
        }
    });
    return ids;
}

int hip_id(int device) {
    const auto& ids = usable_devices();
    if (device < 0 || device >= static_cast<int>(ids.size())) {
        throw Error(MFR_E_NO_DEVICE, "device rocm:" + std::to_string(device) + " is not available");
    }
    return ids[static_cast<size_t>(device)];
}
} // namespace

void set_last_error(const std::string& message) { g_last_error = message; }

} // namespace mfr

using mfr::check;
using mfr::guarded;
using mfr::require;

namespace {

__global__ void fill_kernel(unsigned char* dst, int elem_size, int64_t n, uint64_t value) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        switch (elem_size) {
        case 1:
            dst[i] = static_cast<unsigned char>(value);
            break;
        case 2:
            reinterpret_cast<uint16_t*>(dst)[i] = static_cast<uint16_t>(value);
            break;
        case 4:
            reinterpret_cast<uint32_t*>(dst)[i] = static_cast<uint32_t>(value);
            break;
        default:
            reinterpret_cast<uint64_t*>(dst)[i] = value;
            break;
        }
    }
}

struct CopyShape {
    int ndim;
    int64_t shape[MFR_MAX_COPY_DIMS];
    int64_t strides[MFR_MAX_COPY_DIMS];
};

// dst[i] = src[offset(i)] where offset walks the strided view in row-major order. One thread
// per element; the index is decomposed from the last (fastest) dimension.
template <typename T>
__global__ void strided_copy_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t n,
                                    CopyShape s) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        int64_t rest = i;
        int64_t offset = 0;
        for (int d = s.ndim - 1; d >= 0; --d) {
            const int64_t size = s.shape[d];
            const int64_t index = rest % size;
            rest /= size;
            offset += index * s.strides[d];
        }
        dst[i] = src[offset];
    }
}

// dst[i] = src[i] in 16-byte units (both pointers 16-byte aligned): each workgroup copies one
// contiguous chunk, 8 non-temporal loads in flight per thread before the stores. Measured on a
// 1 GiB copy: 5.66 TB/s (read + write) with 4096 workgroups, against 5.0 TB/s for a
// grid-stride loop and 5.1 TB/s for hipMemcpyAsync.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 8;

__global__ __launch_bounds__(kCopyThreads) void copy16_kernel(const u32x4* __restrict__ src,
                                                              u32x4* __restrict__ dst, int64_t n,
                                                              int64_t chunk) {
    const int64_t begin = static_cast<int64_t>(blockIdx.x) * chunk;
    const int64_t end = begin + chunk < n ? begin + chunk : n;
    int64_t i = begin + threadIdx.x;
    for (; i + (kCopyUnroll - 1) * kCopyThreads < end; i += kCopyUnroll * kCopyThreads) {
        u32x4 v[kCopyUnroll];
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u) {
            v[u] = __builtin_nontemporal_load(src + i + u * kCopyThreads);
        }
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u) {
            __builtin_nontemporal_store(v[u], dst + i + u * kCopyThreads);
        }
    }
    for (; i < end; i += kCopyThreads) {
        dst[i] = src[i];
    }
}

// dst[i] = src[0] for i < n (a source whose strides are all 0): one load per thread, then
// stores only.
template <typename T>
__global__ __launch_bounds__(256) void broadcast_kernel(const T* __restrict__ src,
                                                        T* __restrict__ dst, int64_t n) {
    const T value = src[0];
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        dst[i] = value;
    }
}

// A view whose last dimension has unit stride: `rows` rows of `row_units` units (elements, or
// 16-byte groups of them when every row start and length allow it), row r of dst at
// r * row_units, row r of src at the offset of index r in `outer` (the other dimensions, strides
// in units). Each work item copies `chunk` units of one row, so the index is decomposed once per
// item rather than per element.
template <typename U>
__global__ __launch_bounds__(256) void copy_rows_kernel(const U* __restrict__ src,
                                                        U* __restrict__ dst, int64_t rows,
                                                        int64_t row_units, int64_t chunks_per_row,
                                                        int64_t chunk, CopyShape outer) {
    const int64_t items = rows * chunks_per_row;
    for (int64_t w = blockIdx.x; w < items; w += gridDim.x) {
        const int64_t row = w / chunks_per_row;
        const int64_t begin = (w - row * chunks_per_row) * chunk;
        const int64_t end = begin + chunk < row_units ? begin + chunk : row_units;
        int64_t rest = row;
        int64_t offset = 0;
        for (int d = outer.ndim - 1; d >= 0; --d) {
            const int64_t index = rest % outer.shape[d];
            rest /= outer.shape[d];
            offset += index * outer.strides[d];
        }
        const U* in = src + offset;
        U* out = dst + row * row_units;
        for (int64_t j = begin + threadIdx.x; j < end; j += blockDim.x) {
            out[j] = in[j];
        }
    }
}

template <typename T>
void launch_copy_rows(const void* src, void* dst, const CopyShape& cs, int elem_size,
                      hipStream_t stream) {
    const int last = cs.ndim - 1;
    const int64_t row_len = cs.shape[last];
    CopyShape outer{};
    outer.ndim = last;
    int64_t rows = 1;
    bool wide = mfr::aligned16(src) && mfr::aligned16(dst) && (row_len * elem_size) % 16 == 0;
    for (int d = 0; d < last; ++d) {
        outer.shape[d] = cs.shape[d];
        outer.strides[d] = cs.strides[d];
        rows *= cs.shape[d];
        wide = wide && (cs.strides[d] * elem_size) % 16 == 0;
    }
    const int per = wide ? 16 / elem_size : 1; // elements per unit
    for (int d = 0; d < last; ++d) {
        outer.strides[d] /= per;
    }
    const int64_t row_units = row_len / per;
    const int64_t chunk = 2048;
    const int64_t chunks_per_row = (row_units + chunk - 1) / chunk;
    const unsigned blocks = mfr::grid_blocks(rows * chunks_per_row, 1, 65536);
    if (wide) {
        copy_rows_kernel<<<blocks, 256, 0, stream>>>(static_cast<const u32x4*>(src),
                                                     static_cast<u32x4*>(dst), rows, row_units,
                                                     chunks_per_row, chunk, outer);
    } else {
        copy_rows_kernel<<<blocks, 256, 0, stream>>>(static_cast<const T*>(src),
                                                     static_cast<T*>(dst), rows, row_units,
                                                     chunks_per_row, chunk, outer);
    }
    mfr::check_launch("copy_rows_kernel");
}

template <typename T>
void launch_broadcast(const void* src, void* dst, int64_t n, hipStream_t stream) {
    broadcast_kernel<<<mfr::grid_blocks(n, 256 * 4, 8192), 256, 0, stream>>>(
        static_cast<const T*>(src), static_cast<T*>(dst), n);
    mfr::check_launch("broadcast_kernel");
}

// Drops size-1 dimensions and merges neighbours that are contiguous with each other
// (stride[d] == shape[d+1] * stride[d+1]), so a packed view becomes one dimension of stride 1.
// ---- transposed views ---------------------------------------------------------------------
//
// dst (packed row-major over cs.shape) from a source whose last dimension is strided but whose
// dimension `da` is contiguous (a transposed matrix, or a batch of them): 64 x 64 tiles through
// LDS, read along da (coalesced in the source) and written along the last dimension (coalesced
// in dst). The padded row keeps the column reads free of bank conflicts.
constexpr int kTransposeTile = 64;
constexpr int kTransposeThreads = 256; // 64 x 4

struct TransposeShape {
    CopyShape cs;
    int da;                // the dimension with unit source stride
    int64_t tiles_a;       // tiles along da
    int64_t tiles_b;       // tiles along the last dimension
    int64_t jobs;          // tiles_a * tiles_b * (product of the other dimensions)
    int64_t dst_stride_a;  // dst elements between consecutive indices of da
};

template <typename T>
__global__ __launch_bounds__(kTransposeThreads) void transpose_kernel(const T* __restrict__ src,
                                                                      T* __restrict__ dst,
                                                                      TransposeShape t) {
    __shared__ T tile[kTransposeTile][kTransposeTile + 1];
    const int last = t.cs.ndim - 1;
    const int64_t size_a = t.cs.shape[t.da];
    const int64_t size_b = t.cs.shape[last];
    const int64_t stride_b = t.cs.strides[last];
    const int tx = threadIdx.x % kTransposeTile;
    const int ty = threadIdx.x / kTransposeTile;
    const int64_t per_rest = t.tiles_a * t.tiles_b;
    for (int64_t job = blockIdx.x; job < t.jobs; job += gridDim.x) {
        int64_t rest = job / per_rest;
        const int64_t within = job - rest * per_rest;
        const int64_t a0 = (within / t.tiles_b) * kTransposeTile;
        const int64_t b0 = (within % t.tiles_b) * kTransposeTile;
        // Offsets of the other dimensions, in the source and in dst.
        int64_t src_off = 0, dst_off = 0, dst_stride = 1;
        for (int d = last; d >= 0; --d) {
            if (d != t.da && d != last) {
                const int64_t index = rest % t.cs.shape[d];
                rest /= t.cs.shape[d];
                src_off += index * t.cs.strides[d];
                dst_off += index * dst_stride;
            }
            dst_stride *= t.cs.shape[d];
        }
        for (int i = ty; i < kTransposeTile; i += kTransposeThreads / kTransposeTile) {
            const int64_t a = a0 + tx, b = b0 + i;
            if (a < size_a && b < size_b) {
                tile[i][tx] = src[src_off + a + b * stride_b];
            }
        }
        __syncthreads();
        for (int i = ty; i < kTransposeTile; i += kTransposeThreads / kTransposeTile) {
            const int64_t a = a0 + i, b = b0 + tx;
            if (a < size_a && b < size_b) {
                dst[dst_off + a * t.dst_stride_a + b] = tile[tx][i];
            }
        }
        __syncthreads();
    }
}

// The transposed form of cs, if it has one: a strided last dimension and an earlier dimension
// with unit stride, both at least 16 long.
bool transpose_shape(const CopyShape& cs, TransposeShape* t) {
    const int last = cs.ndim - 1;
    if (cs.ndim < 2 || cs.strides[last] == 1 || cs.shape[last] < 16) {
        return false;
    }
    int da = -1;
    for (int d = last - 1; d >= 0; --d) {
        if (cs.strides[d] == 1) {
            da = d;
            break;
        }
    }
    if (da < 0 || cs.shape[da] < 16) {
        return false;
    }
    t->cs = cs;
    t->da = da;
    t->tiles_a = (cs.shape[da] + kTransposeTile - 1) / kTransposeTile;
    t->tiles_b = (cs.shape[last] + kTransposeTile - 1) / kTransposeTile;
    int64_t rest = 1, stride_a = 1;
    for (int d = 0; d < cs.ndim; ++d) {
        if (d != da && d != last) {
            rest *= cs.shape[d];
        }
        if (d > da) {
            stride_a *= cs.shape[d];
        }
    }
    t->jobs = t->tiles_a * t->tiles_b * rest;
    t->dst_stride_a = stride_a;
    return true;
}

template <typename T>
void launch_transpose(const void* src, void* dst, const TransposeShape& t, hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>(t.jobs < 65536 ? t.jobs : 65536);
    transpose_kernel<T><<<blocks, kTransposeThreads, 0, stream>>>(static_cast<const T*>(src),
                                                                  static_cast<T*>(dst), t);
    mfr::check_launch("transpose_kernel");
}

void collapse(CopyShape& s) {
    CopyShape out{};
    out.ndim = 0;
    for (int d = 0; d < s.ndim; ++d) {
        if (s.shape[d] == 1) {
            continue;
        }
        if (out.ndim > 0 && out.strides[out.ndim - 1] == s.shape[d] * s.strides[d]) {
            out.shape[out.ndim - 1] *= s.shape[d];
            out.strides[out.ndim - 1] = s.strides[d];
        } else {
            out.shape[out.ndim] = s.shape[d];
            out.strides[out.ndim] = s.strides[d];
            ++out.ndim;
        }
    }
    if (out.ndim == 0) { // a single element
        out.ndim = 1;
        out.shape[0] = 1;
        out.strides[0] = 1;
    }
    s = out;
}

// Copies between pageable host memory and the device of at least this many bytes go through
// the stream's pinned staging slots. From pageable memory directly, the runtime's own path
// measured about 4 GB/s for 1 GiB on an MI355X box; small copies keep it (one call, no staging).
constexpr size_t kStagedCopyBytes = size_t{1} << 20;

// The stream's two pinned staging slots and their events, allocated once. The caller holds
// s.staging_mutex.
void ensure_staging(mfr_stream& s) {
    for (int slot = 0; slot < 2; ++slot) {
        if (s.staging[slot] == nullptr) {
            check(hipHostMalloc(&s.staging[slot], mfr_stream::kStagingBytes, hipHostMallocDefault),
                  "hipHostMalloc(staging)");
        }
        if (s.staging_done[slot] == nullptr) {
            check(hipEventCreateWithFlags(&s.staging_done[slot], hipEventDisableTiming),
                  "hipEventCreateWithFlags(staging)");
        }
    }
}

// The CPU's part of a staged copy (pageable memory to or from a pinned slot), split over the
// calling thread and kHelpers helper threads. One thread copies about 28 GB/s on an MI355X box's
// host, below the 57 GB/s of the slot's DMA, and a first write into fresh pageable memory is
// slower still (its page faults); two threads reach the DMA's rate and four pass it. The helpers
// start at the first large copy and then wait for work. One copy uses them at a time: a copy
// that finds them busy (another thread's copy on another stream) runs alone, as does a copy in
// a process forked after they started (a child has no helper threads). The object is never
// destroyed, so a helper still waiting at exit waits on live memory.
class CopyHelpers {
  public:
    static constexpr int kHelpers = 3;
    static constexpr size_t kMinBytes = size_t{1} << 20; // below this one thread copies

    static void copy(void* dst, const void* src, size_t bytes) {
        CopyHelpers* helpers = bytes >= kMinBytes ? instance() : nullptr;
        if (helpers == nullptr || helpers->pid_ != getpid() || !helpers->busy_.try_lock()) {
            std::memcpy(dst, src, bytes);
            return;
        }
        std::lock_guard<std::mutex> own(helpers->busy_, std::adopt_lock);
        helpers->run(static_cast<unsigned char*>(dst), static_cast<const unsigned char*>(src),
                     bytes);
    }

  private:
    static CopyHelpers* instance() {
        static CopyHelpers* const helpers = start();
        return helpers;
    }

    // All helpers or none: a copy waits for exactly kHelpers parts.
    static CopyHelpers* start() {
        auto* helpers = new CopyHelpers();
        std::vector<std::thread> threads;
        try {
            for (int i = 0; i < kHelpers; ++i) {
                threads.emplace_back(&CopyHelpers::serve, helpers, i);
            }
        } catch (...) {
            // Fewer threads than asked for: stop those started (they exit at the next wake-up)
            // and copy alone from then on.
            {
                std::lock_guard<std::mutex> lock(helpers->mutex_);
                helpers->stop_ = true;
                ++helpers->generation_;
            }
            helpers->work_.notify_all();
            for (auto& t : threads) {
                t.join();
            }
            return nullptr;
        }
        for (auto& t : threads) {
            t.detach();
        }
        return helpers;
    }

    // Part i of a copy split in kHelpers + 1 parts of whole 64-byte lines; the last takes the rest.
    static void part(int i, unsigned char* dst, const unsigned char* src, size_t bytes) {
        const size_t share = (bytes / (kHelpers + 1)) & ~size_t{63};
        const size_t begin = static_cast<size_t>(i) * share;
        const size_t end = i == kHelpers ? bytes : begin + share;
        std::memcpy(dst + begin, src + begin, end - begin);
    }

    void run(unsigned char* dst, const unsigned char* src, size_t bytes) {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            dst_ = dst;
            src_ = src;
            bytes_ = bytes;
            pending_ = kHelpers;
            ++generation_;
        }
        work_.notify_all();
        part(kHelpers, dst, src, bytes);
        std::unique_lock<std::mutex> lock(mutex_);
        done_.wait(lock, [&] { return pending_ == 0; });
    }

    void serve(int index) {
        std::uint64_t seen = 0;
        std::unique_lock<std::mutex> lock(mutex_);
        for (;;) {
            work_.wait(lock, [&] { return generation_ != seen; });
            if (stop_) {
                return;
            }
            seen = generation_;
            unsigned char* const dst = dst_;
            const unsigned char* const src = src_;
            const size_t bytes = bytes_;
            lock.unlock();
            part(index, dst, src, bytes);
            lock.lock();
            if (--pending_ == 0) {
                done_.notify_one();
            }
        }
    }

    const pid_t pid_ = getpid();
    std::mutex busy_; // held by the copy that uses the helpers
    std::mutex mutex_;
    std::condition_variable work_, done_;
    std::uint64_t generation_ = 0;
    bool stop_ = false;
    int pending_ = 0;
    unsigned char* dst_ = nullptr;
    const unsigned char* src_ = nullptr;
    size_t bytes_ = 0;
};

} // namespace

extern "C" {

const char* mfr_last_error(void) { return mfr::g_last_error.c_str(); }

int mfr_get_device_count(int* count) {
    return guarded([&] {
        require(count != nullptr, "mfr_get_device_count: null output");
        *count = static_cast<int>(mfr::usable_devices().size());
    });
}

int mfr_get_device_info(int device, char* name, size_t cap, size_t* memory_bytes,
                        int* compute_units, int* clock_khz) {
    return guarded([&] {
        hipDeviceProp_t prop;
        check(hipGetDeviceProperties(&prop, mfr::hip_id(device)), "hipGetDeviceProperties");
        if (name != nullptr && cap > 0) {
            // Some drivers leave the marketing name empty; the architecture name is always set.
            const char* source = prop.name[0] != '\0' ? prop.name : prop.gcnArchName;
            std::strncpy(name, source, cap - 1);
            name[cap - 1] = '\0';
        }
        if (memory_bytes != nullptr) {
            *memory_bytes = prop.totalGlobalMem;
        }
        if (compute_units != nullptr) {
            *compute_units = prop.multiProcessorCount;
        }
        if (clock_khz != nullptr) {
            *clock_khz = prop.clockRate;
        }
    });
}

int mfr_malloc(int device, size_t bytes, void** ptr) {
    return guarded([&] {
        require(ptr != nullptr, "mfr_malloc: null output");
        *ptr = nullptr;
        if (bytes == 0) {
            return;
        }
        check(hipSetDevice(mfr::hip_id(device)), "hipSetDevice");
        check(hipMalloc(ptr, bytes), "hipMalloc");
    });
}

int mfr_free(int device, void* ptr) {
    return guarded([&] {
        if (ptr == nullptr) {
            return;
        }
        check(hipSetDevice(mfr::hip_id(device)), "hipSetDevice");
        check(hipFree(ptr), "hipFree");
    });
}

int mfr_stream_create(int device, mfr_stream_t* stream) {
    return guarded([&] {
        require(stream != nullptr, "mfr_stream_create: null output");
        auto s = new mfr_stream;
        s->device = mfr::hip_id(device);
        try {
            s->activate();
            // Default priority on purpose: streams of different priorities are not mixed.
            check(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking),
                  "hipStreamCreateWithFlags");
            check(hipDeviceGetAttribute(&s->compute_units, hipDeviceAttributeMultiprocessorCount,
                                        s->device),
                  "hipDeviceGetAttribute");
        } catch (...) {
            delete s;
            throw;
        }
        *stream = s;
    });
}

int mfr_stream_wrap(int device, void* hip_stream, mfr_stream_t* stream) {
    return guarded([&] {
        require(stream != nullptr, "mfr_stream_wrap: null output");
        auto s = new mfr_stream;
        s->device = mfr::hip_id(device);
        s->stream = static_cast<hipStream_t>(hip_stream);
        s->owned = false;
        check(hipDeviceGetAttribute(&s->compute_units, hipDeviceAttributeMultiprocessorCount,
                                    s->device),
              "hipDeviceGetAttribute");
        *stream = s;
    });
}

int mfr_stream_destroy(mfr_stream_t stream) {
    return guarded([&] {
        if (stream == nullptr) {
            return;
        }
        stream->activate();
        check(hipStreamSynchronize(stream->stream), "hipStreamSynchronize");
        if (stream->workspace != nullptr) {
            check(hipFree(stream->workspace), "hipFree(workspace)");
        }
        for (int slot = 0; slot < 2; ++slot) {
            if (stream->staging[slot] != nullptr) {
                check(hipHostFree(stream->staging[slot]), "hipHostFree(staging)");
            }
            if (stream->staging_done[slot] != nullptr) {
                check(hipEventDestroy(stream->staging_done[slot]), "hipEventDestroy(staging)");
            }
        }
        if (stream->owned && stream->stream != nullptr) {
            check(hipStreamDestroy(stream->stream), "hipStreamDestroy");
        }
        delete stream;
    });
}

int mfr_stream_sync(mfr_stream_t stream) {
    return guarded([&] {
        auto& s = mfr::stream_of(stream);
        check(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
    });
}

void* mfr_stream_handle(mfr_stream_t stream) {
    return stream == nullptr ? nullptr : static_cast<void*>(stream->stream);
}

int mfr_stream_device(mfr_stream_t stream) {
    if (stream == nullptr) {
        return -1;
    }
    const auto& ids = mfr::usable_devices();
    for (size_t i = 0; i < ids.size(); ++i) {
        if (ids[i] == stream->device) {
            return static_cast<int>(i);
        }
    }
    return -1;
}

int mfr_memcpy_h2d(mfr_stream_t stream, void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        auto& s = mfr::stream_of(stream);
        if (bytes == 0) {
            return;
        }
        require(dst != nullptr && src != nullptr, "mfr_memcpy_h2d: null pointer");
        if (bytes < kStagedCopyBytes) {
            check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s.stream),
                  "hipMemcpyAsync");
        } else {
            std::lock_guard<std::mutex> hold(s.staging_mutex);
            ensure_staging(s);
            const auto* from = static_cast<const unsigned char*>(src);
            auto* to = static_cast<unsigned char*>(dst);
            for (size_t off = 0, i = 0; off < bytes; off += mfr_stream::kStagingBytes, ++i) {
                const size_t n = std::min(mfr_stream::kStagingBytes, bytes - off);
                const int slot = static_cast<int>(i & 1);
                // The DMA that last read this slot (two chunks back) has finished.
                check(hipEventSynchronize(s.staging_done[slot]), "hipEventSynchronize");
                CopyHelpers::copy(s.staging[slot], from + off, n);
                check(hipMemcpyAsync(to + off, s.staging[slot], n, hipMemcpyHostToDevice,
                                     s.stream),
                      "hipMemcpyAsync");
                check(hipEventRecord(s.staging_done[slot], s.stream), "hipEventRecord");
            }
        }
        // Complete before returning, so the caller may reuse or free the source.
        check(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
    });
}

int mfr_memcpy_d2h(mfr_stream_t stream, void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        auto& s = mfr::stream_of(stream);
        if (bytes == 0) {
            check(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
            return;
        }
        require(dst != nullptr && src != nullptr, "mfr_memcpy_d2h: null pointer");
        if (bytes < kStagedCopyBytes) {
            check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s.stream),
                  "hipMemcpyAsync");
            check(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
            return;
        }
        std::lock_guard<std::mutex> hold(s.staging_mutex);
        ensure_staging(s);
        const auto* from = static_cast<const unsigned char*>(src);
        auto* to = static_cast<unsigned char*>(dst);
        const size_t chunk = mfr_stream::kStagingBytes;
        const size_t chunks = (bytes + chunk - 1) / chunk;
        // Chunk i goes device -> slot i % 2 -> dst. Chunk i + 1's DMA is queued before chunk i is
        // copied out; its slot held chunk i - 1, which the previous step finished copying out.
        const auto queue = [&](size_t i) {
            const size_t n = std::min(chunk, bytes - i * chunk);
            const int slot = static_cast<int>(i & 1);
            check(hipMemcpyAsync(s.staging[slot], from + i * chunk, n, hipMemcpyDeviceToHost,
                                 s.stream),
                  "hipMemcpyAsync");
            check(hipEventRecord(s.staging_done[slot], s.stream), "hipEventRecord");
        };
        queue(0);
        for (size_t i = 0; i < chunks; ++i) {
            if (i + 1 < chunks) {
                queue(i + 1);
            }
            const int slot = static_cast<int>(i & 1);
            check(hipEventSynchronize(s.staging_done[slot]), "hipEventSynchronize");
            CopyHelpers::copy(to + i * chunk, s.staging[slot], std::min(chunk, bytes - i * chunk));
        }
        check(hipStreamSynchronize(s.stream), "hipStreamSynchronize");
    });
}

int mfr_memcpy_d2d(mfr_stream_t stream, void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        auto& s = mfr::stream_of(stream);
        if (bytes == 0) {
            return;
        }
        require(dst != nullptr && src != nullptr, "mfr_memcpy_d2d: null pointer");
        check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s.stream),
              "hipMemcpyAsync");
    });
}

int mfr_event_create(mfr_event_t* event) {
    return guarded([&] {
        require(event != nullptr, "mfr_event_create: null output");
        auto e = new mfr_event;
        const hipError_t status = hipEventCreate(&e->event);
        if (status != hipSuccess) {
            delete e;
            check(status, "hipEventCreate");
        }
        *event = e;
    });
}

int mfr_event_destroy(mfr_event_t event) {
    return guarded([&] {
        if (event == nullptr) {
            return;
        }
        check(hipEventDestroy(event->event), "hipEventDestroy");
        delete event;
    });
}

int mfr_event_record(mfr_event_t event, mfr_stream_t stream) {
    return guarded([&] {
        require(event != nullptr, "mfr_event_record: null event");
        auto& s = mfr::stream_of(stream);
        check(hipEventRecord(event->event, s.stream), "hipEventRecord");
    });
}

int mfr_event_elapsed_ms(mfr_event_t start, mfr_event_t end, float* ms) {
    return guarded([&] {
        require(start != nullptr && end != nullptr && ms != nullptr,
                "mfr_event_elapsed_ms: null argument");
        check(hipEventSynchronize(end->event), "hipEventSynchronize");
        check(hipEventElapsedTime(ms, start->event, end->event), "hipEventElapsedTime");
    });
}

int mfr_fill(mfr_stream_t stream, void* dst, int32_t elem_size, int64_t n, uint64_t value) {
    return guarded([&] {
        auto& s = mfr::stream_of(stream);
        require(elem_size == 1 || elem_size == 2 || elem_size == 4 || elem_size == 8,
                "mfr_fill: element size must be 1, 2, 4 or 8");
        require(n >= 0, "mfr_fill: negative count");
        if (n == 0) {
            return;
        }
        require(dst != nullptr, "mfr_fill: null destination");
        fill_kernel<<<mfr::grid_blocks(n, 256, 65536), 256, 0, s.stream>>>(
            static_cast<unsigned char*>(dst), elem_size, n, value);
        mfr::check_launch("fill_kernel");
    });
}

int mfr_strided_copy(mfr_stream_t stream, const void* src, void* dst, int32_t elem_size,
                     int32_t ndim, const int64_t* shape, const int64_t* strides) {
    return guarded([&] {
        auto& s = mfr::stream_of(stream);
        require(ndim >= 0 && ndim <= MFR_MAX_COPY_DIMS, "mfr_strided_copy: too many dimensions");
        require(elem_size == 1 || elem_size == 2 || elem_size == 4 || elem_size == 8,
                "mfr_strided_copy: element size must be 1, 2, 4 or 8");
        CopyShape cs{};
        cs.ndim = ndim;
        int64_t n = 1;
        for (int d = 0; d < ndim; ++d) {
            require(shape[d] >= 0, "mfr_strided_copy: negative dimension");
            cs.shape[d] = shape[d];
            cs.strides[d] = strides[d];
            n *= shape[d];
        }
        if (n == 0) {
            return;
        }
        require(src != nullptr && dst != nullptr, "mfr_strided_copy: null pointer");
        collapse(cs);
        if (cs.ndim == 1 && cs.strides[0] == 1) {
            // Packed source: a plain copy.
            const size_t bytes = static_cast<size_t>(n) * static_cast<size_t>(elem_size);
            if (bytes % 16 == 0 && mfr::aligned16(src) && mfr::aligned16(dst)) {
                const int64_t units = static_cast<int64_t>(bytes / 16);
                // Up to 4096 chunks, each at least one unrolled step of the workgroup.
                const int64_t step = static_cast<int64_t>(kCopyThreads) * kCopyUnroll;
                int64_t blocks = (units + step - 1) / step;
                blocks = blocks < 1 ? 1 : (blocks > 4096 ? 4096 : blocks);
                const int64_t chunk = (units + blocks - 1) / blocks;
                copy16_kernel<<<static_cast<unsigned>(blocks), kCopyThreads, 0, s.stream>>>(
                    static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), units, chunk);
                mfr::check_launch("copy16_kernel");
            } else {
                check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s.stream),
                      "hipMemcpyAsync");
            }
            return;
        }
        if (cs.ndim == 1 && cs.strides[0] == 0) {
            // One element repeated (a broadcast scalar, e.g. -inf expanded to a score tensor).
            switch (elem_size) {
            case 1:
                launch_broadcast<uint8_t>(src, dst, n, s.stream);
                break;
            case 2:
                launch_broadcast<uint16_t>(src, dst, n, s.stream);
                break;
            case 4:
                launch_broadcast<uint32_t>(src, dst, n, s.stream);
                break;
            default:
                launch_broadcast<uint64_t>(src, dst, n, s.stream);
                break;
            }
            return;
        }
        if (cs.strides[cs.ndim - 1] == 1 && cs.shape[cs.ndim - 1] >= 64) {
            // Rows with a unit stride (sliced, broadcast or strided outer dimensions).
            switch (elem_size) {
            case 1:
                launch_copy_rows<uint8_t>(src, dst, cs, elem_size, s.stream);
                break;
            case 2:
                launch_copy_rows<uint16_t>(src, dst, cs, elem_size, s.stream);
                break;
            case 4:
                launch_copy_rows<uint32_t>(src, dst, cs, elem_size, s.stream);
                break;
            default:
                launch_copy_rows<uint64_t>(src, dst, cs, elem_size, s.stream);
                break;
            }
            return;
        }
        TransposeShape ts;
        if (transpose_shape(cs, &ts)) {
            switch (elem_size) {
            case 1:
                launch_transpose<uint8_t>(src, dst, ts, s.stream);
                break;
            case 2:
                launch_transpose<uint16_t>(src, dst, ts, s.stream);
                break;
            case 4:
                launch_transpose<uint32_t>(src, dst, ts, s.stream);
                break;
            default:
                launch_transpose<uint64_t>(src, dst, ts, s.stream);
                break;
            }
            return;
        }
        const unsigned blocks = mfr::grid_blocks(n, 256, 65536);
        switch (elem_size) {
        case 1:
            strided_copy_kernel<<<blocks, 256, 0, s.stream>>>(
                static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), n, cs);
            break;
        case 2:
            strided_copy_kernel<<<blocks, 256, 0, s.stream>>>(
                static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), n, cs);
            break;
        case 4:
            strided_copy_kernel<<<blocks, 256, 0, s.stream>>>(
                static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), n, cs);
            break;
        default:
            strided_copy_kernel<<<blocks, 256, 0, s.stream>>>(
                static_cast<const uint64_t*>(src), static_cast<uint64_t*>(dst), n, cs);
            break;
        }
        mfr::check_launch("strided_copy_kernel");
    });
}

} // extern "C"
