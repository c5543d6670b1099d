// Shared pieces of libmfr_rocm.so: error reporting across the C ABI, the stream object and its
// workspace, and small device helpers. Only .hip files of this library include it.
#pragma once

#include "mfr_rocm.h"

#include <hip/hip_runtime.h>

#include "gelu_tanh.hpp"

#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>

namespace mfr {

// An error that becomes a status code at the C boundary (no exception leaves an extern "C"
// function). `code` is one of MFR_E_*.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& what) : std::runtime_error(what), code(c) {}
};

void set_last_error(const std::string& message);

// Throws Error(MFR_E_RUNTIME, "ROCm <what> failed: <hip message>") on failure, the message shape
// of the reference's CUDA backend (src/backends/cuda/backend.cpp:22-34).
inline void check(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        throw Error(MFR_E_RUNTIME, std::string("ROCm ") + what + " failed: " +
                                       hipGetErrorString(status));
    }
}

inline void require(bool condition, const std::string& message) {
    if (!condition) {
        throw Error(MFR_E_INVALID, message);
    }
}

// Runs `body` and turns any exception into a status code plus mfr_last_error().
template <typename Body> int guarded(Body&& body) {
    try {
        body();
        return MFR_OK;
    } catch (const Error& e) {
        set_last_error(e.what());
        return e.code;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return MFR_E_RUNTIME;
    } catch (...) {
        set_last_error("unknown error");
        return MFR_E_RUNTIME;
    }
}

} // namespace mfr

// One HIP stream on one device, plus the device workspace its kernels use for partial results
// (gemv-T partial sums, GEMM split-K sums and staged operands). The workspace belongs to the
// stream: kernels queued on one stream run in order, so they can share it; two streams never
// share one.
//
// Several host threads may call into one stream (a backend hands every thread the same stream
// of a device). A call that uses the workspace holds `workspace_mutex` from reserve() until its
// last launch is queued: another thread's reserve() could otherwise free the buffer between this
// thread's reserve() and its launches. Once the launches are queued, stream order protects them
// (reserve() waits for the stream before it frees).
struct mfr_stream {
    int device = 0;
    hipStream_t stream = nullptr;
    bool owned = true;
    void* workspace = nullptr;
    size_t workspace_bytes = 0;
    int compute_units = 256; // of the stream's device, read at creation
    std::mutex workspace_mutex;

    // Pinned host staging for copies from and to pageable host memory (allocated on first use,
    // freed with the stream): two slots, each with an event recorded after the DMA that last
    // read or filled it, so the CPU's copy into (or out of) one slot overlaps the DMA of the
    // other. `staging_mutex` is held for a whole copy.
    static constexpr size_t kStagingBytes = size_t{16} << 20;
    void* staging[2] = {nullptr, nullptr};
    hipEvent_t staging_done[2] = {nullptr, nullptr};
    std::mutex staging_mutex;

    // Makes this stream's device current on the calling thread (each ABI call does, as the
    // reference's CudaStream::activate does per call).
    void activate() const { mfr::check(hipSetDevice(device), "hipSetDevice"); }

    // At least `bytes` of workspace. Growing it waits for the stream (the old buffer may still be
    // in use by queued kernels) and is rare: the size only ever grows. The caller holds
    // workspace_mutex.
    void* reserve(size_t bytes) {
        if (bytes <= workspace_bytes) {
            return workspace;
        }
        if (workspace != nullptr) {
            mfr::check(hipStreamSynchronize(stream), "hipStreamSynchronize");
            mfr::check(hipFree(workspace), "hipFree");
            workspace = nullptr;
            workspace_bytes = 0;
        }
        const size_t rounded = (bytes + (size_t{1} << 20) - 1) & ~((size_t{1} << 20) - 1);
        mfr::check(hipMalloc(&workspace, rounded), "hipMalloc(workspace)");
        workspace_bytes = rounded;
        return workspace;
    }
};

struct mfr_event {
    hipEvent_t event = nullptr;
};

namespace mfr {

inline mfr_stream& stream_of(mfr_stream_t s) {
    require(s != nullptr, "null stream");
    s->activate();
    return *s;
}

inline unsigned grid_blocks(int64_t work, int64_t per_block, int64_t cap = int64_t{1} << 30) {
    int64_t blocks = (work + per_block - 1) / per_block;
    if (blocks < 1) {
        blocks = 1;
    }
    return static_cast<unsigned>(blocks < cap ? blocks : cap);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Launch-time check: a kernel launch error is reported by the next HIP call otherwise.
inline void check_launch(const char* what) { check(hipGetLastError(), what); }

} // namespace mfr

// ---- device helpers --------------------------------------------------------------------------

namespace mfr {

// MI355X's last-level cache (Infinity Cache). An output larger than this is written with
// non-temporal stores: no later kernel would find it cached anyway.
constexpr double kLastLevelCacheBytes = 256.0 * 1024 * 1024;

} // namespace mfr

namespace mfr::dev {

constexpr int kWave = 64;

typedef float native_float4 __attribute__((ext_vector_type(4)));

// 16-byte load marked non-temporal: streamed data that is read once should not displace
// reused data (x, C0) from the caches. p must be 16-byte aligned.
// A 16-byte non-temporal store (not kept in the caches), for outputs written once and too large
// for the last-level cache.
__device__ inline void store_streaming(float* p, float4 v) {
    const native_float4 n = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(n, reinterpret_cast<native_float4*>(p));
}

__device__ inline float4 load_streaming(const float* p) {
    const native_float4 v = __builtin_nontemporal_load(reinterpret_cast<const native_float4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ inline double wave_sum(double v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        v += __shfl_xor(v, offset, kWave);
    }
    return v;
}

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        v = fmaxf(v, __shfl_xor(v, offset, kWave));
    }
    return v;
}

// Lane exchanges in the vector ALU (no LDS-crossbar permute and no wait on the LDS counter).
// swap_pair<true>(x, a, b): gfx950's v_permlane32_swap given x twice, so a holds lanes 0-31's
// values and b lanes 32-63's, each in both halves: lane l finds its own value and lane l ^ 32's
// in (a, b), in that order for l < 32 and swapped for l >= 32. swap_pair<false> does the same
// for 16-lane rows (v_permlane16_swap: a the even rows', b the odd rows'), partners l and l ^ 16.
// A max or a sum of a and b therefore gives every lane of a pair the same bits.
template <bool HALVES>
__device__ inline void swap_pair(float x, float& a, float& b) {
    const unsigned u = __float_as_uint(x);
    const auto r = HALVES ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                          : __builtin_amdgcn_permlane16_swap(u, u, false, false);
    // The elements are read into scalars first: a bit cast of an element of the returned vector
    // reads element 0 whatever index it names.
    const unsigned lo = r[0], hi = r[1];
    a = __uint_as_float(lo);
    b = __uint_as_float(hi);
}

// Lane l ^ m's value for m = 1, 2, 4, 8, through DPP: quad permutations for 1 and 2, a row
// rotation by 8 for 8, and for 4 a row shift left by 4 in the lanes with bit 2 clear (DPP banks
// 0 and 2) merged with a shift right by 4 in the others (banks 1 and 3).
template <int M>
__device__ inline float xor_lane(float x) {
    const int u = __float_as_int(x);
    int r;
    if constexpr (M == 1) {
        r = __builtin_amdgcn_update_dpp(u, u, 0xB1, 0xF, 0xF, false); // quad_perm [1,0,3,2]
    } else if constexpr (M == 2) {
        r = __builtin_amdgcn_update_dpp(u, u, 0x4E, 0xF, 0xF, false); // quad_perm [2,3,0,1]
    } else if constexpr (M == 4) {
        const int up = __builtin_amdgcn_update_dpp(u, u, 0x104, 0xF, 0x5, false); // row_shl:4
        r = __builtin_amdgcn_update_dpp(up, u, 0x114, 0xF, 0xA, false);          // row_shr:4
    } else {
        static_assert(M == 8, "xor_lane takes 1, 2, 4 or 8");
        r = __builtin_amdgcn_update_dpp(u, u, 0x128, 0xF, 0xF, false); // row_ror:8
    }
    return __int_as_float(r);
}

// The sum over the 64 lanes by the xor butterfly (partners l ^ 32, 16, 8, 4, 2, 1 in turn), the
// total in every lane; each step adds a lane's value and its partner's, so the bits are those
// of v += __shfl_xor(v, m) over the same steps.
__device__ inline float butterfly_sum(float v) {
    float a, b;
    swap_pair<true>(v, a, b);
    v = a + b;
    swap_pair<false>(v, a, b);
    v = a + b;
    v += xor_lane<8>(v);
    v += xor_lane<4>(v);
    v += xor_lane<2>(v);
    v += xor_lane<1>(v);
    return v;
}

__device__ inline int wave_or(int v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        v |= __shfl_xor(v, offset, kWave);
    }
    return v;
}

// mensurflow::gelu in double, rounded once to float (elementwise.cpp:173-194): the tanh form in
// gelu_tanh.hpp; the erf form 0.5 v erfc(-v / sqrt(2)) with the device library's erfc. The
// library is compiled with -ffp-contract=off, so the products and sums round as in the reference.
__device__ inline float gelu(float value, int act) {
    if (act == MFR_ACT_GELU_TANH) {
        return gelu_math::gelu_tanh(value);
    }
    if (__builtin_isinf(value)) {
        return value < 0.0f ? -0.0f : value;
    }
    const double v = static_cast<double>(value);
    return static_cast<float>(0.5 * v * erfc(-v * 0.70710678118654752440));
}

__device__ inline float activate(float value, int act) {
    return act == MFR_ACT_NONE ? value : gelu(value, act);
}

} // namespace mfr::dev
