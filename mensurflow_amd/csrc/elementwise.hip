// Elementwise, softmax and argmax kernels of the hot path on gfx950. All are one pass over HBM
// (or two for softmax rows that do not fit in registers); each follows the reference CPU
// kernel's arithmetic so results round the same way:
//   bias_add + gelu   src/backends/cpu/ops/elementwise/elementwise.cpp:128-137, 173-194
//   where             elementwise.cpp:64-70
//   softmax           src/backends/cpu/ops/softmax/softmax.cpp:13-49
//   argmax            src/backends/cpu/ops/reduction/reduction.cpp:284-296
#include "common.hpp"

#include <cmath>

namespace {

using mfr::dev::kWave;

// y[r, j] = act(x[r, j] + bias[j]); bias may be null (y = act(x)). One thread per 4 elements of
// a row when cols % 4 == 0 (16-byte accesses), else per element.
template <bool VEC4>
__global__ void bias_act_kernel(const float* __restrict__ x, const float* __restrict__ bias,
                                float* y, int64_t rows, int64_t cols, int act) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    if constexpr (VEC4) {
        const int64_t quads_per_row = cols / 4;
        const int64_t n = rows * quads_per_row;
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
             i += stride) {
            const int64_t col = (i % quads_per_row) * 4;
            float4 v = reinterpret_cast<const float4*>(x)[i];
            if (bias != nullptr) {
                const float4 b = *reinterpret_cast<const float4*>(bias + col);
                v.x = v.x + b.x;
                v.y = v.y + b.y;
                v.z = v.z + b.z;
                v.w = v.w + b.w;
            }
            if (act != MFR_ACT_NONE) {
                v.x = mfr::dev::gelu(v.x, act);
                v.y = mfr::dev::gelu(v.y, act);
                v.z = mfr::dev::gelu(v.z, act);
                v.w = mfr::dev::gelu(v.w, act);
            }
            reinterpret_cast<float4*>(y)[i] = v;
        }
    } else {
        const int64_t n = rows * cols;
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
             i += stride) {
            float v = x[i];
            if (bias != nullptr) {
                v = v + bias[i % cols];
            }
            y[i] = mfr::dev::activate(v, act);
        }
    }
}

__global__ void where_kernel(const uint8_t* __restrict__ cond, const float* __restrict__ x,
                             const float* __restrict__ y, float* __restrict__ out, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        out[i] = cond[i] != 0 ? x[i] : y[i];
    }
}

// The reference's line maximum: a NaN anywhere makes it NaN (the scan stops at the first NaN),
// otherwise the largest value (-inf for an empty or all -inf line).
__device__ inline float line_max(float m, int has_nan) { return has_nan ? NAN : m; }

// Softmax of contiguous lines (inner == 1), one wavefront per line, the line held in registers:
// each lane keeps kPer values at positions lane + 64*i.
template <int kPer>
__global__ __launch_bounds__(256) void softmax_rows_reg_kernel(const float* __restrict__ x,
                                                               float* __restrict__ y,
                                                               int64_t lines, int64_t length) {
    const int lane = threadIdx.x % kWave;
    const int64_t line = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) +
                         threadIdx.x / kWave;
    if (line >= lines) {
        return;
    }
    const float* in = x + line * length;
    float* out = y + line * length;
    float v[kPer];
    float m = -INFINITY;
    int has_nan = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int64_t j = lane + static_cast<int64_t>(kWave) * i;
        v[i] = j < length ? in[j] : -INFINITY;
        has_nan |= __builtin_isnan(v[i]) ? 1 : 0;
        m = fmaxf(m, v[i]);
    }
    m = line_max(mfr::dev::wave_max(m), mfr::dev::wave_or(has_nan));
    if (m == -INFINITY) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int64_t j = lane + static_cast<int64_t>(kWave) * i;
            if (j < length) {
                out[j] = 0.0f; // every element masked out
            }
        }
        return;
    }
    double sum = 0.0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int64_t j = lane + static_cast<int64_t>(kWave) * i;
        if (j < length) {
            v[i] = expf(v[i] - m);
            sum += static_cast<double>(v[i]);
        }
    }
    sum = mfr::dev::wave_sum(sum);
    const float scale = static_cast<float>(1.0 / sum);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int64_t j = lane + static_cast<int64_t>(kWave) * i;
        if (j < length) {
            out[j] = v[i] * scale;
        }
    }
}

// Any line shape: one wavefront per line, three passes over the line in memory.
__global__ __launch_bounds__(256) void softmax_lines_kernel(const float* __restrict__ x,
                                                            float* __restrict__ y, int64_t outer,
                                                            int64_t length, int64_t inner) {
    const int lane = threadIdx.x % kWave;
    const int64_t line = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) +
                         threadIdx.x / kWave;
    if (line >= outer * inner) {
        return;
    }
    const int64_t base = (line / inner) * length * inner + line % inner;
    const float* in = x + base;
    float* out = y + base;
    float m = -INFINITY;
    int has_nan = 0;
    for (int64_t j = lane; j < length; j += kWave) {
        const float v = in[j * inner];
        has_nan |= __builtin_isnan(v) ? 1 : 0;
        m = fmaxf(m, v);
    }
    m = line_max(mfr::dev::wave_max(m), mfr::dev::wave_or(has_nan));
    if (m == -INFINITY) {
        for (int64_t j = lane; j < length; j += kWave) {
            out[j * inner] = 0.0f;
        }
        return;
    }
    double sum = 0.0;
    for (int64_t j = lane; j < length; j += kWave) {
        const float e = expf(in[j * inner] - m);
        out[j * inner] = e;
        sum += static_cast<double>(e);
    }
    sum = mfr::dev::wave_sum(sum);
    const float scale = static_cast<float>(1.0 / sum);
    for (int64_t j = lane; j < length; j += kWave) {
        out[j * inner] = out[j * inner] * scale;
    }
}

// First index of the maximum of each row; the first NaN wins. One wavefront per row: each lane
// keeps the first NaN it saw and its best (value, first index), then lanes are combined.
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ x,
                                                     int64_t* __restrict__ out, int64_t rows,
                                                     int64_t width) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) +
                        threadIdx.x / kWave;
    if (row >= rows) {
        return;
    }
    const float* values = x + row * width;
    const int64_t none = INT64_MAX;
    int64_t first_nan = none;
    int64_t best = none;
    float best_value = 0.0f;
    for (int64_t j = lane; j < width; j += kWave) {
        const float v = values[j];
        if (__builtin_isnan(v)) {
            if (first_nan == none) {
                first_nan = j;
            }
        } else if (best == none || v > best_value) {
            best = j;
            best_value = v;
        }
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        const int64_t other_nan = __shfl_xor(first_nan, offset, kWave);
        const int64_t other_best = __shfl_xor(best, offset, kWave);
        const float other_value = __shfl_xor(best_value, offset, kWave);
        first_nan = other_nan < first_nan ? other_nan : first_nan;
        if (other_best != none &&
            (best == none || other_value > best_value ||
             (other_value == best_value && other_best < best))) {
            best = other_best;
            best_value = other_value;
        }
    }
    if (lane == 0) {
        out[row] = first_nan != none ? first_nan : (best != none ? best : 0);
    }
}

__global__ void binary_kernel(int op, const float* __restrict__ a, const float* __restrict__ b,
                              float alpha, float* __restrict__ out, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride) {
        float v;
        if (op == MFR_EW_ADD) {
            v = a[i] + b[i];
        } else if (op == MFR_EW_MUL) {
            v = a[i] * b[i];
        } else {
            v = alpha * a[i];
        }
        out[i] = v;
    }
}

} // namespace

extern "C" {

int mfr_elementwise(mfr_stream_t stream, int op, const float* a, const float* b, float alpha,
                    float* out, int64_t n) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        mfr::require(op == MFR_EW_ADD || op == MFR_EW_MUL || op == MFR_EW_SCAL,
                     "elementwise: unknown op");
        mfr::require(n >= 0, "elementwise: negative count");
        if (n == 0) {
            return;
        }
        mfr::require(a != nullptr && out != nullptr && (op == MFR_EW_SCAL || b != nullptr),
                     "elementwise: null pointer");
        binary_kernel<<<mfr::grid_blocks(n, 256, 16384), 256, 0, s.stream>>>(op, a, b, alpha, out,
                                                                             n);
        mfr::check_launch("binary_kernel");
    });
}

int mfr_bias_act(mfr_stream_t stream, const float* x, const float* bias, float* y, int64_t rows,
                 int64_t cols, int act) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        mfr::require(rows >= 0 && cols >= 0, "bias_act: negative dimension");
        mfr::require(act == MFR_ACT_NONE || act == MFR_ACT_GELU_TANH || act == MFR_ACT_GELU_ERF,
                     "bias_act: unknown activation");
        const int64_t n = rows * cols;
        if (n == 0) {
            return;
        }
        mfr::require(x != nullptr && y != nullptr, "bias_act: null pointer");
        const bool vec4 = cols % 4 == 0 && mfr::aligned16(x) && mfr::aligned16(y) &&
                          (bias == nullptr || mfr::aligned16(bias));
        if (vec4) {
            bias_act_kernel<true><<<mfr::grid_blocks(n / 4, 256, 16384), 256, 0, s.stream>>>(
                x, bias, y, rows, cols, act);
        } else {
            bias_act_kernel<false><<<mfr::grid_blocks(n, 256, 16384), 256, 0, s.stream>>>(
                x, bias, y, rows, cols, act);
        }
        mfr::check_launch("bias_act_kernel");
    });
}

int mfr_where(mfr_stream_t stream, const uint8_t* cond, const float* x, const float* y, float* out,
              int64_t n) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        mfr::require(n >= 0, "where: negative count");
        if (n == 0) {
            return;
        }
        mfr::require(cond != nullptr && x != nullptr && y != nullptr && out != nullptr,
                     "where: null pointer");
        where_kernel<<<mfr::grid_blocks(n, 256, 16384), 256, 0, s.stream>>>(cond, x, y, out, n);
        mfr::check_launch("where_kernel");
    });
}

int mfr_softmax(mfr_stream_t stream, const float* x, float* y, int64_t outer, int64_t length,
                int64_t inner) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        mfr::require(outer >= 0 && length >= 0 && inner >= 0, "softmax: negative dimension");
        const int64_t lines = outer * inner;
        if (lines == 0 || length == 0) {
            return;
        }
        mfr::require(x != nullptr && y != nullptr, "softmax: null pointer");
        const unsigned blocks = mfr::grid_blocks(lines, 4);
        if (inner == 1 && length <= 64 * 4) {
            softmax_rows_reg_kernel<4><<<blocks, 256, 0, s.stream>>>(x, y, lines, length);
        } else if (inner == 1 && length <= 64 * 16) {
            softmax_rows_reg_kernel<16><<<blocks, 256, 0, s.stream>>>(x, y, lines, length);
        } else if (inner == 1 && length <= 64 * 32) {
            softmax_rows_reg_kernel<32><<<blocks, 256, 0, s.stream>>>(x, y, lines, length);
        } else {
            softmax_lines_kernel<<<blocks, 256, 0, s.stream>>>(x, y, outer, length, inner);
        }
        mfr::check_launch("softmax_kernel");
    });
}

int mfr_argmax(mfr_stream_t stream, const float* x, int64_t* out, int64_t rows, int64_t width) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        mfr::require(rows >= 0 && width >= 0, "argmax: negative dimension");
        if (rows == 0) {
            return;
        }
        mfr::require(out != nullptr && (width == 0 || x != nullptr), "argmax: null pointer");
        argmax_kernel<<<mfr::grid_blocks(rows, 4), 256, 0, s.stream>>>(x, out, rows, width);
        mfr::check_launch("argmax_kernel");
    });
}

} // extern "C"
