// Elementwise, softmax and argmax kernels of the hot path on gfx950. All are one pass over HBM
// (or two for softmax rows that do not fit in registers); each follows the reference CPU
// kernel's arithmetic so results round the same way:
//   bias_add + gelu   src/backends/cpu/ops/elementwise/elementwise.cpp:128-137, 173-194
//   where             elementwise.cpp:64-70
//   softmax           src/backends/cpu/ops/softmax/softmax.cpp:13-49
//   argmax            src/backends/cpu/ops/reduction/reduction.cpp:284-296
#include "common.hpp"

#include <type_traits>

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

// Rows that 16-byte accesses cannot take (cols % 4 != 0 or unaligned: X W + b at 4099
// columns), cols >= 64: workgroups take rows in turn, threads the columns of a row (coalesced
// 4-byte accesses, no division per element), ACT fixed per instantiation.
template <int ACT>
__global__ __launch_bounds__(256) void bias_act_rows_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ bias,
                                                            float* y, int64_t rows,
                                                            int64_t cols) {
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + r * cols;
        float* yr = y + r * cols;
        for (int64_t c = threadIdx.x; c < cols; c += 256) {
            float v = xr[c];
            if (bias != nullptr) {
                v = v + bias[c];
            }
            if constexpr (ACT != MFR_ACT_NONE) {
                v = mfr::dev::gelu(v, ACT);
            }
            yr[c] = v;
        }
    }
}

// ---- 16-byte streaming forms (every pointer 16-byte aligned; cond 4-byte aligned) ----------
//
// Each workgroup streams one contiguous chunk of `chunk` quads (4 elements), its threads kStreamUnroll
// quads apart per step with every load of a step issued before any is used, non-temporal (each
// element is read once), as the device copy streams. The last n % 4 elements go to the scalar
// kernels.
constexpr int kStreamThreads = 256;
constexpr int kStreamUnroll = 4;

inline bool aligned_to(const void* p, uintptr_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}

// Workgroups and quads per workgroup for `quads` quads (at most 4096 workgroups).
inline void stream_shape(int64_t quads, unsigned* blocks, int64_t* chunk) {
    const int64_t per_step = static_cast<int64_t>(kStreamThreads) * kStreamUnroll;
    int64_t b = (quads + per_step - 1) / per_step;
    b = b < 1 ? 1 : (b > 4096 ? 4096 : b);
    *chunk = (quads + b - 1) / b;
    *blocks = static_cast<unsigned>((quads + *chunk - 1) / *chunk);
}

// STREAM: non-temporal stores (outputs larger than the last-level cache).
template <bool STREAM>
__global__ __launch_bounds__(kStreamThreads) void where4_kernel(
    const uint32_t* __restrict__ cond, const float4* __restrict__ x, const float4* __restrict__ y,
    float4* __restrict__ out, int64_t quads, int64_t chunk) {
    const int64_t begin = static_cast<int64_t>(blockIdx.x) * chunk;
    const int64_t end = begin + chunk < quads ? begin + chunk : quads;
    for (int64_t i = begin + threadIdx.x; i < end; i += kStreamThreads * kStreamUnroll) {
        uint32_t c[kStreamUnroll];
        float4 xv[kStreamUnroll], yv[kStreamUnroll];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t j = i + u * kStreamThreads;
            if (j < end) {
                c[u] = __builtin_nontemporal_load(cond + j);
                xv[u] = mfr::dev::load_streaming(reinterpret_cast<const float*>(x + j));
                yv[u] = mfr::dev::load_streaming(reinterpret_cast<const float*>(y + j));
            }
        }
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t j = i + u * kStreamThreads;
            if (j < end) {
                float4 v;
                v.x = (c[u] & 0xffu) != 0 ? xv[u].x : yv[u].x;
                v.y = (c[u] & 0xff00u) != 0 ? xv[u].y : yv[u].y;
                v.z = (c[u] & 0xff0000u) != 0 ? xv[u].z : yv[u].z;
                v.w = (c[u] & 0xff000000u) != 0 ? xv[u].w : yv[u].w;
                if constexpr (STREAM) {
                    mfr::dev::store_streaming(reinterpret_cast<float*>(out + j), v);
                } else {
                    out[j] = v;
                }
            }
        }
    }
}

template <int OP, bool STREAM>
__global__ __launch_bounds__(kStreamThreads) void binary4_kernel(const float4* __restrict__ a,
                                                                 const float4* __restrict__ b,
                                                                 float alpha,
                                                                 float4* __restrict__ out,
                                                                 int64_t quads, int64_t chunk) {
    const int64_t begin = static_cast<int64_t>(blockIdx.x) * chunk;
    const int64_t end = begin + chunk < quads ? begin + chunk : quads;
    for (int64_t i = begin + threadIdx.x; i < end; i += kStreamThreads * kStreamUnroll) {
        float4 av[kStreamUnroll], bv[kStreamUnroll];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t j = i + u * kStreamThreads;
            if (j < end) {
                av[u] = mfr::dev::load_streaming(reinterpret_cast<const float*>(a + j));
                if constexpr (OP != MFR_EW_SCAL) {
                    bv[u] = mfr::dev::load_streaming(reinterpret_cast<const float*>(b + j));
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t j = i + u * kStreamThreads;
            if (j < end) {
                float4 v;
                if constexpr (OP == MFR_EW_ADD) {
                    v = make_float4(av[u].x + bv[u].x, av[u].y + bv[u].y, av[u].z + bv[u].z,
                                    av[u].w + bv[u].w);
                } else if constexpr (OP == MFR_EW_SUB) {
                    v = make_float4(av[u].x - bv[u].x, av[u].y - bv[u].y, av[u].z - bv[u].z,
                                    av[u].w - bv[u].w);
                } else if constexpr (OP == MFR_EW_MUL) {
                    v = make_float4(av[u].x * bv[u].x, av[u].y * bv[u].y, av[u].z * bv[u].z,
                                    av[u].w * bv[u].w);
                } else {
                    v = make_float4(alpha * av[u].x, alpha * av[u].y, alpha * av[u].z,
                                    alpha * av[u].w);
                }
                if constexpr (STREAM) {
                    mfr::dev::store_streaming(reinterpret_cast<float*>(out + j), v);
                } else {
                    out[j] = v;
                }
            }
        }
    }
}

// ---- where over strided operands -------------------------------------------------------------
//
// out (contiguous, row-major) = cond ? x : y where each operand is read through its own strides,
// 0 on a broadcast dimension (attention's -inf scalar and [Lq, Lk] mask expanded over
// [B, H, Lq, Lk] read 1 element and 1 MiB, not 512 and 128 MiB). The output is walked as rows of
// its last dimension; a row's operand bases come from its index over the outer dimensions.
//
// Launch: workgroup (i, j) takes rows R * i .. R * i + R - 1 and, in each, the column chunks
// j, j + gridDim.y, ... of 256 threads. The R rows' loads are all issued before any is used, and
// the row index is divided into its outer coordinates once per workgroup (in 32 bits where the
// row count allows), then stepped (a 64-bit division per dimension per row made the attention
// mask's where bound by integer arithmetic, not memory; once per workgroup in 64 bits it still
// cost attention's mask 103 against 78 us). R: 8 for the in-place kernel (attention's mask over
// 512 MiB of scores: 130, 97, 78 and 80 us with 2, 4, 8 and 16 rows per workgroup), 4 for the
// others (the same where out of place: 239, 247, 228 and 251 us with 1, 2, 4 and 8).
struct WhereLayout {
    int outer_dims;                     // dimensions before the last
    int64_t shape[MFR_MAX_COPY_DIMS];   // outer extents, outermost first
    int64_t cs[MFR_MAX_COPY_DIMS];      // outer strides of cond, x, y
    int64_t xs[MFR_MAX_COPY_DIMS];
    int64_t ys[MFR_MAX_COPY_DIMS];
    int64_t rows, row_len;              // product of the outer extents; the last extent
    int64_t c_inner, x_inner, y_inner;  // strides along the last dimension
};

constexpr int kWhereRowsInPlace = 8;
constexpr int kWhereRows = 4;

// The operand offsets of R consecutive rows from `first` (rows past the end get whatever the
// odometer gives; callers skip them).
template <int R> struct WhereRows {
    int64_t c[R], x[R], y[R];

    __device__ WhereRows(const WhereLayout& l, int64_t first) {
        // Outer coordinates of `first`, innermost first: in 32 bits when every row index fits
        // (a 64-bit division is a long instruction sequence, run by every workgroup of R rows
        // once per dimension), else in 64.
        int64_t idx[MFR_MAX_COPY_DIMS];
        int64_t oc = 0, ox = 0, oy = 0;
        // The innermost outer dimension's index, extent and strides.
        int64_t i0 = 0, n0 = 1, c0 = 0, x0 = 0, y0 = 0;
        const bool narrow = l.rows <= int64_t{0xffffffff};
        uint32_t row32 = static_cast<uint32_t>(first);
        int64_t row = first;
#pragma unroll
        for (int d = MFR_MAX_COPY_DIMS - 1; d >= 0; --d) {
            idx[d] = 0;
            if (d < l.outer_dims) {
                int64_t i;
                if (narrow) {
                    const uint32_t n = static_cast<uint32_t>(l.shape[d]);
                    i = row32 % n;
                    row32 /= n;
                } else {
                    i = row % l.shape[d];
                    row /= l.shape[d];
                }
                idx[d] = i;
                oc += i * l.cs[d];
                ox += i * l.xs[d];
                oy += i * l.ys[d];
                if (d == l.outer_dims - 1) {
                    i0 = i;
                    n0 = l.shape[d];
                    c0 = l.cs[d];
                    x0 = l.xs[d];
                    y0 = l.ys[d];
                }
            }
        }
        if (i0 + R <= n0) {
            // The R rows stay within the innermost outer dimension: each row is the one before
            // plus that dimension's strides (attention's rows: 8 of every 1024 queries).
#pragma unroll
            for (int u = 0; u < R; ++u) {
                c[u] = oc + u * c0;
                x[u] = ox + u * x0;
                y[u] = oy + u * y0;
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < R; ++u) {
            c[u] = oc;
            x[u] = ox;
            y[u] = oy;
            // Next row: the innermost outer index steps, carrying outward.
            bool carry = true;
#pragma unroll
            for (int d = MFR_MAX_COPY_DIMS - 1; d >= 0; --d) {
                if (carry && d < l.outer_dims) {
                    oc += l.cs[d];
                    ox += l.xs[d];
                    oy += l.ys[d];
                    if (++idx[d] < l.shape[d]) {
                        carry = false;
                    } else {
                        idx[d] = 0;
                        oc -= l.cs[d] * l.shape[d];
                        ox -= l.xs[d] * l.shape[d];
                        oy -= l.ys[d] * l.shape[d];
                    }
                }
            }
        }
    }
};

__device__ inline uint32_t where_cond4(const uint8_t* cond, int64_t base, int64_t inner,
                                       int64_t q) {
    if (inner == 0) {
        return cond[base] != 0 ? 0x01010101u : 0u;
    }
    return *reinterpret_cast<const uint32_t*>(cond + base + 4 * q);
}

__device__ inline float4 where_value4(const float* v, int64_t base, int64_t inner, int64_t q) {
    if (inner == 0) {
        const float w = v[base];
        return make_float4(w, w, w, w);
    }
    return mfr::dev::load_streaming(v + base + 4 * q);
}

// Rows whose length is a multiple of 4, out 16-byte aligned; each operand's inner stride is 0
// (one value per row) or 1 with 16-byte (x, y) / 4-byte (cond) aligned row starts, checked on the
// host. A thread takes one quad of each of the workgroup's rows.
template <bool STREAM, int R = kWhereRows>
__global__ __launch_bounds__(256) void where_rows4_kernel(const uint8_t* __restrict__ cond,
                                                          const float* __restrict__ x,
                                                          const float* __restrict__ y,
                                                          float* __restrict__ out, WhereLayout l) {
    const int64_t quads = l.row_len / 4;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * R;
    const WhereRows<R> r(l, first);
    for (int64_t q = static_cast<int64_t>(blockIdx.y) * 256 + threadIdx.x; q < quads;
         q += static_cast<int64_t>(gridDim.y) * 256) {
        uint32_t c[R];
        float4 xv[R], yv[R];
#pragma unroll
        for (int u = 0; u < R; ++u) {
            if (first + u < l.rows) {
                c[u] = where_cond4(cond, r.c[u], l.c_inner, q);
                xv[u] = where_value4(x, r.x[u], l.x_inner, q);
                yv[u] = where_value4(y, r.y[u], l.y_inner, q);
            }
        }
#pragma unroll
        for (int u = 0; u < R; ++u) {
            if (first + u < l.rows) {
                float4 v;
                v.x = (c[u] & 0xffu) != 0 ? xv[u].x : yv[u].x;
                v.y = (c[u] & 0xff00u) != 0 ? xv[u].y : yv[u].y;
                v.z = (c[u] & 0xff0000u) != 0 ? xv[u].z : yv[u].z;
                v.w = (c[u] & 0xff000000u) != 0 ? xv[u].w : yv[u].w;
                float* o = out + (first + u) * l.row_len + 4 * q;
                if constexpr (STREAM) {
                    mfr::dev::store_streaming(o, v);
                } else {
                    *reinterpret_cast<float4*>(o) = v;
                }
            }
        }
    }
}

// In place: out is also one of the operands, through the output's own (packed) layout, so the
// elements that keep that operand are already right. Only the others are written: from y where
// cond is false (out aliases x, KEEP_X) or from x where it is true. The aliased operand is never
// read. For attention's masks (where(keep, scores, -inf, out=scores)) that is the masked keys'
// -inf alone, not a read and a write of every score.
template <bool KEEP_X, bool STREAM, int R = kWhereRowsInPlace>
__global__ __launch_bounds__(256) void where_rows4_inplace_kernel(const uint8_t* __restrict__ cond,
                                                                  const float* __restrict__ other,
                                                                  float* out, WhereLayout l) {
    const int64_t quads = l.row_len / 4;
    const int64_t other_inner = KEEP_X ? l.y_inner : l.x_inner;
    const int64_t first = static_cast<int64_t>(blockIdx.x) * R;
    const WhereRows<R> r(l, first);
    for (int64_t q = static_cast<int64_t>(blockIdx.y) * 256 + threadIdx.x; q < quads;
         q += static_cast<int64_t>(gridDim.y) * 256) {
        uint32_t take[R];
#pragma unroll
        for (int u = 0; u < R; ++u) {
            // Lanes (bytes) that take `other`: cond false when out is x, true when it is y.
            const uint32_t c = first + u < l.rows ? where_cond4(cond, r.c[u], l.c_inner, q)
                                                  : (KEEP_X ? 0x01010101u : 0u);
            take[u] = KEEP_X ? ~c & 0x01010101u : c & 0x01010101u;
        }
#pragma unroll
        for (int u = 0; u < R; ++u) {
            if (take[u] == 0u) {
                continue;
            }
            const float4 v = where_value4(other, KEEP_X ? r.y[u] : r.x[u], other_inner, q);
            float* dst = out + (first + u) * l.row_len + 4 * q;
            if (take[u] == 0x01010101u) {
                if constexpr (STREAM) {
                    mfr::dev::store_streaming(dst, v);
                } else {
                    *reinterpret_cast<float4*>(dst) = v;
                }
            } else {
                if (take[u] & 0x1u) dst[0] = v.x;
                if (take[u] & 0x100u) dst[1] = v.y;
                if (take[u] & 0x10000u) dst[2] = v.z;
                if (take[u] & 0x1000000u) dst[3] = v.w;
            }
        }
    }
}

// Any strides: one element of each of the workgroup's rows per thread and step.
template <int R = kWhereRows>
__global__ __launch_bounds__(256) void where_rows_kernel(const uint8_t* __restrict__ cond,
                                                         const float* __restrict__ x,
                                                         const float* __restrict__ y,
                                                         float* __restrict__ out, WhereLayout l) {
    const int64_t first = static_cast<int64_t>(blockIdx.x) * R;
    const WhereRows<R> r(l, first);
    for (int64_t j = static_cast<int64_t>(blockIdx.y) * 256 + threadIdx.x; j < l.row_len;
         j += static_cast<int64_t>(gridDim.y) * 256) {
        float v[R];
#pragma unroll
        for (int u = 0; u < R; ++u) {
            if (first + u < l.rows) {
                v[u] = cond[r.c[u] + j * l.c_inner] != 0 ? x[r.x[u] + j * l.x_inner]
                                                         : y[r.y[u] + j * l.y_inner];
            }
        }
#pragma unroll
        for (int u = 0; u < R; ++u) {
            if (first + u < l.rows) {
                out[(first + u) * l.row_len + j] = v[u];
            }
        }
    }
}

// The reference's line maximum: a NaN anywhere makes it NaN (the scan stops at the first NaN),
// otherwise the largest value (-inf for an empty or all -inf line).
__device__ inline float line_max(float m, int has_nan) { return has_nan ? NAN : m; }

// Softmax of contiguous lines (inner == 1), one wavefront per line, the line held in registers:
// each lane keeps kPer values at positions lane + 64*i.
template <int kPer, bool STREAM>
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
            if constexpr (STREAM) {
                __builtin_nontemporal_store(v[i] * scale, out + j);
            } else {
                out[j] = v[i] * scale;
            }
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
        } else if (op == MFR_EW_SUB) {
            v = a[i] - b[i];
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
        mfr::require(op == MFR_EW_ADD || op == MFR_EW_SUB || op == MFR_EW_MUL ||
                         op == MFR_EW_SCAL,
                     "elementwise: unknown op");
        mfr::require(n >= 0, "elementwise: negative count");
        if (n == 0) {
            return;
        }
        mfr::require(a != nullptr && out != nullptr && (op == MFR_EW_SCAL || b != nullptr),
                     "elementwise: null pointer");
        int64_t done = 0;
        if (aligned_to(a, 16) && aligned_to(out, 16) && (op == MFR_EW_SCAL || aligned_to(b, 16)) &&
            n >= 4) {
            const int64_t quads = n / 4;
            unsigned blocks = 0;
            int64_t chunk = 0;
            stream_shape(quads, &blocks, &chunk);
            const auto* a4 = reinterpret_cast<const float4*>(a);
            const auto* b4 = reinterpret_cast<const float4*>(b);
            auto* o4 = reinterpret_cast<float4*>(out);
            // Outputs past the last-level cache stream (512 MiB add: 300 -> 290 us).
            const bool stream_out = 4.0 * static_cast<double>(n) > mfr::kLastLevelCacheBytes;
            auto run = [&](auto op_tag, auto stream_tag) {
                binary4_kernel<decltype(op_tag)::value, decltype(stream_tag)::value>
                    <<<blocks, kStreamThreads, 0, s.stream>>>(a4, b4, alpha, o4, quads, chunk);
            };
            using Add = std::integral_constant<int, MFR_EW_ADD>;
            using Sub = std::integral_constant<int, MFR_EW_SUB>;
            using Mul = std::integral_constant<int, MFR_EW_MUL>;
            using Scal = std::integral_constant<int, MFR_EW_SCAL>;
            const auto with_stream = [&](auto stream_tag) {
                if (op == MFR_EW_ADD) {
                    run(Add{}, stream_tag);
                } else if (op == MFR_EW_SUB) {
                    run(Sub{}, stream_tag);
                } else if (op == MFR_EW_MUL) {
                    run(Mul{}, stream_tag);
                } else {
                    run(Scal{}, stream_tag);
                }
            };
            if (stream_out) {
                with_stream(std::true_type{});
            } else {
                with_stream(std::false_type{});
            }
            mfr::check_launch("binary4_kernel");
            done = 4 * quads;
        }
        if (done < n) {
            const int64_t rest = n - done;
            binary_kernel<<<mfr::grid_blocks(rest, 256, 16384), 256, 0, s.stream>>>(
                op, a + done, op == MFR_EW_SCAL ? b : b + done, alpha, out + done, rest);
            mfr::check_launch("binary_kernel");
        }
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
        } else if (cols >= 64) {
            const unsigned grid = static_cast<unsigned>(rows < 16384 ? rows : 16384);
            if (act == MFR_ACT_NONE) {
                bias_act_rows_kernel<MFR_ACT_NONE><<<grid, 256, 0, s.stream>>>(x, bias, y, rows,
                                                                               cols);
            } else if (act == MFR_ACT_GELU_TANH) {
                bias_act_rows_kernel<MFR_ACT_GELU_TANH><<<grid, 256, 0, s.stream>>>(x, bias, y,
                                                                                    rows, cols);
            } else {
                bias_act_rows_kernel<MFR_ACT_GELU_ERF><<<grid, 256, 0, s.stream>>>(x, bias, y,
                                                                                   rows, cols);
            }
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
        int64_t done = 0;
        if (aligned_to(cond, 4) && aligned_to(x, 16) && aligned_to(y, 16) && aligned_to(out, 16) &&
            n >= 4) {
            const int64_t quads = n / 4;
            unsigned blocks = 0;
            int64_t chunk = 0;
            stream_shape(quads, &blocks, &chunk);
            // Outputs past the last-level cache stream (512 MiB: 327 -> 314 us).
            const bool stream_out = 4.0 * static_cast<double>(n) > mfr::kLastLevelCacheBytes;
            const auto* c4 = reinterpret_cast<const uint32_t*>(cond);
            const auto* x4 = reinterpret_cast<const float4*>(x);
            const auto* y4 = reinterpret_cast<const float4*>(y);
            auto* o4 = reinterpret_cast<float4*>(out);
            if (stream_out) {
                where4_kernel<true><<<blocks, kStreamThreads, 0, s.stream>>>(c4, x4, y4, o4, quads,
                                                                             chunk);
            } else {
                where4_kernel<false><<<blocks, kStreamThreads, 0, s.stream>>>(c4, x4, y4, o4,
                                                                              quads, chunk);
            }
            mfr::check_launch("where4_kernel");
            done = 4 * quads;
        }
        if (done < n) {
            const int64_t rest = n - done;
            where_kernel<<<mfr::grid_blocks(rest, 256, 16384), 256, 0, s.stream>>>(
                cond + done, x + done, y + done, out + done, rest);
            mfr::check_launch("where_kernel");
        }
    });
}

int mfr_where_nd(mfr_stream_t stream, int32_t ndim, const int64_t* shape, const uint8_t* cond,
                 const int64_t* cond_strides, const float* x, const int64_t* x_strides,
                 const float* y, const int64_t* y_strides, float* out) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        mfr::require(ndim >= 0 && ndim <= MFR_MAX_COPY_DIMS, "where_nd: too many dimensions");
        mfr::require(ndim == 0 || (shape != nullptr && cond_strides != nullptr &&
                                   x_strides != nullptr && y_strides != nullptr),
                     "where_nd: null shape or strides");
        // Dimensions of extent 1 are dropped (never stepped along); a 0-d call is one element.
        WhereLayout l{};
        int64_t ext[MFR_MAX_COPY_DIMS], cs[MFR_MAX_COPY_DIMS], xs[MFR_MAX_COPY_DIMS],
            ys[MFR_MAX_COPY_DIMS];
        int dims = 0;
        int64_t total = 1;
        for (int d = 0; d < ndim; ++d) {
            mfr::require(shape[d] >= 0, "where_nd: negative dimension");
            mfr::require(cond_strides[d] >= 0 && x_strides[d] >= 0 && y_strides[d] >= 0,
                         "where_nd: negative stride");
            total *= shape[d];
            if (shape[d] != 1) {
                ext[dims] = shape[d];
                cs[dims] = cond_strides[d];
                xs[dims] = x_strides[d];
                ys[dims] = y_strides[d];
                ++dims;
            }
        }
        if (total == 0) {
            return;
        }
        mfr::require(cond != nullptr && x != nullptr && y != nullptr && out != nullptr,
                     "where_nd: null pointer");
        if (dims == 0) {
            ext[0] = 1;
            cs[0] = xs[0] = ys[0] = 0;
            dims = 1;
        }
        l.outer_dims = dims - 1;
        l.rows = 1;
        for (int d = 0; d + 1 < dims; ++d) {
            l.shape[d] = ext[d];
            l.cs[d] = cs[d];
            l.xs[d] = xs[d];
            l.ys[d] = ys[d];
            l.rows *= ext[d];
        }
        l.row_len = ext[dims - 1];
        l.c_inner = cs[dims - 1];
        l.x_inner = xs[dims - 1];
        l.y_inner = ys[dims - 1];
        // Quads need: unit or zero inner strides, rows of a multiple of 4, and aligned row starts
        // (every outer stride a multiple of the vector's elements, aligned bases).
        auto rows_aligned = [&](const int64_t* strides, int64_t inner, int64_t elems,
                                const void* base, uintptr_t bytes) {
            if (inner == 0) {
                return true;
            }
            if (inner != 1 || !aligned_to(base, bytes)) {
                return false;
            }
            for (int d = 0; d < l.outer_dims; ++d) {
                if (strides[d] % elems != 0) {
                    return false;
                }
            }
            return true;
        };
        const bool quads = l.row_len % 4 == 0 && aligned_to(out, 16) &&
                           rows_aligned(l.cs, l.c_inner, 4, cond, 4) &&
                           rows_aligned(l.xs, l.x_inner, 4, x, 16) &&
                           rows_aligned(l.ys, l.y_inner, 4, y, 16);
        // R rows per workgroup along x; a row's columns in 256-thread chunks along y.
        const auto grid = [&](int rows_per_group) {
            const int64_t row_groups = (l.rows + rows_per_group - 1) / rows_per_group;
            mfr::require(row_groups < (int64_t{1} << 31), "where_nd: too many rows");
            const int64_t columns = quads ? l.row_len / 4 : l.row_len;
            const int64_t chunks = (columns + 255) / 256;
            return dim3(static_cast<unsigned>(row_groups),
                        static_cast<unsigned>(chunks < 65535 ? (chunks > 0 ? chunks : 1) : 65535));
        };
        const dim3 blocks = grid(kWhereRows);
        const dim3 blocks_in_place = grid(kWhereRowsInPlace);
        // Whether an operand is out itself, read through out's packed layout.
        const auto is_out = [&](const float* base, const int64_t* strides, int64_t inner) {
            if (base != out || inner != 1) {
                return false;
            }
            int64_t packed = l.row_len;
            for (int d = l.outer_dims - 1; d >= 0; --d) {
                if (strides[d] != packed) {
                    return false;
                }
                packed *= l.shape[d];
            }
            return true;
        };
        const bool stream_out = 4.0 * static_cast<double>(total) > mfr::kLastLevelCacheBytes;
        const bool out_is_x = is_out(x, l.xs, l.x_inner);
        const bool out_is_y = !out_is_x && is_out(y, l.ys, l.y_inner);
        if (quads && (out_is_x || out_is_y)) {
            const dim3 g = blocks_in_place;
            const float* other = out_is_x ? y : x;
            if (out_is_x && stream_out) {
                where_rows4_inplace_kernel<true, true><<<g, 256, 0, s.stream>>>(cond, other, out, l);
            } else if (out_is_x) {
                where_rows4_inplace_kernel<true, false><<<g, 256, 0, s.stream>>>(cond, other, out, l);
            } else if (stream_out) {
                where_rows4_inplace_kernel<false, true><<<g, 256, 0, s.stream>>>(cond, other, out, l);
            } else {
                where_rows4_inplace_kernel<false, false><<<g, 256, 0, s.stream>>>(cond, other, out, l);
            }
            mfr::check_launch("where_rows4_inplace_kernel");
        } else if (quads) {
            if (stream_out) {
                where_rows4_kernel<true><<<blocks, 256, 0, s.stream>>>(cond, x, y, out, l);
            } else {
                where_rows4_kernel<false><<<blocks, 256, 0, s.stream>>>(cond, x, y, out, l);
            }
            mfr::check_launch("where_rows4_kernel");
        } else {
            where_rows_kernel<><<<blocks, 256, 0, s.stream>>>(cond, x, y, out, l);
            mfr::check_launch("where_rows_kernel");
        }
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
        // Outputs past the last-level cache stream (512 MiB: 182 -> 178 us).
        const bool stream_out =
            4.0 * static_cast<double>(lines) * length > mfr::kLastLevelCacheBytes;
        if (inner == 1 && length <= 64 * 4) {
            softmax_rows_reg_kernel<4, false><<<blocks, 256, 0, s.stream>>>(x, y, lines, length);
        } else if (inner == 1 && length <= 64 * 16 && stream_out) {
            softmax_rows_reg_kernel<16, true><<<blocks, 256, 0, s.stream>>>(x, y, lines, length);
        } else if (inner == 1 && length <= 64 * 16) {
            softmax_rows_reg_kernel<16, false><<<blocks, 256, 0, s.stream>>>(x, y, lines, length);
        } else if (inner == 1 && length <= 64 * 32 && stream_out) {
            softmax_rows_reg_kernel<32, true><<<blocks, 256, 0, s.stream>>>(x, y, lines, length);
        } else if (inner == 1 && length <= 64 * 32) {
            softmax_rows_reg_kernel<32, false><<<blocks, 256, 0, s.stream>>>(x, y, lines, length);
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
