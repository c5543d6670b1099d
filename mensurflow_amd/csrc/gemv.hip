// fp32 matrix-vector products on gfx950, bound by HBM bandwidth:
//
//   y = alpha * op(A) * x + beta * y0       (mfr_sgemv, mfr_smatvec)
//
// Both forms accumulate in double and round once, as the reference's CPU kernels do
// (src/backends/cpu/ops/blas/blas.cpp:55-79). A product of two floats is exact in double, so a
// fused multiply-add in double rounds exactly like the reference's multiply-then-add; only the
// order of the additions differs, and it is fixed, so every call gives the same bits.
//
// N form (y has `rows` entries): one wavefront owns kRowsPerWave (4) rows and walks them with
// 16-byte loads, kUnrollN loads per row in flight per lane; each x chunk is read once for all 4
// rows. The partial sums are reduced across the wavefront with shuffles. Every byte of A is read
// once, coalesced. At 16384 rows this is 4096 wavefronts: one full round of the chip at 4
// wavefronts per SIMD, so no tail of half-empty rounds.
//
// T form (y has `cols` entries): a workgroup owns a strip of 256 columns (64 lanes x 4) and a
// chunk of rows; its four wavefronts split the chunk's rows, each lane keeps 4 column sums, and
// the wavefronts are added in LDS in a fixed order. The chunk's partial sums go to the stream's
// workspace ([chunks][cols] doubles) and a second kernel adds the chunks in order. A is again
// read once, coalesced along the rows.
#include "common.hpp"

namespace {

using mfr::dev::kWave;

constexpr int kRowsPerWave = 4;
constexpr int kWavesPerBlockN = 4;
constexpr int kUnrollN = 4;

// The reference's final rounding: (float)(alpha * sum + (beta == 0 ? 0 : (double)(beta * y0))),
// beta * y0 in float (blas.cpp:77).
__device__ inline float finish(double sum, float alpha, float beta, const float* y0, int64_t i) {
    const double tail = (beta == 0.0f || y0 == nullptr) ? 0.0 : static_cast<double>(beta * y0[i]);
    return static_cast<float>(static_cast<double>(alpha) * sum + tail);
}

// VEC4: rows start 16-byte aligned and cols % 4 == 0 (checked on the host).
template <bool VEC4>
__global__ __launch_bounds__(kWave* kWavesPerBlockN) void gemv_n_kernel(
    const float* __restrict__ a, int64_t lda, const float* __restrict__ x, int64_t rows,
    int64_t cols, float alpha, float beta, const float* __restrict__ y0, float* __restrict__ y) {
    const int lane = threadIdx.x % kWave;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlockN + threadIdx.x / kWave;
    const int64_t row0 = wave * kRowsPerWave;
    if (row0 >= rows) {
        return;
    }
    const int nrows = rows - row0 < kRowsPerWave ? static_cast<int>(rows - row0) : kRowsPerWave;
    double sum[kRowsPerWave];
    const float* arow[kRowsPerWave];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        sum[r] = 0.0;
        // Rows past the end repeat the last valid row; their sums are never stored.
        arow[r] = a + (row0 + (r < nrows ? r : nrows - 1)) * lda;
    }
    if constexpr (VEC4) {
        const int64_t quads = cols / 4;                 // float4 per row
        const int64_t step = static_cast<int64_t>(kWave) * kUnrollN; // quads per iteration
        int64_t q = lane;
        for (; q + (kUnrollN - 1) * kWave < quads; q += step) {
            float4 xv[kUnrollN];
            float4 av[kRowsPerWave][kUnrollN];
#pragma unroll
            for (int u = 0; u < kUnrollN; ++u) {
                xv[u] = reinterpret_cast<const float4*>(x)[q + u * kWave];
#pragma unroll
                for (int r = 0; r < kRowsPerWave; ++r) {
                    av[r][u] = mfr::dev::load_streaming(arow[r] + 4 * (q + u * kWave));
                }
            }
#pragma unroll
            for (int u = 0; u < kUnrollN; ++u) {
                const double x0 = xv[u].x, x1 = xv[u].y, x2 = xv[u].z, x3 = xv[u].w;
#pragma unroll
                for (int r = 0; r < kRowsPerWave; ++r) {
                    sum[r] = fma(static_cast<double>(av[r][u].x), x0, sum[r]);
                    sum[r] = fma(static_cast<double>(av[r][u].y), x1, sum[r]);
                    sum[r] = fma(static_cast<double>(av[r][u].z), x2, sum[r]);
                    sum[r] = fma(static_cast<double>(av[r][u].w), x3, sum[r]);
                }
            }
        }
        for (; q < quads; q += kWave) {
            const float4 xv = reinterpret_cast<const float4*>(x)[q];
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) {
                const float4 av = reinterpret_cast<const float4*>(arow[r])[q];
                sum[r] = fma(static_cast<double>(av.x), static_cast<double>(xv.x), sum[r]);
                sum[r] = fma(static_cast<double>(av.y), static_cast<double>(xv.y), sum[r]);
                sum[r] = fma(static_cast<double>(av.z), static_cast<double>(xv.z), sum[r]);
                sum[r] = fma(static_cast<double>(av.w), static_cast<double>(xv.w), sum[r]);
            }
        }
    } else {
        for (int64_t j = lane; j < cols; j += kWave) {
            const double xj = static_cast<double>(x[j]);
#pragma unroll
            for (int r = 0; r < kRowsPerWave; ++r) {
                sum[r] = fma(static_cast<double>(arow[r][j]), xj, sum[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        sum[r] = mfr::dev::wave_sum(sum[r]);
    }
    if (lane == 0) {
        for (int r = 0; r < nrows; ++r) {
            y[row0 + r] = finish(sum[r], alpha, beta, y0, row0 + r);
        }
    }
}

constexpr int kStripCols = 256; // columns per workgroup in the T form: 64 lanes x 4
constexpr int kWavesPerBlockT = 4;
constexpr int kUnrollT = 8;

// Partial sums of one (column strip, row chunk) tile of A^T x: out[chunk][col], in double.
// VEC4: lda % 4 == 0, cols % 4 == 0 and A 16-byte aligned, so a lane's 4 columns are one float4.
template <bool VEC4>
__global__ __launch_bounds__(kWave* kWavesPerBlockT) void gemv_t_partial_kernel(
    const float* __restrict__ a, int64_t lda, const float* __restrict__ x, int64_t rows,
    int64_t cols, int64_t rows_per_chunk, double* __restrict__ partial) {
    __shared__ double exchange[kWavesPerBlockT - 1][kStripCols];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int64_t strip = blockIdx.x;
    const int64_t chunk = blockIdx.y;
    const int64_t r_begin = chunk * rows_per_chunk;
    const int64_t r_end = r_begin + rows_per_chunk < rows ? r_begin + rows_per_chunk : rows;
    // Column of component c of this lane: VEC4 -> 4 adjacent columns, else 4 columns 64 apart.
    const int64_t col_base = strip * kStripCols + (VEC4 ? 4 * lane : lane);
    double sum[4] = {0.0, 0.0, 0.0, 0.0};
    if constexpr (VEC4) {
        const bool active = col_base < cols;
        int64_t r = r_begin + wave;
        const int64_t row_step = kWavesPerBlockT;
        for (; r + (kUnrollT - 1) * row_step < r_end; r += kUnrollT * row_step) {
            float4 av[kUnrollT];
            float xr[kUnrollT];
#pragma unroll
            for (int u = 0; u < kUnrollT; ++u) {
                const int64_t row = r + u * row_step;
                xr[u] = x[row];
                av[u] = active ? mfr::dev::load_streaming(a + row * lda + col_base)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < kUnrollT; ++u) {
                const double xv = static_cast<double>(xr[u]);
                sum[0] = fma(static_cast<double>(av[u].x), xv, sum[0]);
                sum[1] = fma(static_cast<double>(av[u].y), xv, sum[1]);
                sum[2] = fma(static_cast<double>(av[u].z), xv, sum[2]);
                sum[3] = fma(static_cast<double>(av[u].w), xv, sum[3]);
            }
        }
        for (; r < r_end; r += row_step) {
            const double xv = static_cast<double>(x[r]);
            if (active) {
                const float4 av = *reinterpret_cast<const float4*>(a + r * lda + col_base);
                sum[0] = fma(static_cast<double>(av.x), xv, sum[0]);
                sum[1] = fma(static_cast<double>(av.y), xv, sum[1]);
                sum[2] = fma(static_cast<double>(av.z), xv, sum[2]);
                sum[3] = fma(static_cast<double>(av.w), xv, sum[3]);
            }
        }
    } else {
        for (int64_t r = r_begin + wave; r < r_end; r += kWavesPerBlockT) {
            const double xv = static_cast<double>(x[r]);
            const float* row = a + r * lda;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int64_t col = col_base + c * kWave;
                if (col < cols) {
                    sum[c] = fma(static_cast<double>(row[col]), xv, sum[c]);
                }
            }
        }
    }
    // Wavefronts 1..3 hand their sums to wavefront 0, which adds them in order 0, 1, 2, 3.
    auto local_col = [&](int c) { return VEC4 ? 4 * lane + c : lane + c * kWave; };
    if (wave > 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            exchange[wave - 1][local_col(c)] = sum[c];
        }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            double total = sum[c];
#pragma unroll
            for (int w = 0; w < kWavesPerBlockT - 1; ++w) {
                total += exchange[w][local_col(c)];
            }
            const int64_t col = strip * kStripCols + local_col(c);
            if (col < cols) {
                partial[chunk * cols + col] = total;
            }
        }
    }
}

// y[j] = finish(sum over chunks (in order) of partial[chunk][j]).
__global__ void gemv_t_finish_kernel(const double* __restrict__ partial, int64_t chunks,
                                     int64_t cols, float alpha, float beta,
                                     const float* __restrict__ y0, float* __restrict__ y) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (j >= cols) {
        return;
    }
    double sum = 0.0;
    for (int64_t c = 0; c < chunks; ++c) {
        sum += partial[c * cols + j];
    }
    y[j] = finish(sum, alpha, beta, y0, j);
}

// Rows per chunk of the T form: enough (strip, chunk) tiles to cover the chip several times
// (256 CUs), each chunk a multiple of the unrolled row step, at least 64 rows.
int64_t t_rows_per_chunk(int64_t rows, int64_t strips) {
    // 1024 workgroups of 4 wavefronts: one full round of 256 CUs x 4 SIMDs x 4 wavefronts.
    const int64_t target_tiles = 1024;
    int64_t chunks = (target_tiles + strips - 1) / strips;
    if (chunks < 1) {
        chunks = 1;
    }
    int64_t per = (rows + chunks - 1) / chunks;
    const int64_t step = static_cast<int64_t>(kWavesPerBlockT) * kUnrollT;
    per = (per + step - 1) / step * step;
    return per < 64 ? 64 : per;
}

void launch_gemv(mfr_stream& s, bool trans, int64_t rows, int64_t cols, float alpha,
                 const float* a, int64_t lda, const float* x, float beta, const float* y0,
                 float* y) {
    mfr::require(rows >= 0 && cols >= 0, "gemv: negative dimension");
    mfr::require(lda >= cols, "gemv: lda smaller than cols");
    const int64_t outputs = trans ? cols : rows;
    if (outputs == 0) {
        return;
    }
    mfr::require(y != nullptr, "gemv: null y");
    mfr::require(!(beta != 0.0f && y0 == nullptr), "gemv: beta requires y0");
    // With no products (inputs == 0) A and x are never read: y = alpha * 0 + beta * y0.
    const int64_t inputs = trans ? rows : cols;
    mfr::require(inputs == 0 || (a != nullptr && x != nullptr), "gemv: null A or x");
    const bool vec4 = mfr::aligned16(a) && lda % 4 == 0 && cols % 4 == 0 &&
                      (!trans ? mfr::aligned16(x) : true);
    if (!trans) {
        const int64_t waves = (rows + kRowsPerWave - 1) / kRowsPerWave;
        const unsigned blocks = mfr::grid_blocks(waves, kWavesPerBlockN);
        if (vec4) {
            gemv_n_kernel<true><<<blocks, kWave * kWavesPerBlockN, 0, s.stream>>>(
                a, lda, x, rows, cols, alpha, beta, y0, y);
        } else {
            gemv_n_kernel<false><<<blocks, kWave * kWavesPerBlockN, 0, s.stream>>>(
                a, lda, x, rows, cols, alpha, beta, y0, y);
        }
        mfr::check_launch("gemv_n_kernel");
        return;
    }
    const int64_t strips = (cols + kStripCols - 1) / kStripCols;
    const int64_t per = rows > 0 ? t_rows_per_chunk(rows, strips) : 1;
    const int64_t chunks = rows > 0 ? (rows + per - 1) / per : 0;
    mfr::require(strips < (int64_t{1} << 31) && chunks < 65536, "gemv: matrix too large");
    double* partial = nullptr;
    if (chunks > 0) {
        partial = static_cast<double*>(
            s.reserve(static_cast<size_t>(chunks) * static_cast<size_t>(cols) * sizeof(double)));
        const dim3 grid(static_cast<unsigned>(strips), static_cast<unsigned>(chunks));
        if (vec4) {
            gemv_t_partial_kernel<true><<<grid, kWave * kWavesPerBlockT, 0, s.stream>>>(
                a, lda, x, rows, cols, per, partial);
        } else {
            gemv_t_partial_kernel<false><<<grid, kWave * kWavesPerBlockT, 0, s.stream>>>(
                a, lda, x, rows, cols, per, partial);
        }
        mfr::check_launch("gemv_t_partial_kernel");
    }
    gemv_t_finish_kernel<<<mfr::grid_blocks(cols, 256), 256, 0, s.stream>>>(
        partial, chunks, cols, alpha, beta, y0, y);
    mfr::check_launch("gemv_t_finish_kernel");
}

} // namespace

extern "C" {

int mfr_sgemv(mfr_stream_t stream, int trans, int64_t rows, int64_t cols, float alpha,
              const float* a, int64_t lda, const float* x, float beta, const float* y0, float* y) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        launch_gemv(s, trans != 0, rows, cols, alpha, a, lda, x, beta, y0, y);
    });
}

int mfr_smatvec(mfr_stream_t stream, int64_t m, int64_t k, const float* a, int64_t lda,
                const float* x, float* y) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        launch_gemv(s, false, m, k, 1.0f, a, lda, x, 0.0f, nullptr, y);
    });
}

} // extern "C"
