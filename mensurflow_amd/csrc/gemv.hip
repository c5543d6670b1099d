// fp32 matrix-vector products on gfx950, bound by HBM bandwidth:
//
//   y = alpha * op(A) * x + beta * y0       (mfr_sgemv, mfr_smatvec)
//
// Both forms accumulate in double and round once, as the reference's CPU kernels do
// (src/backends/cpu/ops/blas/blas.cpp:55-79). A product of two floats is exact in double, so a
// fused multiply-add in double rounds exactly like the reference's multiply-then-add; only the
// order of the additions differs, and it is fixed, so every call gives the same bits.
//
// N form (y has `rows` entries): one wavefront owns kRowsPerWave (8) rows and walks them with
// 16-byte loads, kUnrollN loads per row in flight per lane; each x chunk is read once for all 8
// rows. The partial sums are reduced across the wavefront with shuffles. Every byte of A is read
// once, coalesced. Workgroups of 2 wavefronts stream 16 consecutive rows; at 16384 rows that is
// 1024 workgroups (4 per CU), one round of the chip. Measured against 4 rows per wavefront in
// workgroups of 4: 6.89 vs 6.52 TB/s, the read rate of a plain contiguous stream (6.92 TB/s).
//
// T form (y has `cols` entries): a workgroup of one wavefront owns a strip of 256 columns
// (64 lanes x 4) and a chunk of rows, walks the rows in order with kUnrollT rows in flight, and
// each lane keeps 4 column sums. The chunk's partial sums go to the stream's workspace
// ([chunks][cols] doubles) and a second kernel adds the chunks in order. A is again read once,
// coalesced along the rows. At 16384^2: 64 strips x 32 chunks = 2048 wavefronts. Measured
// against four wavefronts splitting each chunk's rows (exchanging sums in LDS) with 8 rows in
// flight: 6.96 vs 6.44 TB/s.
#include "common.hpp"

namespace {

using mfr::dev::kWave;

constexpr int kRowsPerWave = 8;
constexpr int kWavesPerBlockN = 2;
constexpr int kUnrollN = 4;

// The reference's final rounding: (float)(alpha * sum + (beta == 0 ? 0 : (double)(beta * y0))),
// beta * y0 in float (blas.cpp:77).
__device__ inline float finish(double sum, float alpha, float beta, const float* y0, int64_t i) {
    const double tail = (beta == 0.0f || y0 == nullptr) ? 0.0 : static_cast<double>(beta * y0[i]);
    return static_cast<float>(static_cast<double>(alpha) * sum + tail);
}

// Per-lane sums of rows row0 .. row0 + kRowsPerWave - 1 of A times x. FULL: all kRowsPerWave
// rows exist, so they are lda apart from row0 and the compiler walks them from one base (that
// schedule streams faster); otherwise rows past the end repeat the last valid row, and their sums
// are never stored. VEC4: rows start 16-byte aligned and cols % 4 == 0 (checked on the host).
template <bool VEC4, bool FULL>
__device__ inline void gemv_n_rows(const float* __restrict__ a, int64_t lda,
                                   const float* __restrict__ x, int64_t cols, int64_t row0,
                                   int nrows, int lane, double (&sum)[kRowsPerWave]) {
    const float* arow[kRowsPerWave];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        sum[r] = 0.0;
        arow[r] = a + (row0 + (FULL || r < nrows ? r : nrows - 1)) * lda;
    }
    if constexpr (VEC4) {
        const int64_t quads = cols / 4;                              // float4 per row
        const int64_t step = static_cast<int64_t>(kWave) * kUnrollN; // quads per iteration
        const int64_t main_quads = quads / step * step;
        int64_t q = lane;
        for (; q < main_quads; q += step) {
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
}

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
    if (nrows == kRowsPerWave) {
        gemv_n_rows<VEC4, true>(a, lda, x, cols, row0, nrows, lane, sum);
    } else {
        gemv_n_rows<VEC4, false>(a, lda, x, cols, row0, nrows, lane, sum);
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
constexpr int kUnrollT = 16;

// Partial sums of one (column strip, row chunk) tile of A^T x: out[chunk][col], in double; one
// wavefront, rows in increasing order. VEC4: lda % 4 == 0, cols % 4 == 0 and A 16-byte aligned,
// so a lane's 4 columns are one float4; otherwise its columns are 64 apart.
template <bool VEC4>
__global__ __launch_bounds__(kWave) void gemv_t_partial_kernel(
    const float* __restrict__ a, int64_t lda, const float* __restrict__ x, int64_t rows,
    int64_t cols, int64_t rows_per_chunk, double* __restrict__ partial) {
    const int lane = threadIdx.x;
    const int64_t strip = blockIdx.x;
    const int64_t chunk = blockIdx.y;
    const int64_t r_begin = chunk * rows_per_chunk;
    const int64_t r_end = r_begin + rows_per_chunk < rows ? r_begin + rows_per_chunk : rows;
    // Column of component c of this lane: VEC4 -> 4 adjacent columns, else 4 columns 64 apart.
    auto local_col = [&](int c) { return VEC4 ? 4 * lane + c : lane + c * kWave; };
    const int64_t col_base = strip * kStripCols + local_col(0);
    double sum[4] = {0.0, 0.0, 0.0, 0.0};
    if constexpr (VEC4) {
        const bool active = col_base < cols;
        // A strip wholly inside the matrix (all but possibly the last) loads unconditionally;
        // the condition is uniform across the wavefront.
        const bool full_strip = (strip + 1) * kStripCols <= cols;
        int64_t r = r_begin;
        if (full_strip && r + kUnrollT <= r_end) {
            // x[r .. r+15] is the same for every lane (a scalar load); it is fetched one
            // iteration ahead (index clamped to the last row) so its latency overlaps the
            // current iteration instead of stalling the stream of A loads.
            float xr[kUnrollT];
#pragma unroll
            for (int u = 0; u < kUnrollT; ++u) {
                xr[u] = x[r + u];
            }
            for (; r + kUnrollT <= r_end; r += kUnrollT) {
                float4 av[kUnrollT];
#pragma unroll
                for (int u = 0; u < kUnrollT; ++u) {
                    av[u] = mfr::dev::load_streaming(a + (r + u) * lda + col_base);
                }
                float xn[kUnrollT];
#pragma unroll
                for (int u = 0; u < kUnrollT; ++u) {
                    const int64_t next = r + kUnrollT + u;
                    xn[u] = x[next < rows ? next : rows - 1];
                }
#pragma unroll
                for (int u = 0; u < kUnrollT; ++u) {
                    const double xv = static_cast<double>(xr[u]);
                    sum[0] = fma(static_cast<double>(av[u].x), xv, sum[0]);
                    sum[1] = fma(static_cast<double>(av[u].y), xv, sum[1]);
                    sum[2] = fma(static_cast<double>(av[u].z), xv, sum[2]);
                    sum[3] = fma(static_cast<double>(av[u].w), xv, sum[3]);
                }
#pragma unroll
                for (int u = 0; u < kUnrollT; ++u) {
                    xr[u] = xn[u];
                }
            }
        }
        for (; r < r_end; ++r) {
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
        for (int64_t r = r_begin; r < r_end; ++r) {
            const double xv = static_cast<double>(x[r]);
            const float* row = a + r * lda;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int64_t col = strip * kStripCols + local_col(c);
                if (col < cols) {
                    sum[c] = fma(static_cast<double>(row[col]), xv, sum[c]);
                }
            }
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int64_t col = strip * kStripCols + local_col(c);
        if (col < cols) {
            partial[chunk * cols + col] = sum[c];
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

// Rows per chunk of the T form: about 2048 (strip, chunk) wavefronts (2 per SIMD of 256 CUs,
// each with kUnrollT rows in flight), each chunk a multiple of the unrolled row step and at least
// 64 rows.
int64_t t_rows_per_chunk(int64_t rows, int64_t strips) {
    const int64_t target_tiles = 2048;
    int64_t chunks = (target_tiles + strips - 1) / strips;
    if (chunks < 1) {
        chunks = 1;
    }
    int64_t per = (rows + chunks - 1) / chunks;
    per = (per + kUnrollT - 1) / kUnrollT * kUnrollT;
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
    // Held until both kernels are queued: another thread's reserve() may not free `partial`
    // in between.
    std::lock_guard<std::mutex> hold(s.workspace_mutex);
    if (chunks > 0) {
        partial = static_cast<double*>(
            s.reserve(static_cast<size_t>(chunks) * static_cast<size_t>(cols) * sizeof(double)));
        const dim3 grid(static_cast<unsigned>(strips), static_cast<unsigned>(chunks));
        if (vec4) {
            gemv_t_partial_kernel<true><<<grid, kWave, 0, s.stream>>>(
                a, lda, x, rows, cols, per, partial);
        } else {
            gemv_t_partial_kernel<false><<<grid, kWave, 0, s.stream>>>(
                a, lda, x, rows, cols, per, partial);
        }
        mfr::check_launch("gemv_t_partial_kernel");
    }
    gemv_t_finish_kernel<<<mfr::grid_blocks(cols, 256), 256, 0, s.stream>>>(
        partial, chunks, cols, alpha, beta, y0, y);
    mfr::check_launch("gemv_t_finish_kernel");
}

// ---- dot --------------------------------------------------------------------------------------
//
// dot(x, y) = sum of x[i] y[i], as the reference's dot_f32 (src/backends/cpu/ops/blas/blas.cpp:
// 14-21): each product in double (exact), the sum in double, rounded once. Two passes in a fixed
// order that depends on n alone (so every device and every call gives the same bits): chunk c of
// kDotChunk elements is one workgroup, its threads walk it in float4 steps (thread t takes
// elements 4t .. 4t + 3 of each 1024, adding them in increasing order), and the threads' sums
// are added in a fixed tree; the second pass adds the chunks' sums the same way. HBM-bound:
// 8 bytes per element read.
constexpr int kDotThreads = 256;
constexpr int64_t kDotStep = 4 * kDotThreads;  // elements per workgroup step
constexpr int64_t kDotChunk = 16 * kDotStep;   // elements per workgroup (16384)

// The sum of v over the workgroup's threads in a fixed order: halves added pairwise in LDS.
__device__ inline double block_sum(double v, double* lds) {
    lds[threadIdx.x] = v;
    __syncthreads();
#pragma unroll
    for (int half = kDotThreads / 2; half > 0; half >>= 1) {
        if (static_cast<int>(threadIdx.x) < half) {
            lds[threadIdx.x] += lds[threadIdx.x + half];
        }
        __syncthreads();
    }
    return lds[0];
}

// VEC4: x and y 16-byte aligned (chunks start on multiples of kDotChunk elements, so every
// full float4 group is aligned too).
template <bool VEC4>
__global__ __launch_bounds__(kDotThreads) void dot_partial_kernel(const float* __restrict__ x,
                                                                  const float* __restrict__ y,
                                                                  int64_t n,
                                                                  double* __restrict__ partial) {
    __shared__ double lds[kDotThreads];
    const int64_t begin = static_cast<int64_t>(blockIdx.x) * kDotChunk;
    const int64_t end = begin + kDotChunk < n ? begin + kDotChunk : n;
    double sum = 0.0;
    for (int64_t i = begin + 4 * static_cast<int64_t>(threadIdx.x); i < end; i += kDotStep) {
        if (VEC4 && i + 3 < end) {
            const float4 a = mfr::dev::load_streaming(x + i);
            const float4 b = mfr::dev::load_streaming(y + i);
            sum = fma(static_cast<double>(a.x), static_cast<double>(b.x), sum);
            sum = fma(static_cast<double>(a.y), static_cast<double>(b.y), sum);
            sum = fma(static_cast<double>(a.z), static_cast<double>(b.z), sum);
            sum = fma(static_cast<double>(a.w), static_cast<double>(b.w), sum);
        } else {
            for (int64_t e = i; e < i + 4 && e < end; ++e) {
                sum = fma(static_cast<double>(x[e]), static_cast<double>(y[e]), sum);
            }
        }
    }
    const double total = block_sum(sum, lds);
    if (threadIdx.x == 0) {
        partial[blockIdx.x] = total;
    }
}

// *out = the chunks' sums added in a fixed order (thread t takes chunks t, t + 256, ... in
// order, then the tree), rounded to float.
__global__ __launch_bounds__(kDotThreads) void dot_finish_kernel(const double* __restrict__ partial,
                                                                 int64_t chunks,
                                                                 float* __restrict__ out) {
    __shared__ double lds[kDotThreads];
    double sum = 0.0;
    for (int64_t c = threadIdx.x; c < chunks; c += kDotThreads) {
        sum += partial[c];
    }
    const double total = block_sum(sum, lds);
    if (threadIdx.x == 0) {
        *out = static_cast<float>(total);
    }
}

void launch_dot(mfr_stream& s, int64_t n, const float* x, const float* y, float* out) {
    mfr::require(n >= 0, "dot: negative length");
    mfr::require(out != nullptr, "dot: null out");
    mfr::require(n == 0 || (x != nullptr && y != nullptr), "dot: null x or y");
    const int64_t chunks = (n + kDotChunk - 1) / kDotChunk;
    mfr::require(chunks < (int64_t{1} << 31), "dot: vector too long");
    // Held until both kernels are queued (another thread's reserve() may not free `partial`).
    std::lock_guard<std::mutex> hold(s.workspace_mutex);
    double* partial = nullptr;
    if (chunks > 0) {
        partial = static_cast<double*>(s.reserve(static_cast<size_t>(chunks) * sizeof(double)));
        const unsigned grid = static_cast<unsigned>(chunks);
        if (mfr::aligned16(x) && mfr::aligned16(y)) {
            dot_partial_kernel<true><<<grid, kDotThreads, 0, s.stream>>>(x, y, n, partial);
        } else {
            dot_partial_kernel<false><<<grid, kDotThreads, 0, s.stream>>>(x, y, n, partial);
        }
        mfr::check_launch("dot_partial_kernel");
    }
    dot_finish_kernel<<<1, kDotThreads, 0, s.stream>>>(partial, chunks, out);
    mfr::check_launch("dot_finish_kernel");
}

} // namespace

extern "C" {

int mfr_sdot(mfr_stream_t stream, int64_t n, const float* x, const float* y, float* out) {
    return mfr::guarded([&] {
        auto& s = mfr::stream_of(stream);
        launch_dot(s, n, x, y, out);
    });
}

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
