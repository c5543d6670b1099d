/*
 * oracle.c -- CPU restatement of mensurflow's fp32 BLAS hot path. TEST INFRASTRUCTURE ONLY:
 * the checker for the HIP kernels, never part of the product. See oracle.h for the contract of
 * each function; citations are path:line into bakir004/mensurflow.
 *
 * Built with -ffp-contract=off: the reference compiles its portable loops without FMA
 * (MENSURFLOW_NATIVE is OFF by default, CMakeLists.txt:20), so a*b + c must round twice here
 * too. Where the reference uses FMA (the AVX2 GEMM micro-kernel) this file calls fmaf().
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int orc_set_threads(int threads) {
#ifdef _OPENMP
    int previous = omp_get_max_threads();
    if (threads > 0) {
        omp_set_num_threads(threads);
    }
    return previous;
#else
    (void)threads;
    return 1;
#endif
}

/* ---- Philox4x32-10 and the seeded factories ----------------------------------------------- */

/* Ten rounds of the Philox4x32 bijection (Salmon et al., SC11) with the Weyl key schedule.
 * philox.hpp:14-27. */
void orc_philox4x32_10(const uint32_t counter[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t x0 = counter[0], x1 = counter[1], x2 = counter[2], x3 = counter[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; ++round) {
        const uint64_t lo_mul = (uint64_t)0xD2511F53u * x0;
        const uint64_t hi_mul = (uint64_t)0xCD9E8D57u * x2;
        const uint32_t y0 = (uint32_t)(hi_mul >> 32) ^ x1 ^ k0;
        const uint32_t y1 = (uint32_t)hi_mul;
        const uint32_t y2 = (uint32_t)(lo_mul >> 32) ^ x3 ^ k1;
        const uint32_t y3 = (uint32_t)lo_mul;
        x0 = y0;
        x1 = y1;
        x2 = y2;
        x3 = y3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = x0;
    out[1] = x1;
    out[2] = x2;
    out[3] = x3;
}

/* Block `block` of the stream of `seed`: counter {lo(block), hi(block), 0, 0}, key {lo(seed),
 * hi(seed)} (philox.hpp:29-34). */
static void philox_words(uint64_t seed, uint64_t block, uint32_t words[4]) {
    const uint32_t counter[4] = {(uint32_t)block, (uint32_t)(block >> 32), 0u, 0u};
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    orc_philox4x32_10(counter, key, words);
}

/* Element i of a factory call is word (offset + i) % 4 of block (offset + i) / 4
 * (random.cpp:16-37): the same stream for any split of a range into calls. */
void orc_uniform_f32(float* out, int64_t n, float low, float high, uint64_t seed, uint64_t offset) {
    if (low == high) {
        for (int64_t i = 0; i < n; ++i) {
            out[i] = low;
        }
        return;
    }
    const double width = (double)high - (double)low;
    const float last = nextafterf(high, low);
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t position = offset + (uint64_t)i;
        uint32_t words[4];
        philox_words(seed, position / 4, words);
        /* 24 high bits as an exact fraction in [0, 1) (random.cpp:56-60). */
        const double u = (double)(words[position % 4] >> 8) * 0x1p-24;
        const float value = (float)((double)low + width * u);
        const float above = low < value ? value : low; /* max(low, value) */
        out[i] = above < last ? above : last;          /* min(last, above) */
    }
}

/* Box-Muller on midpoint uniforms: words (0,1) give positions 0 and 1 of a block (cosine,
 * sine), words (2,3) positions 2 and 3 (random.cpp:65-96). */
void orc_normal_f32(float* out, int64_t n, float mean, float stddev, uint64_t seed,
                    uint64_t offset) {
    if (stddev == 0.0f) {
        for (int64_t i = 0; i < n; ++i) {
            out[i] = mean;
        }
        return;
    }
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t position = offset + (uint64_t)i;
        uint32_t words[4];
        philox_words(seed, position / 4, words);
        const unsigned pair = (unsigned)((position % 4) / 2);
        const unsigned lane = (unsigned)(position % 2);
        const double u1 = ((double)words[2 * pair] + 0.5) * 0x1p-32;
        const double u2 = ((double)words[2 * pair + 1] + 0.5) * 0x1p-32;
        const double radius = sqrt(-2.0 * log(u1));
        const double angle = 6.283185307179586476925286766559 * u2;
        const double z = lane == 0 ? radius * cos(angle) : radius * sin(angle);
        out[i] = (float)((double)mean + (double)stddev * z);
    }
}

/* ---- GEMM ---------------------------------------------------------------------------------- */

enum { ROWS_PER_TASK = 4, COLS_PER_TASK = 256 };

void orc_sgemm_packed(int64_t m, int64_t n, int64_t k, const float* a, int64_t rsa, int64_t csa,
                      const float* b, int64_t rsb, int64_t csb, float* c, int64_t ldc, int64_t kc) {
    if (m == 0 || n == 0) {
        return;
    }
    if (k == 0) {
        for (int64_t i = 0; i < m; ++i) {
            memset(c + i * ldc, 0, (size_t)n * sizeof(float));
        }
        return;
    }
    if (kc <= 0 || kc > k || (m == 1 && csb == 1)) {
        kc = k;
    }
    /* B gathered into a dense [k][n] copy: data movement only, the arithmetic is unchanged. */
    float* bp = (float*)malloc((size_t)k * (size_t)n * sizeof(float));
#pragma omp parallel for schedule(static) if (k * n > 65536)
    for (int64_t p = 0; p < k; ++p) {
        for (int64_t j = 0; j < n; ++j) {
            bp[p * n + j] = b[p * rsb + j * csb];
        }
    }
    const int64_t row_tasks = (m + ROWS_PER_TASK - 1) / ROWS_PER_TASK;
    const int64_t col_tasks = (n + COLS_PER_TASK - 1) / COLS_PER_TASK;
#pragma omp parallel for collapse(2) schedule(dynamic) if (m * n * k > 262144)
    for (int64_t rt = 0; rt < row_tasks; ++rt) {
        for (int64_t ct = 0; ct < col_tasks; ++ct) {
            const int64_t i0 = rt * ROWS_PER_TASK;
            const int64_t j0 = ct * COLS_PER_TASK;
            const int64_t rows = m - i0 < ROWS_PER_TASK ? m - i0 : ROWS_PER_TASK;
            const int64_t cols = n - j0 < COLS_PER_TASK ? n - j0 : COLS_PER_TASK;
            float total[ROWS_PER_TASK][COLS_PER_TASK];
            float block[ROWS_PER_TASK][COLS_PER_TASK];
            for (int64_t pc = 0; pc < k; pc += kc) {
                const int64_t depth = k - pc < kc ? k - pc : kc;
                for (int64_t r = 0; r < rows; ++r) {
                    for (int64_t j = 0; j < cols; ++j) {
                        block[r][j] = 0.0f;
                    }
                }
                /* One FMA chain per entry, in increasing p (the micro-kernel's depth loop,
                 * gemm_packed.cpp:335-369). */
                for (int64_t p = pc; p < pc + depth; ++p) {
                    const float* brow = bp + p * n + j0;
                    for (int64_t r = 0; r < rows; ++r) {
                        const float ar = a[(i0 + r) * rsa + p * csa];
                        for (int64_t j = 0; j < cols; ++j) {
                            block[r][j] = fmaf(ar, brow[j], block[r][j]);
                        }
                    }
                }
                /* Stored at the first depth block, added to at the rest (gemm_packed.cpp:
                 * 371-377, compute_block's accumulate flag at 1486). */
                for (int64_t r = 0; r < rows; ++r) {
                    for (int64_t j = 0; j < cols; ++j) {
                        total[r][j] = pc == 0 ? block[r][j] : total[r][j] + block[r][j];
                    }
                }
            }
            for (int64_t r = 0; r < rows; ++r) {
                memcpy(c + (i0 + r) * ldc + j0, total[r], (size_t)cols * sizeof(float));
            }
        }
    }
    free(bp);
}

void orc_axpby_f32(float* out, const float* x, float alpha, const float* y0, float beta,
                   int64_t n) {
    const int second = y0 != NULL && beta != 0.0f;
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; ++i) {
        float value = x[i];
        if (alpha != 1.0f) {
            value = alpha * value;
        }
        if (second) {
            const float scaled = beta * y0[i];
            value = value + scaled;
        }
        out[i] = value;
    }
}

void orc_add_f32(const float* a, const float* b, float* out, int64_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; ++i) {
        out[i] = a[i] + b[i];
    }
}

void orc_sub_f32(const float* a, const float* b, float* out, int64_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; ++i) {
        out[i] = a[i] - b[i];
    }
}

float orc_dot_f32(const float* x, const float* y, int64_t n) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        sum += (double)x[i] * (double)y[i];
    }
    return (float)sum;
}

void orc_mul_f32(const float* a, const float* b, float* out, int64_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; ++i) {
        out[i] = a[i] * b[i];
    }
}

/* ---- GEMV ---------------------------------------------------------------------------------- */

void orc_matvec_f32(const float* a, const float* x, float* y, int64_t m, int64_t k) {
#pragma omp parallel for schedule(static) if (m * k > 262144)
    for (int64_t i = 0; i < m; ++i) {
        double sum = 0.0;
        for (int64_t j = 0; j < k; ++j) {
            sum += (double)a[i * k + j] * (double)x[j];
        }
        y[i] = (float)sum;
    }
}

void orc_gemv_f32(const float* a, const float* x, float* y, int64_t rows, int64_t cols,
                  float alpha, float beta, const float* y0, int trans) {
    const int64_t outputs = trans ? cols : rows;
    const int64_t inputs = trans ? rows : cols;
    if (!trans) {
#pragma omp parallel for schedule(static) if (rows * cols > 262144)
        for (int64_t i = 0; i < outputs; ++i) {
            double sum = 0.0;
            for (int64_t j = 0; j < inputs; ++j) {
                sum += (double)a[i * cols + j] * (double)x[j];
            }
            const double tail = beta == 0.0f ? 0.0 : (double)(beta * y0[i]);
            y[i] = (float)((double)alpha * sum + tail);
        }
        return;
    }
    /* Transposed: the same per-output sum in increasing row index (blas.cpp:72-76), computed
     * a row at a time so the matrix is read in order. */
    double* sums = (double*)calloc((size_t)outputs, sizeof(double));
    const int64_t chunk = 1024;
#pragma omp parallel for schedule(static) if (rows * cols > 262144)
    for (int64_t c0 = 0; c0 < outputs; c0 += chunk) {
        const int64_t c1 = c0 + chunk < outputs ? c0 + chunk : outputs;
        for (int64_t j = 0; j < inputs; ++j) {
            const double xj = (double)x[j];
            const float* row = a + j * cols;
            for (int64_t i = c0; i < c1; ++i) {
                sums[i] += (double)row[i] * xj;
            }
        }
    }
    for (int64_t i = 0; i < outputs; ++i) {
        const double tail = beta == 0.0f ? 0.0 : (double)(beta * y0[i]);
        y[i] = (float)((double)alpha * sums[i] + tail);
    }
    free(sums);
}

/* ---- elementwise ---------------------------------------------------------------------------- */

void orc_bias_add_f32(const float* x, const float* bias, float* out, int64_t n, int64_t features) {
    const int64_t rows = features == 0 ? 0 : n / features;
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t j = 0; j < features; ++j) {
            out[r * features + j] = x[r * features + j] + bias[j];
        }
    }
}

/* exp(-|v|) form of the logistic function: no overflow and no cancellation in either tail
 * (elementwise.cpp:24-27). */
static double stable_sigmoid(double value) {
    const double z = exp(-fabs(value));
    return value < 0.0 ? z / (1.0 + z) : 1.0 / (1.0 + z);
}

static float gelu_one(float value, int approximate) {
    if (isinf(value)) {
        return value < 0.0f ? -0.0f : value;
    }
    const double v = (double)value;
    if (approximate) {
        /* v * sigmoid(2u) == v * (1 + tanh(u)) / 2 (elementwise.cpp:176-184). */
        const double u = 0.79788456080286535588 * v * (1.0 + 0.044715 * v * v);
        return (float)(v * stable_sigmoid(2.0 * u));
    }
    return (float)(0.5 * v * erfc(-v * 0.70710678118654752440));
}

void orc_gelu_f32(const float* x, float* out, int64_t n, int approximate) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; ++i) {
        out[i] = gelu_one(x[i], approximate);
    }
}

void orc_where_f32(const uint8_t* cond, const float* x, const float* y, float* out, int64_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; ++i) {
        out[i] = cond[i] != 0 ? x[i] : y[i];
    }
}

/* ---- softmax, argmax ------------------------------------------------------------------------ */

void orc_softmax_f32(const float* x, float* out, int64_t outer, int64_t length, int64_t inner) {
    const int64_t lines = outer * inner;
#pragma omp parallel for schedule(static) if (lines * length > 65536)
    for (int64_t line = 0; line < lines; ++line) {
        const int64_t base = (line / inner) * length * inner + line % inner;
        const float* in = x + base;
        float* dst = out + base;
        float maximum = -INFINITY;
        for (int64_t j = 0; j < length; ++j) {
            const float value = in[j * inner];
            if (isnan(value) || value > maximum) {
                maximum = value;
                if (isnan(value)) {
                    break; /* a NaN poisons the line (softmax.cpp:22-31) */
                }
            }
        }
        if (maximum == -INFINITY) {
            for (int64_t j = 0; j < length; ++j) {
                dst[j * inner] = 0.0f;
            }
            continue;
        }
        double sum = 0.0;
        for (int64_t j = 0; j < length; ++j) {
            const float e = expf(in[j * inner] - maximum);
            dst[j * inner] = e;
            sum += (double)e;
        }
        const float scale = (float)(1.0 / sum);
        for (int64_t j = 0; j < length; ++j) {
            dst[j * inner] *= scale;
        }
    }
}

void orc_argmax_f32(const float* x, int64_t* out, int64_t rows, int64_t width) {
#pragma omp parallel for schedule(static) if (rows * width > 262144)
    for (int64_t r = 0; r < rows; ++r) {
        const float* values = x + r * width;
        int64_t best = 0;
        for (int64_t i = 1; i < width && !isnan(values[best]); ++i) {
            if (isnan(values[i]) || values[i] > values[best]) {
                best = i;
            }
        }
        out[r] = best;
    }
}

/* ---- double-precision product with magnitudes ------------------------------------------------ */

void orc_matmul_f64(int64_t m, int64_t n, int64_t k, const float* a, int64_t rsa, int64_t csa,
                    const float* b, int64_t rsb, int64_t csb, double* value, double* magnitude) {
#pragma omp parallel for schedule(dynamic, 4) if (m * n * k > 262144)
    for (int64_t i = 0; i < m; ++i) {
        for (int64_t j = 0; j < n; ++j) {
            double sum = 0.0, scale = 0.0;
            for (int64_t p = 0; p < k; ++p) {
                const double product = (double)a[i * rsa + p * csa] * (double)b[p * rsb + j * csb];
                sum += product;
                scale += fabs(product);
            }
            value[i * n + j] = sum;
            if (magnitude != NULL) {
                magnitude[i * n + j] = scale;
            }
        }
    }
}
