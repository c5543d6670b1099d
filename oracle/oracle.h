/*
 * oracle.h -- CPU restatement of mensurflow's fp32 BLAS hot path, used ONLY as test
 * infrastructure: the checker that tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg compare the HIP kernels against. Nothing in the product (mensurflow_amd/, libmfr_rocm.so)
 * links or calls it.
 *
 * Each function restates the behaviour (not the text) of the reference function it cites, as
 * path:line into bakir004/mensurflow. Every function is pinned by tests/test_oracle.py: golden
 * vectors from the reference's own tests, vectors written by the reference's kernels compiled
 * from their sources (oracle/_ref, tests/golden/ref_vectors.npz), and closed forms. A function
 * without such a check would say "parity unpinned" here; none does.
 */
#ifndef MFR_ORACLE_H
#define MFR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Philox4x32-10 (src/backends/cpu/ops/random/philox.hpp:14-34). */
void orc_philox4x32_10(const uint32_t counter[4], const uint32_t key[2], uint32_t out[4]);

/* uniform_f32 / normal_f32 (src/backends/cpu/ops/random/random.cpp:47-96): counter-based,
 * offset counts output elements. */
void orc_uniform_f32(float* out, int64_t n, float low, float high, uint64_t seed, uint64_t offset);
void orc_normal_f32(float* out, int64_t n, float mean, float stddev, uint64_t seed,
                    uint64_t offset);

/* The packed CPU GEMM's arithmetic (src/backends/cpu/ops/gemm/gemm_packed.cpp:314-378,
 * 980-1090, 1387-1490): C[m,n] (row stride ldc) = A*B where every entry is the sum over depth
 * blocks of `kc` (C stored at the first block, added to at the rest) of an fp32 FMA chain in
 * increasing p starting from 0. kc <= 0 means one block of the whole depth. A one-row product
 * with unit column stride in B uses one block (row_times_matrix, gemm_packed.cpp:1125-1189).
 * k == 0 gives zeros. */
void orc_sgemm_packed(int64_t m, int64_t n, int64_t k, const float* a, int64_t rsa, int64_t csa,
                      const float* b, int64_t rsb, int64_t csb, float* c, int64_t ldc, int64_t kc);

/* out = fl(fl(alpha*x) + fl(beta*y0)), with the reference's skips: alpha == 1 leaves x as is,
 * y0 == NULL or beta == 0 drops the second term. The alpha/beta passes of mensurflow::gemm
 * (src/ops/blas.cpp:246-257) and of the batched finish pass (gemm_batched.cpp:12-28). */
void orc_axpby_f32(float* out, const float* x, float alpha, const float* y0, float beta, int64_t n);

/* add_f32 / sub_f32 / mul_f32 (src/backends/cpu/ops/elementwise/elementwise.cpp:72-91). */
void orc_add_f32(const float* a, const float* b, float* out, int64_t n);
void orc_sub_f32(const float* a, const float* b, float* out, int64_t n);
void orc_mul_f32(const float* a, const float* b, float* out, int64_t n);

/* dot_f32 (src/backends/cpu/ops/blas/blas.cpp:14-21): the products in double (exact), summed in
 * double in increasing index order (the reference's single-thread order), rounded once. */
float orc_dot_f32(const float* x, const float* y, int64_t n);

/* matvec_f32 / gemv_f32 (src/backends/cpu/ops/blas/blas.cpp:55-79): double accumulation in
 * increasing index, one rounding. */
void orc_matvec_f32(const float* a, const float* x, float* y, int64_t m, int64_t k);
void orc_gemv_f32(const float* a, const float* x, float* y, int64_t rows, int64_t cols,
                  float alpha, float beta, const float* y0, int trans);

/* bias_add_f32, gelu_f32, where_f32 (src/backends/cpu/ops/elementwise/elementwise.cpp:24-27,
 * 64-70, 128-137, 173-194). */
void orc_bias_add_f32(const float* x, const float* bias, float* out, int64_t n, int64_t features);
void orc_gelu_f32(const float* x, float* out, int64_t n, int approximate);
void orc_where_f32(const uint8_t* cond, const float* x, const float* y, float* out, int64_t n);

/* softmax_f32 (src/backends/cpu/ops/softmax/softmax.cpp:13-49). */
void orc_softmax_f32(const float* x, float* out, int64_t outer, int64_t length, int64_t inner);

/* argmax_f32 (src/backends/cpu/ops/reduction/reduction.cpp:284-296). */
void orc_argmax_f32(const float* x, int64_t* out, int64_t rows, int64_t width);

/* Double-precision product with per-entry magnitude sum_p |a*b| (the scale the reference's
 * tests measure fp32 rounding against, tests/reference/blas.hpp:38-59). Strided like
 * orc_sgemm_packed; value and magnitude are contiguous [m,n]. magnitude may be NULL. */
void orc_matmul_f64(int64_t m, int64_t n, int64_t k, const float* a, int64_t rsa, int64_t csa,
                    const float* b, int64_t rsb, int64_t csb, double* value, double* magnitude);

/* Threads used by the OpenMP loops above (0 = OpenMP default). Returns the previous setting. */
int orc_set_threads(int threads);

#ifdef __cplusplus
}
#endif

#endif /* MFR_ORACLE_H */
