// ref_shim.cpp -- extern "C" entry points onto the reference's own CPU kernels, compiled from
// the reference sources where they lie (see oracle/Makefile). TEST INFRASTRUCTURE ONLY: the
// resulting oracle/_ref/libmfref.so is used to pin the C restatement in oracle.c and, in
// bench.py, as the CPU baseline. It is never linked into the product.
//
// The reference functions called here are declared in the reference's own headers, included
// from /root/reference/src; this file only forwards plain arguments to them.
#include "backends/cpu/ops/blas/blas.hpp"
#include "backends/cpu/ops/elementwise/elementwise.hpp"
#include "backends/cpu/ops/gemm/gemm_batched.hpp"
#include "backends/cpu/ops/gemm/gemm_packed.hpp"
#include "backends/cpu/ops/random/philox.hpp"
#include "backends/cpu/ops/random/random.hpp"
#include "backends/cpu/ops/reduction/reduction.hpp"
#include "backends/cpu/ops/softmax/softmax.hpp"
#include "backends/cpu/threads.hpp"

#include <cstdint>

namespace cpu = mensurflow::cpu;

extern "C" {

void ref_philox4x32_10(const std::uint32_t counter[4], const std::uint32_t key[2],
                       std::uint32_t out[4]) {
    const cpu::PhiloxCounter r = cpu::philox4x32_10({counter[0], counter[1], counter[2], counter[3]},
                                                    {key[0], key[1]});
    for (int i = 0; i < 4; ++i) {
        out[i] = r[static_cast<std::size_t>(i)];
    }
}

void ref_uniform_f32(float* out, std::int64_t n, float low, float high, std::uint64_t seed,
                     std::uint64_t offset) {
    cpu::uniform_f32(out, n, low, high, seed, offset);
}

void ref_normal_f32(float* out, std::int64_t n, float mean, float stddev, std::uint64_t seed,
                    std::uint64_t offset) {
    cpu::normal_f32(out, n, mean, stddev, seed, offset);
}

int ref_packed_supported() { return cpu::packed_gemm_supported() ? 1 : 0; }

std::int64_t ref_get_kc() { return cpu::packed_gemm_blocking().kc; }

void ref_set_kc(std::int64_t kc) {
    cpu::PackedGemmBlocking blocking = cpu::packed_gemm_blocking();
    blocking.kc = kc;
    cpu::set_packed_gemm_blocking(blocking);
}

void ref_set_threads(int threads) { cpu::set_max_threads(threads); }

int ref_max_threads() { return cpu::max_threads(); }

void ref_matmul_packed(const float* a, std::int64_t rsa, std::int64_t csa, const float* b,
                       std::int64_t rsb, std::int64_t csb, float* c, std::int64_t ldc,
                       std::int64_t m, std::int64_t n, std::int64_t k, int parallel) {
    if (parallel) {
        cpu::matmul_f32_packed_parallel_strided(a, rsa, csa, b, rsb, csb, c, ldc, m, n, k);
    } else {
        cpu::matmul_f32_packed_strided(a, rsa, csa, b, rsb, csb, c, ldc, m, n, k);
    }
}

void ref_matvec_f32(const float* a, const float* x, float* y, std::int64_t m, std::int64_t k) {
    cpu::matvec_f32(a, x, y, m, k);
}

void ref_gemv_f32(const float* a, const float* x, float* y, std::int64_t rows, std::int64_t cols,
                  float alpha, float beta, const float* y0, int trans) {
    cpu::gemv_f32(a, x, y, rows, cols, alpha, beta, y0, trans != 0);
}

// The three kernels mensurflow::gemm's composition dispatches after the product
// (src/ops/blas.cpp:246-257): mul by the 0-d alpha, scal of C0 by beta, add.
void ref_mul_f32(const float* a, const float* b, float* out, std::int64_t n) {
    cpu::mul_f32(a, b, out, n);
}

void ref_scal_f32(float alpha, const float* x, float* out, std::int64_t n) {
    cpu::scal_f32(alpha, x, out, n);
}

void ref_add_f32(const float* a, const float* b, float* out, std::int64_t n) {
    cpu::add_f32(a, b, out, n);
}

// sub (src/backends/cpu/ops/elementwise/elementwise.cpp:79) and dot (blas.cpp:14-21), the two
// ops the reference's CUDA backend registers besides add and mul.
void ref_sub_f32(const float* a, const float* b, float* out, std::int64_t n) {
    cpu::sub_f32(a, b, out, n);
}

float ref_dot_f32(const float* x, const float* y, std::int64_t n) { return cpu::dot_f32(x, y, n); }

// gemm_strided_batched's CPU kernel (gemm_batched.cpp:58-70): packed GEMM per matrix, then the
// finish pass alpha * C + beta * C0 (gemm_batched.cpp:12-28). C and C0 are contiguous
// [batch, m, n]; matrix i of A / B starts at the given element offsets.
void ref_gemm_batched_f32(const float* a, const std::int64_t* a_offsets, std::int64_t rsa,
                          std::int64_t csa, const float* b, const std::int64_t* b_offsets,
                          std::int64_t rsb, std::int64_t csb, float* c, const float* c0,
                          std::int64_t batch, std::int64_t m, std::int64_t n, std::int64_t k,
                          float alpha, float beta) {
    cpu::BatchedGemm g;
    g.a = a;
    g.a_offsets = a_offsets;
    g.rsa = rsa;
    g.csa = csa;
    g.b = b;
    g.b_offsets = b_offsets;
    g.rsb = rsb;
    g.csb = csb;
    g.c = c;
    g.c0 = c0;
    g.batch = batch;
    g.m = m;
    g.n = n;
    g.k = k;
    g.alpha = alpha;
    g.beta = beta;
    cpu::gemm_batched_f32_parallel(g);
}

void ref_bias_add_f32(const float* x, const float* bias, float* out, std::int64_t n,
                      std::int64_t features) {
    cpu::bias_add_f32(x, bias, out, n, features);
}

void ref_gelu_f32(const float* x, float* out, std::int64_t n, int approximate) {
    cpu::gelu_f32(x, out, n, approximate != 0);
}

void ref_where_f32(const std::uint8_t* cond, const float* x, const float* y, float* out,
                   std::int64_t n) {
    cpu::where_f32(cond, x, y, out, n);
}

void ref_softmax_f32(const float* x, float* out, std::int64_t outer, std::int64_t length,
                     std::int64_t inner) {
    cpu::softmax_f32(x, out, outer, length, inner);
}

void ref_argmax_f32(const float* x, std::int64_t* out, std::int64_t rows, std::int64_t width) {
    cpu::argmax_f32(x, out, rows, width);
}

} // extern "C"
