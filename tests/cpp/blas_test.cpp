// BLAS ops through the public API on every device (the cases of the reference's
// tests/ops/matmul_test.cpp, p0_extended_test.cpp, matvec_test.cpp and gemm_batched_test.cpp):
// known values, sizes around tile edges, strided layouts, alpha/beta, broadcast batches, empty
// inputs and errors. Quarter-integer inputs make every fp32 sum exact, so CPU and GPU results
// must agree in every bit with the exact product.
#include "core/dispatcher.hpp"
#include "oracle.h"
#include "oracle_cpu.hpp"
#include "reference_math.hpp"
#include "test_util.hpp"

using namespace mensurflow;

namespace {

struct Shape3 {
    std::int64_t m, n, k;
};

const Shape3 kShapes[] = {{1, 1, 1},     {1, 5, 1},     {5, 1, 3},      {3, 5, 7},
                          {16, 16, 16},  {17, 31, 13},  {64, 64, 64},   {65, 129, 130},
                          {100, 300, 50}, {200, 100, 300}, {2, 1000, 3}, {1000, 2, 3},
                          {257, 129, 257}, {129, 255, 33}};

std::vector<float> exact(const std::vector<float>& a, const std::vector<float>& b, std::int64_t m,
                         std::int64_t n, std::int64_t k) {
    const auto r = reference::matmul(a, b, m, n, k);
    std::vector<float> out(r.value.size());
    for (std::size_t i = 0; i < out.size(); ++i) {
        out[i] = static_cast<float>(r.value[i]);
    }
    return out;
}

// The reference's layouts (tests/ops/matmul_test.cpp:189-214): 0 contiguous, 1 sliced out of a
// wider matrix, 2 transposed storage, 3 transposed and sliced. Shape {rows, cols} always.
Tensor make_view(const std::vector<float>& values, std::int64_t rows, std::int64_t cols, int kind,
                 Device device) {
    auto stored = [&](std::int64_t sr, std::int64_t sc, std::int64_t r0, std::int64_t c0,
                      bool transposed) {
        std::vector<float> s(static_cast<std::size_t>(sr * sc), -77.0f);
        for (std::int64_t i = 0; i < rows; ++i) {
            for (std::int64_t j = 0; j < cols; ++j) {
                const std::int64_t r = transposed ? r0 + j : r0 + i;
                const std::int64_t c = transposed ? c0 + i : c0 + j;
                s[static_cast<std::size_t>(r * sc + c)] = values[static_cast<std::size_t>(i * cols + j)];
            }
        }
        return Tensor::from_vector(s, {sr, sc}, device);
    };
    switch (kind) {
    case 0:
        return Tensor::from_vector(values, {rows, cols}, device);
    case 1:
        return stored(rows + 2, cols + 9, 1, 3, false).slice(0, 1, 1 + rows).slice(1, 3, 3 + cols);
    case 2:
        return stored(cols, rows, 0, 0, true).transpose(0, 1);
    default:
        return stored(cols + 3, rows + 5, 2, 4, true)
            .slice(0, 2, 2 + cols)
            .slice(1, 4, 4 + rows)
            .transpose(0, 1);
    }
}

void test_matmul(Device device) {
    const Execution on = test::execution_on(device);
    const Tensor a = Tensor::from_vector(std::vector<float>{1, 2, 3, 4, 5, 6}, {2, 3}, device);
    const Tensor b = Tensor::from_vector(std::vector<float>{7, 8, 9, 10, 11, 12}, {3, 2}, device);
    const Tensor c = matmul(a, b, on);
    test::require(c.shape() == (Shape{2, 2}) && c.device() == device && c.is_contiguous(),
                  "result shape, device, layout");
    test::require(c.to_vector<float>() == (std::vector<float>{58, 64, 139, 154}), "known values");
    const auto values = test::quarter_input(5 * 7, 3);
    std::vector<float> eye(49, 0.0f);
    for (int i = 0; i < 7; ++i) {
        eye[static_cast<std::size_t>(i * 8)] = 1.0f;
    }
    test::require(matmul(Tensor::from_vector(values, {5, 7}, device),
                         Tensor::from_vector(eye, {7, 7}, device), on)
                          .to_vector<float>() == values,
                  "A x I == A");
    for (const Shape3& s : kShapes) {
        const auto av = test::quarter_input(s.m * s.k, 4);
        const auto bv = test::quarter_input(s.k * s.n, 5);
        const auto got = matmul(Tensor::from_vector(av, {s.m, s.k}, device),
                                Tensor::from_vector(bv, {s.k, s.n}, device), on)
                             .to_vector<float>();
        test::require(test::same_bits(got, exact(av, bv, s.m, s.n, s.k)),
                      "matmul " + std::to_string(s.m) + "x" + std::to_string(s.n) + "x" +
                          std::to_string(s.k));
    }
    for (const Shape3& s : {Shape3{70, 60, 90}, Shape3{130, 200, 150}}) {
        const auto av = test::quarter_input(s.m * s.k, 21);
        const auto bv = test::quarter_input(s.k * s.n, 22);
        const auto want = exact(av, bv, s.m, s.n, s.k);
        for (int ka = 0; ka < 4; ++ka) {
            for (int kb = 0; kb < 4; ++kb) {
                const auto got = matmul(make_view(av, s.m, s.k, ka, device),
                                        make_view(bv, s.k, s.n, kb, device), on)
                                     .to_vector<float>();
                test::require(test::same_bits(got, want),
                              "strided A" + std::to_string(ka) + " B" + std::to_string(kb));
            }
        }
    }
    // Realistic inputs: within the fp32 bar of the exact product.
    const Tensor ua = uniform({300, 1000}, -1.0f, 1.0f, 7, 0);
    const Tensor ub = uniform({1000, 200}, -1.0f, 1.0f, 7, 300000);
    const auto rel = reference::relative_error(
        matmul(ua.to(device), ub.to(device), on).to_vector<float>(),
        reference::matmul(ua.to_vector<float>(), ub.to_vector<float>(), 300, 200, 1000));
    test::require(rel <= 1e-5 * std::sqrt(1000.0), "uniform inputs: relative error " +
                                                      std::to_string(rel));
    // Empty and k == 0.
    const Tensor none_k = matmul(Tensor::empty({3, 0}, DType::F32, device),
                                 Tensor::empty({0, 4}, DType::F32, device), on);
    test::require(none_k.to_vector<float>() == std::vector<float>(12, 0.0f), "k == 0 -> zeros");
    test::require(matmul(Tensor::empty({0, 5}, DType::F32, device),
                         Tensor::empty({5, 2}, DType::F32, device), on)
                          .numel() == 0,
                  "m == 0");
    // Errors.
    test::require_throws<std::invalid_argument>([&] { matmul(a, a, on); }, "inner mismatch");
    test::require_throws<std::invalid_argument>(
        [&] { matmul(Tensor::from_vector(std::vector<float>{1, 2, 3}, {3}, device), b, on); },
        "1-D operand");
    const Tensor ints = Tensor::from_vector(std::vector<std::int32_t>{1, 2, 3, 4}, {2, 2}, device);
    test::require_throws<detail::NotImplemented>([&] { matmul(ints, ints, on); }, "no i32 kernel");
}

void test_gemm(Device device) {
    const Execution on = test::execution_on(device);
    const std::int64_t m = 70, n = 45, k = 96;
    for (bool ta : {false, true}) {
        for (bool tb : {false, true}) {
            const auto av = test::quarter_input(m * k, 31);
            const auto bv = test::quarter_input(k * n, 32);
            const auto cv = test::quarter_input(m * n, 33);
            // stored operands: A is [k,m] when transposed, B is [n,k] when transposed
            std::vector<float> as = av, bs = bv;
            if (ta) {
                for (std::int64_t i = 0; i < m; ++i)
                    for (std::int64_t p = 0; p < k; ++p)
                        as[static_cast<std::size_t>(p * m + i)] = av[static_cast<std::size_t>(i * k + p)];
            }
            if (tb) {
                for (std::int64_t p = 0; p < k; ++p)
                    for (std::int64_t j = 0; j < n; ++j)
                        bs[static_cast<std::size_t>(j * k + p)] = bv[static_cast<std::size_t>(p * n + j)];
            }
            const Tensor A = Tensor::from_vector(as, ta ? Shape{k, m} : Shape{m, k}, device);
            const Tensor B = Tensor::from_vector(bs, tb ? Shape{n, k} : Shape{k, n}, device);
            const Tensor C = Tensor::from_vector(cv, {m, n}, device);
            const auto prod = exact(av, bv, m, n, k);
            std::vector<float> want(prod.size());
            for (std::size_t i = 0; i < want.size(); ++i) {
                want[i] = 1.5f * prod[i] + 0.5f * cv[i];
            }
            const auto got = gemm(A, B, 1.5f, &C, 0.5f, ta, tb, on).to_vector<float>();
            test::require(test::same_bits(got, want),
                          std::string("gemm ta=") + (ta ? "1" : "0") + " tb=" + (tb ? "1" : "0"));
        }
    }
    const Tensor a = Tensor::ones({4, 3}, DType::F32, device);
    const Tensor b = Tensor::ones({3, 2}, DType::F32, device);
    test::require_throws<std::invalid_argument>([&] { gemm(a, b, 1.0f, nullptr, 1.0f, false, false, on); },
                                                "beta requires c");
    const Tensor bad = Tensor::ones({3, 3}, DType::F32, device);
    test::require_throws<std::invalid_argument>([&] { gemm(a, b, 1.0f, &bad, 1.0f, false, false, on); },
                                                "c shape");
    // gemm_epilogue == gelu(bias_add(gemm)) within the fp32 bar
    const Tensor x = normal({64, 300}, 0.0f, 1.0f, 11, 0).to(device);
    const Tensor w = normal({300, 50}, 0.0f, 0.0577f, 12, 0).to(device);
    const Tensor bias = uniform({50}, -0.1f, 0.1f, 13, 0).to(device);
    const auto fused = gemm_epilogue(x, w, &bias, Activation::GeluTanh, 1.0f, nullptr, 0.0f,
                                     false, false, on)
                           .to_vector<float>();
    const auto chain = gelu(bias_add(matmul(x, w, on), bias, on), true, on).to_vector<float>();
    double worst = 0.0;
    for (std::size_t i = 0; i < fused.size(); ++i) {
        worst = std::fmax(worst, std::fabs(static_cast<double>(fused[i]) - chain[i]));
    }
    test::require(worst <= 1e-5, "gemm_epilogue vs chain: " + std::to_string(worst));
}

void test_gemv(Device device) {
    const Execution on = test::execution_on(device);
    const Tensor matrix = Tensor::from_vector(std::vector<float>{1, 2, 3, 4, 5, 6}, {2, 3}, device);
    const Tensor ones3 = Tensor::from_vector(std::vector<float>{1, 1, 1}, {3}, device);
    test::require(gemv(matrix, ones3, 1.0f, nullptr, 0.0f, false, on).to_vector<float>() ==
                      (std::vector<float>{6, 15}),
                  "gemv");
    const Tensor y0 = Tensor::from_vector(std::vector<float>{2, 3}, {2}, device);
    test::require(gemv(matrix, ones3, 2.0f, &y0, 0.5f, false, on).to_vector<float>() ==
                      (std::vector<float>{13, 31.5f}),
                  "gemv alpha beta");
    const Tensor ones2 = Tensor::from_vector(std::vector<float>{1, 1}, {2}, device);
    test::require(gemv(matrix, ones2, 1.0f, nullptr, 0.0f, true, on).to_vector<float>() ==
                      (std::vector<float>{5, 7, 9}),
                  "gemv transpose");
    test::require(matvec(matrix, ones3, on).to_vector<float>() == (std::vector<float>{6, 15}),
                  "matvec");
    // A transposed view goes through contiguous() first.
    test::require(gemv(matrix.transpose(0, 1), ones2, 1.0f, nullptr, 0.0f, false, on)
                          .to_vector<float>() == (std::vector<float>{5, 7, 9}),
                  "gemv of a view");
    test::require(matvec(Tensor::empty({4, 0}, DType::F32, device),
                         Tensor::empty({0}, DType::F32, device), on)
                          .to_vector<float>() == std::vector<float>(4, 0.0f),
                  "matvec k == 0");
    test::require_throws<std::invalid_argument>(
        [&] { gemv(matrix, ones3, 1.0f, nullptr, 1.0f, false, on); }, "beta without y");
}

void test_batched(Device device) {
    const Execution on = test::execution_on(device);
    const auto big = test::quarter_input(6 * 4 * 5, 7);
    const Tensor full = Tensor::from_vector(big, {6, 4, 5}, device);
    const Tensor every_other = full.slice(0, 0, 6, 2); // [3,4,5], batch stride 40
    const Tensor b = Tensor::from_vector(test::quarter_input(3 * 5 * 2, 8), {3, 5, 2}, device);
    test::require(gemm_strided_batched(every_other, b, 1.0f, nullptr, 0.0f, false, false, on)
                          .to_vector<float>() ==
                      gemm_strided_batched(every_other.contiguous(), b, 1.0f, nullptr, 0.0f, false,
                                           false, on)
                          .to_vector<float>(),
                  "sliced batch == packed");
    const Tensor bt = Tensor::from_vector(test::quarter_input(3 * 2 * 5, 9), {3, 2, 5}, device);
    const Tensor packed = every_other.contiguous();
    test::require(gemm_strided_batched(packed, bt.transpose(1, 2), 1.0f, nullptr, 0.0f, false,
                                       false, on)
                          .to_vector<float>() ==
                      gemm_strided_batched(packed, bt, 1.0f, nullptr, 0.0f, false, true, on)
                          .to_vector<float>(),
                  "transposed view == transpose_b");
    const Tensor one = Tensor::from_vector(test::quarter_input(4 * 5, 10), {1, 4, 5}, device);
    const Tensor expanded = one.expand({3, 4, 5});
    test::require(gemm_strided_batched(expanded, b, 1.0f, nullptr, 0.0f, false, false, on)
                          .to_vector<float>() ==
                      gemm_strided_batched(expanded.contiguous(), b, 1.0f, nullptr, 0.0f, false,
                                           false, on)
                          .to_vector<float>(),
                  "expanded batch == packed");
    const Tensor x = Tensor::from_vector(test::quarter_input(8 * 6, 11), {8, 6}, device);
    const Tensor y = Tensor::from_vector(test::quarter_input(6 * 3, 12), {6, 3}, device);
    test::require(gemm_strided_batched(x, y, 1.0f, nullptr, 0.0f, false, false, on)
                          .to_vector<float>() == matmul(x, y, on).to_vector<float>(),
                  "2-D == matmul");
    // 4 batch dimensions with a broadcast one, alpha/beta and c broadcast over the batch.
    const Tensor q = Tensor::from_vector(test::quarter_input(2 * 3 * 2 * 7 * 16, 13),
                                         {2, 3, 2, 7, 16}, device);
    const Tensor kk = Tensor::from_vector(test::quarter_input(3 * 1 * 9 * 16, 14), {3, 1, 9, 16},
                                          device);
    const Tensor c = Tensor::from_vector(test::quarter_input(7 * 9, 15), {7, 9}, device);
    const auto got = gemm_strided_batched(q, kk, 0.25f, &c, 2.0f, false, true, on).to_vector<float>();
    const auto qv = q.to_vector<float>();
    const auto kv = kk.to_vector<float>();
    const auto cv = c.to_vector<float>();
    for (int i0 = 0; i0 < 2; ++i0) {
        for (int i1 = 0; i1 < 3; ++i1) {
            for (int i2 = 0; i2 < 2; ++i2) {
                const std::size_t qm = static_cast<std::size_t>(((i0 * 3 + i1) * 2 + i2) * 7 * 16);
                const std::size_t km = static_cast<std::size_t>(i1 * 9 * 16);
                for (int r = 0; r < 7; ++r) {
                    for (int j = 0; j < 9; ++j) {
                        double s = 0.0;
                        for (int p = 0; p < 16; ++p) {
                            s += static_cast<double>(qv[qm + static_cast<std::size_t>(r * 16 + p)]) *
                                 kv[km + static_cast<std::size_t>(j * 16 + p)];
                        }
                        const float want = 0.25f * static_cast<float>(s) + 2.0f * cv[static_cast<std::size_t>(r * 9 + j)];
                        const std::size_t at = static_cast<std::size_t>(
                            (((i0 * 3 + i1) * 2 + i2) * 7 + r) * 9 + j);
                        test::require(got[at] == want, "4-d broadcast batch at " + std::to_string(at));
                    }
                }
            }
        }
    }
    // k == 0 with c: beta * c.
    const Tensor cc = Tensor::from_vector(std::vector<float>{1, 2, 3, 4}, {2, 2}, device);
    test::require(gemm_strided_batched(Tensor::empty({2, 0}, DType::F32, device),
                                       Tensor::empty({0, 2}, DType::F32, device), 1.0f, &cc, 0.5f,
                                       false, false, on)
                          .to_vector<float>() == (std::vector<float>{0.5f, 1, 1.5f, 2}),
                  "k == 0 gives beta * c");
    test::require_throws<std::invalid_argument>(
        [&] { gemm_strided_batched(Tensor::ones({2, 3, 4}, DType::F32, device),
                                   Tensor::ones({3, 4, 5}, DType::F32, device), 1.0f, nullptr, 0.0f,
                                   false, false, on); },
        "batch 2 and 3 do not broadcast");
}

// dot and sub, the ops the reference's CUDA backend serves besides add and mul (the cases of the
// reference's tests/ops/dot_test.cpp:50-120): known values, empty vectors, a strided slice, an
// offset slice, a broadcast scalar, the errors; the products summed in double, so every device
// gives the oracle's bits here; sub with broadcasting.
void test_dot_and_sub(Device device) {
    const Execution on = test::execution_on(device);
    const Tensor a = Tensor::from_vector(std::vector<float>{1, 2, 3}, {3}, device);
    const Tensor b = Tensor::from_vector(std::vector<float>{4, -5, 6}, {3}, device);
    test::require(dot(a, b, on).item<float>() == 12.0f, "1*4 + 2*-5 + 3*6 = 12");
    test::require(dot(a, a, on).item<float>() == 14.0f, "a . a");
    const Tensor none = Tensor::empty({0}, DType::F32, device);
    const Tensor zero = dot(none, none, on);
    test::require(zero.dim() == 0 && zero.device() == device && zero.item<float>() == 0.0f,
                  "empty dot is 0");
    const std::int64_t n = 100003;
    const Tensor x = normal({n}, 0.0f, 1.0f, 31, 0).to(device);
    const Tensor y = normal({n}, 0.0f, 1.0f, 32, 0).to(device);
    const auto xv = x.to_vector<float>();
    const auto yv = y.to_vector<float>();
    const auto oracle_dot = [](const std::vector<float>& p, const std::vector<float>& q) {
        return orc_dot_f32(p.data(), q.data(), static_cast<std::int64_t>(p.size()));
    };
    const float got = dot(x, y, on).item<float>();
    test::require(got == oracle_dot(xv, yv), "dot of 100003 normals: the oracle's bits");
    std::vector<float> ex, ey;
    for (std::int64_t i = 0; i < n; i += 3) {
        ex.push_back(xv[static_cast<std::size_t>(i)]);
        ey.push_back(yv[static_cast<std::size_t>(i)]);
    }
    test::require(dot(x.slice(0, 0, n, 3), y.slice(0, 0, n, 3), on).item<float>() ==
                      oracle_dot(ex, ey),
                  "strided slice");
    const std::vector<float> ox(xv.begin() + 101, xv.begin() + 90101);
    const std::vector<float> oy(yv.begin() + 101, yv.begin() + 90101);
    test::require(dot(x.slice(0, 101, 90101), y.slice(0, 101, 90101), on).item<float>() ==
                      oracle_dot(ox, oy),
                  "offset slice (unaligned start)");
    const Tensor three = Tensor::from_vector(std::vector<float>{3}, {1}, device).expand({n});
    test::require(dot(three, y, on).item<float>() ==
                      oracle_dot(std::vector<float>(static_cast<std::size_t>(n), 3.0f), yv),
                  "expanded scalar");
    const Tensor v4 = Tensor::from_vector(std::vector<float>{1, 2, 3, 4}, {4}, device);
    const Tensor m = Tensor::from_vector(std::vector<float>{1, 2, 3, 4}, {2, 2}, device);
    test::require_throws<std::invalid_argument>([&] { dot(a, v4, on); }, "dot lengths differ");
    test::require_throws<std::invalid_argument>([&] { dot(m, m, on); }, "dot of a matrix");

    // sub: a - b with a row broadcast over a matrix, and elementwise on a long vector.
    const Tensor mat = Tensor::from_vector(std::vector<float>{1, 2, 3, 4, 5, 6}, {2, 3}, device);
    test::require(sub(mat, a, on).to_vector<float>() == (std::vector<float>{0, 0, 0, 3, 3, 3}),
                  "sub with a broadcast row");
    const auto diff = sub(x, y, on).to_vector<float>();
    std::vector<float> want(xv.size());
    orc_sub_f32(xv.data(), yv.data(), want.data(), n);
    test::require(diff == want, "sub of 100003 normals");
}

} // namespace

int main(int argc, char** argv) {
    return test::run("blas_test", argc, argv, [] {
        test::register_oracle_cpu_kernels();
        for (Device device : test::devices()) {
            std::cout << "  blas on " << to_string(device) << '\n';
            test_matmul(device);
            test_gemm(device);
            test_gemv(device);
            test_batched(device);
            test_dot_and_sub(device);
        }
    });
}
