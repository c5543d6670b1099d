// The reference's own device-generic test cases for the path, run on every device (the rocm one
// through the HIP kernels): gemm_strided_batched's API table and error list
// (tests/ops/gemm_batched_test.cpp:201-317), matvec's public checks
// (tests/ops/matvec_test.cpp:74-105), matmul's remaining cases (tests/ops/matmul_test.cpp:207-300)
// and argmax's public checks (tests/ops/argmax_test.cpp:54-76). Inputs are the reference tests'
// quarter-integer generator, so every product sums exactly and results are compared bit for bit
// with a double-precision reference. Where the reference expects "no GPU kernel yet" for the
// batched GEMM (gemm_batched_test.cpp:306-317), the rocm device now has one and is checked for
// results instead.
#include "core/dispatcher.hpp"
#include "oracle_cpu.hpp"
#include "test_util.hpp"

#include <string>
#include <vector>

using namespace mensurflow;

namespace {

using Dims = std::vector<std::int64_t>;

std::int64_t count(const Dims& d) {
    std::int64_t n = 1;
    for (std::int64_t v : d) {
        n *= v;
    }
    return n;
}

// Row-major offset in a tensor of shape `shape` (right-aligned against `index`, size-1 dimensions
// broadcast) of the batch index `index`, in units of the last two dimensions' size.
std::int64_t batch_offset(const Dims& shape, const Dims& index) {
    const std::size_t nb = shape.size() >= 2 ? shape.size() - 2 : 0;
    std::int64_t off = 0;
    for (std::size_t d = 0; d < nb; ++d) {
        const std::size_t id = index.size() - nb + d;
        off = off * shape[d] + (shape[d] == 1 ? 0 : index[id]);
    }
    return off;
}

struct ApiCase {
    const char* name;
    Dims a_shape, b_shape;
    bool transpose_a, transpose_b;
    float alpha;
    Dims c_shape;
    float beta;
    Dims out_shape;
};

// gemm_batched_test.cpp:201-221.
const ApiCase api_cases[] = {
    {"plain batch", {3, 4, 5}, {3, 5, 2}, false, false, 1.0f, {}, 0.0f, {3, 4, 2}},
    {"shared right-hand side", {4, 3, 5}, {5, 2}, false, false, 1.0f, {}, 0.0f, {4, 3, 2}},
    {"shared left-hand side", {3, 5}, {4, 5, 2}, false, false, 1.0f, {}, 0.0f, {4, 3, 2}},
    {"broadcast batch dims", {2, 1, 3, 4}, {5, 4, 6}, false, false, 1.0f, {}, 0.0f, {2, 5, 3, 6}},
    {"plain matrices", {7, 9}, {9, 4}, false, false, 1.0f, {}, 0.0f, {7, 4}},
    {"transpose a", {2, 5, 3}, {2, 5, 4}, true, false, 1.0f, {}, 0.0f, {2, 3, 4}},
    {"transpose b", {2, 3, 5}, {2, 4, 5}, false, true, 1.0f, {}, 0.0f, {2, 3, 4}},
    {"transpose both", {2, 5, 3}, {1, 4, 5}, true, true, 1.0f, {}, 0.0f, {2, 3, 4}},
    {"alpha only", {2, 3, 4}, {2, 4, 5}, false, false, -1.5f, {}, 0.0f, {2, 3, 5}},
    {"alpha and full c", {2, 3, 4}, {2, 4, 5}, false, false, 2.0f, {2, 3, 5}, 0.5f, {2, 3, 5}},
    {"c broadcast over batch", {4, 3, 4}, {4, 5}, false, false, 1.0f, {3, 5}, -1.0f, {4, 3, 5}},
    {"c as a row", {2, 3, 4}, {2, 4, 5}, false, false, 1.0f, {5}, 1.0f, {2, 3, 5}},
    {"c given, beta 0", {2, 3, 4}, {2, 4, 5}, false, false, 1.0f, {2, 3, 5}, 0.0f, {2, 3, 5}},
    {"empty batch", {0, 3, 4}, {0, 4, 5}, false, false, 1.0f, {}, 0.0f, {0, 3, 5}},
    {"empty rows", {2, 0, 4}, {2, 4, 5}, false, false, 1.0f, {}, 0.0f, {2, 0, 5}},
    {"k is 0", {2, 3, 0}, {2, 0, 5}, false, false, 1.0f, {}, 0.0f, {2, 3, 5}},
    {"k is 0 with c", {2, 3, 0}, {2, 0, 5}, false, false, 1.0f, {2, 3, 5}, 3.0f, {2, 3, 5}},
    {"many small", {100, 2, 3}, {100, 3, 2}, false, false, 1.0f, {}, 0.0f, {100, 2, 2}},
    {"larger", {3, 70, 90}, {3, 90, 60}, false, false, 1.0f, {}, 0.0f, {3, 70, 60}},
};

// alpha * op(a) op(b) + beta * c over broadcast batches, in double: exact for these inputs.
std::vector<float> batched_exact(const ApiCase& t, const std::vector<float>& a,
                                 const std::vector<float>& b, const std::vector<float>& c) {
    const Dims& out = t.out_shape;
    const std::size_t nd = out.size();
    const std::int64_t m = out[nd - 2], n = out[nd - 1];
    const Dims& as = t.a_shape;
    const Dims& bs = t.b_shape;
    const std::int64_t k = t.transpose_a ? as[as.size() - 2] : as[as.size() - 1];
    const std::int64_t a_rows = as[as.size() - 2], a_cols = as[as.size() - 1];
    const std::int64_t b_rows = bs[bs.size() - 2], b_cols = bs[bs.size() - 1];
    Dims batch(out.begin(), out.end() - 2);
    std::vector<float> result(static_cast<std::size_t>(count(out)));
    const std::int64_t batches = count(batch);
    for (std::int64_t flat = 0; flat < batches; ++flat) {
        Dims index(batch.size());
        std::int64_t rest = flat;
        for (std::size_t d = batch.size(); d-- > 0;) {
            index[d] = rest % batch[d];
            rest /= batch[d];
        }
        const std::int64_t ao = batch_offset(as, index) * a_rows * a_cols;
        const std::int64_t bo = batch_offset(bs, index) * b_rows * b_cols;
        for (std::int64_t i = 0; i < m; ++i) {
            for (std::int64_t j = 0; j < n; ++j) {
                double sum = 0.0;
                for (std::int64_t p = 0; p < k; ++p) {
                    const double av = t.transpose_a ? a[static_cast<std::size_t>(ao + p * a_cols + i)]
                                                    : a[static_cast<std::size_t>(ao + i * a_cols + p)];
                    const double bv = t.transpose_b ? b[static_cast<std::size_t>(bo + j * b_cols + p)]
                                                    : b[static_cast<std::size_t>(bo + p * b_cols + j)];
                    sum += av * bv;
                }
                double v = static_cast<double>(t.alpha) * sum;
                if (!t.c_shape.empty() && t.beta != 0.0f) {
                    // c broadcast to the output: right-aligned, size-1 dimensions repeat.
                    const Dims& cs = t.c_shape;
                    Dims full = index;
                    full.push_back(i);
                    full.push_back(j);
                    std::int64_t co = 0;
                    for (std::size_t d = 0; d < cs.size(); ++d) {
                        const std::size_t id = full.size() - cs.size() + d;
                        co = co * cs[d] + (cs[d] == 1 ? 0 : full[id]);
                    }
                    v += static_cast<double>(t.beta) * c[static_cast<std::size_t>(co)];
                }
                result[static_cast<std::size_t>(flat * m * n + i * n + j)] = static_cast<float>(v);
            }
        }
    }
    return result;
}

void test_batched_api(Device device) {
    const Execution on = test::execution_on(device);
    for (const ApiCase& t : api_cases) {
        const auto a = test::quarter_input(count(t.a_shape), 4);
        const auto b = test::quarter_input(count(t.b_shape), 5);
        const auto c = test::quarter_input(count(t.c_shape), 6);
        const bool has_c = !t.c_shape.empty();
        const Tensor ta = Tensor::from_vector(a, t.a_shape, device);
        const Tensor tb = Tensor::from_vector(b, t.b_shape, device);
        const Tensor tc = has_c ? Tensor::from_vector(c, t.c_shape, device) : Tensor();
        const auto want = batched_exact(t, a, b, c);
        for (const Execution execution : {Execution::Auto, on}) {
            const std::string what = std::string(t.name) + " on " + to_string(device) +
                                     (execution == Execution::Auto ? " (auto)" : "");
            const Tensor out = gemm_strided_batched(ta, tb, t.alpha, has_c ? &tc : nullptr, t.beta,
                                                    t.transpose_a, t.transpose_b, execution);
            test::require(out.shape() == t.out_shape, what + ": shape " + to_string(out.shape()));
            test::require(out.device() == device, what + ": result on the wrong device");
            test::require(out.is_contiguous(), what + ": result not contiguous");
            test::require(test::same_bits(out.to_vector<float>(), want), what + ": values");
        }
    }
}

void test_batched_errors(Device device) {
    const Tensor a = Tensor::ones({2, 3, 4}, DType::F32, device);
    const Tensor b = Tensor::ones({2, 4, 5}, DType::F32, device);
    const Execution on = test::execution_on(device);
    using E = std::invalid_argument;
    auto ones = [&](Dims d, DType t = DType::F32) { return Tensor::ones(d, t, device); };
    test::require_throws<E>([&] { gemm_strided_batched(ones({4}), b, 1, nullptr, 0, false, false, on); }, "1-D a");
    test::require_throws<E>([&] { gemm_strided_batched(a, ones({4}), 1, nullptr, 0, false, false, on); }, "1-D b");
    test::require_throws<E>([&] { gemm_strided_batched(Tensor(), b, 1, nullptr, 0, false, false, on); }, "undefined a");
    test::require_throws<E>([&] { gemm_strided_batched(a, ones({2, 3, 5}), 1, nullptr, 0, false, false, on); },
                            "inner dimensions differ");
    test::require_throws<E>([&] { gemm_strided_batched(a, ones({3, 4, 5}), 1, nullptr, 0, false, false, on); },
                            "batch 2 and 3 do not broadcast");
    test::require_throws<E>([&] { gemm_strided_batched(a, b, 1.0f, nullptr, 1.0f, false, false, on); },
                            "beta without c");
    const Tensor bad_c = ones({4, 5});
    test::require_throws<E>([&] { gemm_strided_batched(a, b, 1.0f, &bad_c, 1.0f, false, false, on); },
                            "c that does not broadcast");
    const Tensor big_c = ones({1, 2, 3, 5});
    test::require_throws<E>([&] { gemm_strided_batched(a, b, 1.0f, &big_c, 1.0f, false, false, on); },
                            "c with more dimensions than the result");
    test::require_throws<E>([&] { gemm_strided_batched(a, ones({2, 4, 5}, DType::I32), 1, nullptr, 0, false, false, on); },
                            "dtypes differ");
    if (device.type != DeviceType::CPU) {
        test::require_throws<E>([&] { gemm_strided_batched(a, b.to(Device{}), 1, nullptr, 0, false, false, on); },
                                "mixed devices");
    }
}

void test_matvec_public(Device device) {
    const Execution on = test::execution_on(device);
    const std::int64_t m = 4, k = 3;
    const auto a = test::quarter_input(m * k, 41);
    const auto x = test::quarter_input(k, 42);
    auto exact_mv = [](const std::vector<float>& av, const std::vector<float>& xv, std::int64_t rows,
                       std::int64_t cols) {
        std::vector<float> y(static_cast<std::size_t>(rows));
        for (std::int64_t i = 0; i < rows; ++i) {
            double s = 0.0;
            for (std::int64_t j = 0; j < cols; ++j) {
                s += static_cast<double>(av[static_cast<std::size_t>(i * cols + j)]) *
                     xv[static_cast<std::size_t>(j)];
            }
            y[static_cast<std::size_t>(i)] = static_cast<float>(s);
        }
        return y;
    };
    const Tensor result =
        matvec(Tensor::from_vector(a, {m, k}, device), Tensor::from_vector(x, {k}, device), on);
    test::require(result.shape() == (Shape{m}) && result.is_contiguous(), "matvec output shape");
    test::require(test::same_bits(result.to_vector<float>(), exact_mv(a, x, m, k)), "public matvec");
    // Rows 1 and 3 of a [6, k] matrix and every other element of a vector: strided views.
    const Tensor stored_a = Tensor::from_vector(test::quarter_input(6 * k, 43), {6, k}, device);
    const Tensor view_a = stored_a.slice(0, 1, 5, 2);
    const Tensor stored_x = Tensor::from_vector(test::quarter_input(2 * k, 44), {2 * k}, device);
    const Tensor view_x = stored_x.slice(0, 0, 2 * k, 2);
    test::require(!view_a.is_contiguous() && !view_x.is_contiguous(), "matvec views");
    test::require(test::same_bits(matvec(view_a, view_x, on).to_vector<float>(),
                                  exact_mv(view_a.to_vector<float>(), view_x.to_vector<float>(), 2, k)),
                  "matvec strided inputs");
    test::require_throws<std::invalid_argument>(
        [&] {
            matvec(Tensor::from_vector(a, {m, k}, device),
                   Tensor::from_vector(test::quarter_input(k + 1, 45), {k + 1}, device), on);
        },
        "matvec mismatched dimensions");
    test::require_throws<detail::NotImplemented>(
        [&] { matvec(Tensor::empty({m, k}, DType::I32, device), Tensor::empty({k}, DType::I32, device), on); },
        "matvec unsupported dtype");
}

void test_matmul_remaining(Device device) {
    const Execution on = test::execution_on(device);
    // 300^3 in the contiguous and transposed layouts (matmul_test.cpp:207-230).
    const std::int64_t s = 300;
    const auto av = test::quarter_input(s * s, 21);
    const auto bv = test::quarter_input(s * s, 22);
    std::vector<float> want(static_cast<std::size_t>(s * s));
    for (std::int64_t i = 0; i < s; ++i) {
        for (std::int64_t j = 0; j < s; ++j) {
            double sum = 0.0;
            for (std::int64_t p = 0; p < s; ++p) {
                sum += static_cast<double>(av[static_cast<std::size_t>(i * s + p)]) *
                       bv[static_cast<std::size_t>(p * s + j)];
            }
            want[static_cast<std::size_t>(i * s + j)] = static_cast<float>(sum);
        }
    }
    auto transposed = [&](const std::vector<float>& v) {
        std::vector<float> t(v.size());
        for (std::int64_t i = 0; i < s; ++i) {
            for (std::int64_t j = 0; j < s; ++j) {
                t[static_cast<std::size_t>(j * s + i)] = v[static_cast<std::size_t>(i * s + j)];
            }
        }
        return Tensor::from_vector(t, {s, s}, device).transpose(0, 1);
    };
    for (int ka : {0, 2}) {
        for (int kb : {0, 2}) {
            const Tensor a = ka == 0 ? Tensor::from_vector(av, {s, s}, device) : transposed(av);
            const Tensor b = kb == 0 ? Tensor::from_vector(bv, {s, s}, device) : transposed(bv);
            test::require(test::same_bits(matmul(a, b, on).to_vector<float>(), want),
                          "300^3 A" + std::to_string(ka) + " B" + std::to_string(kb));
        }
    }
    // Empty n, and the remaining errors (matmul_test.cpp:269-300).
    const Tensor none_n = matmul(Tensor::empty({2, 5}, DType::F32, device),
                                 Tensor::empty({5, 0}, DType::F32, device), on);
    test::require(none_n.shape() == (Shape{2, 0}) && none_n.numel() == 0, "n == 0");
    const Tensor m32 = Tensor::from_vector(std::vector<float>{1, 2, 3, 4, 5, 6}, {3, 2}, device);
    const Tensor m23 = Tensor::from_vector(std::vector<float>{1, 2, 3, 4, 5, 6}, {2, 3}, device);
    const Tensor vec = Tensor::from_vector(std::vector<float>{1, 2, 3}, {3}, device);
    const Tensor ints = Tensor::from_vector(std::vector<std::int32_t>{1, 2, 3, 4, 5, 6}, {2, 3}, device);
    test::require_throws<std::invalid_argument>([&] { matmul(m23, vec, on); }, "1-D right");
    test::require_throws<std::invalid_argument>([&] { matmul(Tensor(), m32, on); }, "undefined");
    test::require_throws<std::invalid_argument>([&] { matmul(ints, m32, on); }, "dtype mismatch");
    test::require_throws<std::runtime_error>([&] { matmul(ints, ints.transpose(0, 1), on); },
                                             "unsupported dtype");
}

void test_argmax_public(Device device) {
    const Execution on = test::execution_on(device);
    const Tensor input = Tensor::from_vector(std::vector<float>{1, 9, 3, 7, 7, 2}, {2, 3}, device);
    const Tensor result = argmax(input, -1, on);
    test::require(result.dtype() == DType::I64 && result.shape() == (Shape{2}),
                  "argmax output dtype and shape");
    test::require(result.to_vector<std::int64_t>() == (std::vector<std::int64_t>{1, 0}),
                  "public argmax");
    const Tensor stored = Tensor::from_vector(std::vector<float>{1, 9, 3, 7, 7, 2, 8, 4}, {2, 4}, device);
    test::require(argmax(stored.slice(1, 0, 4, 2), 1, on).to_vector<std::int64_t>() ==
                      (std::vector<std::int64_t>{1, 1}),
                  "strided argmax");
    test::require_throws<std::invalid_argument>([&] { argmax(input, 0, on); }, "non-last axis");
    test::require_throws<std::invalid_argument>(
        [&] { argmax(Tensor::empty({2, 0}, DType::F32, device), -1, on); }, "empty axis");
    test::require_throws<std::invalid_argument>([&] { argmax(Tensor(), -1, on); }, "undefined input");
}

} // namespace

int main(int argc, char** argv) {
    return test::run("reference_cases_test", argc, argv, [] {
        test::register_oracle_cpu_kernels();
        for (Device device : test::devices()) {
            std::cout << "  the reference's test cases on " << to_string(device) << '\n';
            test_batched_api(device);
            test_batched_errors(device);
            test_matvec_public(device);
            test_matmul_remaining(device);
            test_argmax_public(device);
        }
    });
}
