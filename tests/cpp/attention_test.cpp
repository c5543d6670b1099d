// attention, softmax, where, bias_add, gelu and argmax through the public API on every device
// (the cases of the reference's tests/ops/softmax_loss_test.cpp:481-580, activation_test.cpp,
// elementwise_ops_test.cpp:332-413 and the argmax tests), against double references.
#include "core/dispatcher.hpp"
#include "oracle_cpu.hpp"
#include "reference_math.hpp"
#include "test_util.hpp"

#include <limits>

using namespace mensurflow;

namespace {

void test_attention(Device device) {
    const Execution on = test::execution_on(device);
    const std::int64_t batch = 2, heads = 3, lq = 37, lk = 41, d = 16, dv = 24;
    const Tensor q = normal({batch, heads, lq, d}, 0.0f, 1.0f, 1, 0).to(device);
    const Tensor k = normal({batch, heads, lk, d}, 0.0f, 1.0f, 2, 0).to(device);
    const Tensor v = normal({batch, heads, lk, dv}, 0.0f, 1.0f, 3, 0).to(device);
    // A Bool mask broadcast over heads: [batch, 1, lq, lk]; query 5 of batch 1 sees nothing.
    std::vector<std::uint8_t> keep(static_cast<std::size_t>(batch * lq * lk));
    for (std::size_t i = 0; i < keep.size(); ++i) {
        keep[i] = ((i * 2654435761u) >> 7) % 5 != 0 ? 1 : 0;
    }
    for (std::int64_t j = 0; j < lk; ++j) {
        keep[static_cast<std::size_t>((1 * lq + 5) * lk + j)] = 0;
    }
    const Tensor mask = Tensor::from_host(keep.data(), {batch, 1, lq, lk}, DType::Bool, device);
    const auto qv = q.to_vector<float>();
    const auto kv = k.to_vector<float>();
    const auto vv = v.to_vector<float>();
    const double scale = 1.0 / std::sqrt(static_cast<double>(d));
    for (int variant = 0; variant < 4; ++variant) {
        const bool use_mask = variant & 1;
        const bool causal = variant & 2;
        const auto got = attention(q, k, v, use_mask ? &mask : nullptr, causal, 0.0f, on)
                             .to_vector<float>();
        for (std::int64_t bi = 0; bi < batch; ++bi) {
            for (std::int64_t h = 0; h < heads; ++h) {
                const std::size_t qo = static_cast<std::size_t>((bi * heads + h) * lq * d);
                const std::size_t ko = static_cast<std::size_t>((bi * heads + h) * lk * d);
                const std::size_t vo = static_cast<std::size_t>((bi * heads + h) * lk * dv);
                std::vector<bool> visible;
                if (use_mask || causal) {
                    visible.assign(static_cast<std::size_t>(lq * lk), true);
                    for (std::int64_t i = 0; i < lq; ++i) {
                        for (std::int64_t j = 0; j < lk; ++j) {
                            bool ok = true;
                            if (use_mask) {
                                ok = keep[static_cast<std::size_t>((bi * lq + i) * lk + j)] != 0;
                            }
                            if (causal && j > i) {
                                ok = false;
                            }
                            visible[static_cast<std::size_t>(i * lk + j)] = ok;
                        }
                    }
                }
                const auto want = reference::attention(
                    std::vector<float>(qv.begin() + qo, qv.begin() + qo + lq * d),
                    std::vector<float>(kv.begin() + ko, kv.begin() + ko + lk * d),
                    std::vector<float>(vv.begin() + vo, vv.begin() + vo + lk * dv), lq, lk, d, dv,
                    scale, visible);
                const std::size_t oo = static_cast<std::size_t>((bi * heads + h) * lq * dv);
                for (std::size_t i = 0; i < want.size(); ++i) {
                    const double g = got[oo + i];
                    test::require(std::fabs(g - want[i]) <= 1e-4 * (1.0 + std::fabs(want[i])),
                                  "attention variant " + std::to_string(variant) + " at " +
                                      std::to_string(oo + i));
                }
                if (use_mask && bi == 1) {
                    for (std::int64_t c = 0; c < dv; ++c) {
                        test::require(got[oo + static_cast<std::size_t>(5 * dv + c)] == 0.0f,
                                      "fully masked query gives zeros");
                    }
                }
            }
        }
    }
    // The causal flag and the same lower triangle passed as a mask give the same bits (dv != d,
    // so both compose; on rocm the first takes its -inf from the scores GEMM, the second from
    // where()). With the mask as well, the two masks combine in either order.
    std::vector<std::uint8_t> lower(static_cast<std::size_t>(lq * lk));
    for (std::int64_t i = 0; i < lq; ++i) {
        for (std::int64_t j = 0; j < lk; ++j) {
            const bool kept = j <= i && keep[static_cast<std::size_t>((1 * lq + i) * lk + j)] != 0;
            lower[static_cast<std::size_t>(i * lk + j)] = kept ? 1 : 0;
        }
    }
    const Tensor tril = Tensor::from_host(lower.data(), {lq, lk}, DType::Bool, device);
    const Tensor batch1_mask = mask.slice(0, 1, 2);
    const auto flag = attention(q, k, v, &batch1_mask, true, 0.0f, on).to_vector<float>();
    const auto given = attention(q, k, v, &tril, false, 0.0f, on).to_vector<float>();
    test::require(std::memcmp(flag.data(), given.data(), flag.size() * sizeof(float)) == 0,
                  "causal flag and lower-triangle mask agree bit for bit");
}

// d = 64: the fused kernel on rocm (the composition elsewhere), with ragged lengths around its
// 128-query / 64-key blocks, k and v shared over the batch dimension, a [batch, 1, lq, lk]
// mask, and an explicit scale.
void test_attention_fused_shapes(Device device) {
    const Execution on = test::execution_on(device);
    const std::int64_t batch = 2, heads = 2, lq = 150, lk = 170, d = 64;
    const float scale = 0.2f;
    const Tensor q = normal({batch, heads, lq, d}, 0.0f, 1.0f, 11, 0).to(device);
    const Tensor k = normal({1, heads, lk, d}, 0.0f, 1.0f, 12, 0).to(device);
    const Tensor v = normal({1, heads, lk, d}, 0.0f, 1.0f, 13, 0).to(device);
    std::vector<std::uint8_t> keep(static_cast<std::size_t>(batch * lq * lk));
    for (std::size_t i = 0; i < keep.size(); ++i) {
        keep[i] = ((i * 2246822519u) >> 9) % 3 != 0 ? 1 : 0;
    }
    const Tensor mask = Tensor::from_host(keep.data(), {batch, 1, lq, lk}, DType::Bool, device);
    const auto qv = q.to_vector<float>();
    const auto kv = k.to_vector<float>();
    const auto vv = v.to_vector<float>();
    for (int variant = 0; variant < 4; ++variant) {
        const bool use_mask = variant & 1;
        const bool causal = variant & 2;
        const Tensor result = attention(q, k, v, use_mask ? &mask : nullptr, causal, scale, on);
        test::require(result.shape() == Shape{batch, heads, lq, d}, "fused attention shape");
        const auto got = result.to_vector<float>();
        for (std::int64_t bi = 0; bi < batch; ++bi) {
            for (std::int64_t h = 0; h < heads; ++h) {
                std::vector<bool> visible(static_cast<std::size_t>(lq * lk), true);
                for (std::int64_t i = 0; i < lq; ++i) {
                    for (std::int64_t j = 0; j < lk; ++j) {
                        bool ok = !use_mask || keep[static_cast<std::size_t>((bi * lq + i) * lk +
                                                                             j)] != 0;
                        visible[static_cast<std::size_t>(i * lk + j)] = ok && !(causal && j > i);
                    }
                }
                const std::size_t qo = static_cast<std::size_t>((bi * heads + h) * lq * d);
                const std::size_t ko = static_cast<std::size_t>(h * lk * d);
                const auto want = reference::attention(
                    std::vector<float>(qv.begin() + qo, qv.begin() + qo + lq * d),
                    std::vector<float>(kv.begin() + ko, kv.begin() + ko + lk * d),
                    std::vector<float>(vv.begin() + ko, vv.begin() + ko + lk * d), lq, lk, d, d,
                    scale, visible);
                for (std::size_t i = 0; i < want.size(); ++i) {
                    const double g = got[qo + i];
                    test::require(std::fabs(g - want[i]) <= 1e-4 * (1.0 + std::fabs(want[i])),
                                  "fused attention variant " + std::to_string(variant) + " at " +
                                      std::to_string(qo + i));
                }
            }
        }
    }
}

void test_softmax_where_argmax(Device device) {
    const Execution on = test::execution_on(device);
    const float inf = std::numeric_limits<float>::infinity();
    const Tensor x = Tensor::from_vector(std::vector<float>{0, 1, 2, -inf, -inf, -inf, 3, 3, 3},
                                         {3, 3}, device);
    const auto s = softmax(x, -1, on).to_vector<float>();
    const double e0 = std::exp(-2.0), e1 = std::exp(-1.0);
    const double total = e0 + e1 + 1.0;
    test::require(std::fabs(s[0] - e0 / total) < 1e-6 && std::fabs(s[2] - 1.0 / total) < 1e-6,
                  "softmax values");
    test::require(s[3] == 0.0f && s[4] == 0.0f && s[5] == 0.0f, "masked line gives zeros");
    test::require(std::fabs(s[6] - 1.0 / 3.0) < 1e-7, "equal values");
    // softmax over a middle axis
    const Tensor y = normal({3, 5, 7}, 0.0f, 2.0f, 4, 0).to(device);
    const auto sy = softmax(y, 1, on).to_vector<float>();
    for (int a = 0; a < 3; ++a) {
        for (int c = 0; c < 7; ++c) {
            double sum = 0.0;
            for (int b = 0; b < 5; ++b) {
                sum += sy[static_cast<std::size_t>((a * 5 + b) * 7 + c)];
            }
            test::require(std::fabs(sum - 1.0) < 1e-6, "axis-1 lines sum to one");
        }
    }
    // where with broadcasting (a scalar and a mask row)
    const Tensor cond = Tensor::from_host(std::vector<std::uint8_t>{1, 0, 1}.data(), {3},
                                          DType::Bool, device);
    const Tensor big = Tensor::from_vector(std::vector<float>{1, 2, 3, 4, 5, 6}, {2, 3}, device);
    const Tensor minus = Tensor::full({}, -inf, DType::F32, device);
    test::require(where(cond, big, minus, on).to_vector<float>() ==
                      (std::vector<float>{1, -inf, 3, 4, -inf, 6}),
                  "where broadcast");
    // argmax: ties give the first index, the first NaN wins
    const float nan = std::numeric_limits<float>::quiet_NaN();
    const Tensor am = Tensor::from_vector(std::vector<float>{1, 3, 3, 2, 0, nan, 5, nan}, {2, 4},
                                          device);
    test::require(argmax(am, -1, on).to_vector<std::int64_t>() == (std::vector<std::int64_t>{1, 1}),
                  "argmax ties and NaN");
    test::require_throws<std::invalid_argument>([&] { argmax(am, 0, on); }, "last axis only");
}

void test_bias_gelu(Device device) {
    const Execution on = test::execution_on(device);
    const Tensor x = Tensor::from_vector(std::vector<float>{1, 2, 3, 4, 5, 6}, {2, 3}, device);
    const Tensor b = Tensor::from_vector(std::vector<float>{0.5f, -1, 2}, {3}, device);
    test::require(bias_add(x, b, on).to_vector<float>() ==
                      (std::vector<float>{1.5f, 1, 5, 4.5f, 4, 8}),
                  "bias_add");
    test::require(x.to_vector<float>() == (std::vector<float>{1, 2, 3, 4, 5, 6}),
                  "bias_add leaves its input");
    test::require_throws<std::invalid_argument>([&] { bias_add(x, x, on); }, "bias must be 1-D");
    const float g = gelu(Tensor::full({}, 1.0, DType::F32, device), false, on).item<float>();
    test::require(std::fabs(g - 0.841344746f) < 1e-7f, "gelu(1)");
    const float inf = std::numeric_limits<float>::infinity();
    const auto gi = gelu(Tensor::from_vector(std::vector<float>{inf, -inf}, {2}, device), true, on)
                        .to_vector<float>();
    test::require(gi[0] == inf && gi[1] == 0.0f && std::signbit(gi[1]), "gelu of +-inf");
    const Tensor v = normal({500}, 0.0f, 3.0f, 5, 0).to(device);
    const auto vv = v.to_vector<float>();
    const auto gt = gelu(v, true, on).to_vector<float>();
    for (std::size_t i = 0; i < vv.size(); ++i) {
        const double t = vv[i];
        const double u = std::sqrt(2.0 / std::acos(-1.0)) * (t + 0.044715 * t * t * t);
        const double want = 0.5 * t * (1.0 + std::tanh(u));
        test::require(std::fabs(gt[i] - want) <= 1e-6 * (1.0 + std::fabs(want)), "gelu tanh form");
    }
}

} // namespace

int main(int argc, char** argv) {
    return test::run("attention_test", argc, argv, [] {
        test::register_oracle_cpu_kernels();
        for (Device device : test::devices()) {
            std::cout << "  attention and elementwise on " << to_string(device) << '\n';
            test_attention(device);
            test_attention_fused_shapes(device);
            test_softmax_where_argmax(device);
            test_bias_gelu(device);
        }
    });
}
