// Double-precision references for the C++ tests: a plain triple loop with the per-entry
// magnitude sum|a*b| that fp32 rounding error is measured against (the reference's
// tests/reference/blas.hpp idea), and naive attention in double.
#pragma once

#include <cmath>
#include <cstdint>
#include <limits>
#include <vector>

namespace reference {

struct Product {
    std::vector<double> value, magnitude;
};

// C[m,n] = A[m,k] B[k,n], row-major contiguous inputs.
inline Product matmul(const std::vector<float>& a, const std::vector<float>& b, std::int64_t m,
                      std::int64_t n, std::int64_t k) {
    Product r;
    r.value.assign(static_cast<std::size_t>(m * n), 0.0);
    r.magnitude.assign(static_cast<std::size_t>(m * n), 0.0);
    for (std::int64_t i = 0; i < m; ++i) {
        for (std::int64_t p = 0; p < k; ++p) {
            const double av = a[static_cast<std::size_t>(i * k + p)];
            for (std::int64_t j = 0; j < n; ++j) {
                const double prod = av * b[static_cast<std::size_t>(p * n + j)];
                r.value[static_cast<std::size_t>(i * n + j)] += prod;
                r.magnitude[static_cast<std::size_t>(i * n + j)] += std::fabs(prod);
            }
        }
    }
    return r;
}

// Max over entries of |got - want| / (magnitude + tiny).
inline double relative_error(const std::vector<float>& got, const Product& want) {
    double worst = 0.0;
    for (std::size_t i = 0; i < got.size(); ++i) {
        const double err = std::fabs(static_cast<double>(got[i]) - want.value[i]);
        worst = std::fmax(worst, err / (want.magnitude[i] + 1e-30));
    }
    return worst;
}

// One batch of attention: q [lq,d], k [lk,d], v [lk,dv]; keep[i*lk+j] (empty = all visible).
inline std::vector<double> attention(const std::vector<float>& q, const std::vector<float>& k,
                                     const std::vector<float>& v, std::int64_t lq, std::int64_t lk,
                                     std::int64_t d, std::int64_t dv, double scale,
                                     const std::vector<bool>& keep) {
    std::vector<double> out(static_cast<std::size_t>(lq * dv), 0.0);
    std::vector<double> score(static_cast<std::size_t>(lk));
    for (std::int64_t i = 0; i < lq; ++i) {
        double top = -std::numeric_limits<double>::infinity();
        for (std::int64_t j = 0; j < lk; ++j) {
            double s = 0.0;
            for (std::int64_t c = 0; c < d; ++c) {
                s += static_cast<double>(q[static_cast<std::size_t>(i * d + c)]) *
                     k[static_cast<std::size_t>(j * d + c)];
            }
            const bool visible = keep.empty() || keep[static_cast<std::size_t>(i * lk + j)];
            score[static_cast<std::size_t>(j)] =
                visible ? s * scale : -std::numeric_limits<double>::infinity();
            top = std::fmax(top, score[static_cast<std::size_t>(j)]);
        }
        if (top == -std::numeric_limits<double>::infinity()) {
            continue;
        }
        double sum = 0.0;
        for (auto& s : score) {
            s = std::exp(s - top);
            sum += s;
        }
        for (std::int64_t c = 0; c < dv; ++c) {
            double acc = 0.0;
            for (std::int64_t j = 0; j < lk; ++j) {
                acc += score[static_cast<std::size_t>(j)] / sum * v[static_cast<std::size_t>(j * dv + c)];
            }
            out[static_cast<std::size_t>(i * dv + c)] = acc;
        }
    }
    return out;
}

} // namespace reference
