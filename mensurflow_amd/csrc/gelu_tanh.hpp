// The tanh form of mensurflow::gelu (src/backends/cpu/ops/elementwise/elementwise.cpp:24-27,
// 173-194) in double, rounded once to float, for the HIP kernels (through common.hpp) and for a
// CPU test that runs the same operations over every float input against the oracle
// (tests/cpp/gelu_exhaustive_test.cpp).
//
// The reference computes u = sqrt(2/pi) v (1 + 0.044715 v^2), z = exp(-|2u|) with glibc's exp,
// s = z / (1 + z) for 2u < 0 and 1 / (1 + z) otherwise, and rounds v * s to float. Here exp is
// Tang's table-driven method and the division the hardware reciprocal with one Newton step and
// a remainder correction: fewer double operations than the device library's exp and division,
// and the same float as the reference for all 2^32 inputs (the exhaustive test, with the
// reciprocal's start exact and 2^-20 off). Compiled with -ffp-contract=off, so the products and
// sums not written as fma round as in the reference.
#pragma once

#include <cmath>

#if defined(__HIPCC__)
#define MFR_GELU_FN __device__ inline
#define MFR_GELU_TABLE static __constant__
#define MFR_GELU_RCP(d) __builtin_amdgcn_rcp(d)
#else
#define MFR_GELU_FN inline
#define MFR_GELU_TABLE static const
#ifndef MFR_GELU_RCP
#define MFR_GELU_RCP(d) (1.0 / (d))
#endif
#endif

namespace mfr::gelu_math {

// 2^(j/64) for j = 0..63, each rounded to the nearest double (computed to 60 digits).
MFR_GELU_TABLE double kExp2Table[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0,
};

// exp(t) for t <= 0 in double by Tang's table-driven method (ACM TOMS 15(2), 1989): with
// k = rint(t * 64/ln2) = 64m + j, t = k ln2/64 + r, |r| <= ln2/128, and
// exp(t) = 2^m * 2^(j/64) * (1 + p(r)), p the degree-5 Taylor polynomial of e^r - 1 (its
// truncation is below 3.5e-17, a third of an ulp). ln2/64 is split into a 36-bit head, so
// k * head is exact for |k| < 2^17, and a tail. t below -800 is taken as -800 (exp gives 0 for
// both); a NaN t also gives 0 (only a NaN input makes t NaN, and its result is NaN anyway).
// `table` is kExp2Table or a copy of it (a kernel may keep one in LDS).
MFR_GELU_FN double exp_nonpositive(double t, const double* table) {
    constexpr double kInvStep = 0x1.71547652b82fep+6;  // 64 / ln2
    constexpr double kStepHead = 0x1.62e42fefa0000p-7; // ln2/64, 36 bits
    constexpr double kStepTail = 0x1.cf79abc9e3b3ap-46; // ln2/64 - head
    t = fmax(t, -800.0);
    const double kd = rint(t * kInvStep);
    const int k = static_cast<int>(kd);
    double r = fma(-kd, kStepHead, t);
    r = fma(-kd, kStepTail, r);
    double q = fma(r, 1.0 / 120.0, 1.0 / 24.0);
    q = fma(r, q, 1.0 / 6.0);
    q = fma(r, q, 0.5);
    const double pm1 = fma(r * r, q, r); // e^r - 1
    const double two_j = table[k & 63];
    return ldexp(fma(two_j, pm1, two_j), k >> 6);
}

// num / d for d in [1, 2]: the reciprocal, one Newton step and one correction of the quotient
// with its remainder.
MFR_GELU_FN double divide_by_1_to_2(double num, double d) {
    double q = MFR_GELU_RCP(d);
    const double e = fma(-d, q, 1.0);
    q = fma(q, e, q);
    const double s = num * q;
    const double rem = fma(-d, s, num);
    return fma(rem, q, s);
}

// 2u = 2 sqrt(2/pi) v (1 + 0.044715 v^2) takes the factor 2 into the constant, which is exact (a
// product by 2 only moves the exponent), so it is the reference's 2u to the bit. No branch: the
// formula runs for every input (a kernel's unrolled epilogue then has no branch between values).
// For +inf it gives +inf, as the reference does; for -inf it gives NaN (-inf * 0), and the
// reference's -0 is selected at the end.
MFR_GELU_FN float gelu_tanh(float value, const double* table) {
    const double v = static_cast<double>(value);
    const double twice = (2.0 * 0.79788456080286535588) * v * (1.0 + 0.044715 * v * v);
    const double z = exp_nonpositive(-fabs(twice), table);
    const double s = divide_by_1_to_2(twice < 0.0 ? z : 1.0, 1.0 + z);
    const float result = static_cast<float>(v * s);
    return value == -__builtin_inff() ? -0.0f : result;
}

MFR_GELU_FN float gelu_tanh(float value) { return gelu_tanh(value, kExp2Table); }

} // namespace mfr::gelu_math
