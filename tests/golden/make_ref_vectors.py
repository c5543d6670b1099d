"""Writes tests/golden/ref_vectors.npz: small input/output vectors of the reference's own CPU
kernels (bakir004/mensurflow), produced by oracle/_ref/libmfref.so, which is compiled from the
reference sources where they lie (oracle/Makefile, target `ref`).

The vectors pin the C restatement in oracle/ for the parts whose last bits depend on the
reference's exact arithmetic: the packed GEMM's depth blocking, libm's exp/erfc/log/cos/sin
inside gelu, softmax and normal, and the double-accumulating gemv. They travel with the tree, so
the oracle stays pinned where the reference is absent.

Run from the repository root:  python tests/golden/make_ref_vectors.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import Reference  # noqa: E402

OUT = os.path.join(HERE, "ref_vectors.npz")

# (alpha, beta) pairs of the gemm composition vectors; alpha 1 and beta 0 skip their pass.
AXPBY_CASES = [(1.5, 0.5), (1.0, 0.5), (1.5, 0.0), (-2.0, -0.75), (1.0, 0.0), (0.125, 3.0)]


def main() -> None:
    ref = Reference()
    ref.set_threads(4)
    v: dict[str, np.ndarray] = {}
    seed = 0x5EED

    # Seeded factories, including an offset inside a Philox block.
    v["uniform_out"] = ref.uniform(1003, -1.0, 1.0, seed, 3)
    v["normal_out"] = ref.normal(1003, 0.0, 1.0, seed + 1, 5)

    # Packed GEMM at two depth blockings; shapes around the 6x16 tile and the block edges.
    for idx, (m, n, k) in enumerate([(17, 31, 13), (65, 129, 300), (40, 48, 1000)]):
        a = ref.uniform(m * k, -1.0, 1.0, seed + 10 + idx, 0).reshape(m, k)
        b = ref.uniform(k * n, -1.0, 1.0, seed + 20 + idx, 0).reshape(k, n)
        v[f"gemm{idx}_a"] = a
        v[f"gemm{idx}_b"] = b
        for kc in (256, 768):
            ref.set_kc(kc)
            v[f"gemm{idx}_c_kc{kc}"] = ref.matmul(a, b, parallel=True)
    ref.set_kc(768)

    # gemv / matvec with double accumulation.
    rows, cols = 37, 53
    a = ref.uniform(rows * cols, -1.0, 1.0, seed + 30, 0).reshape(rows, cols)
    xn = ref.uniform(cols, -1.0, 1.0, seed + 31, 0)
    xt = ref.uniform(rows, -1.0, 1.0, seed + 32, 0)
    y0n = ref.normal(rows, 0.0, 1.0, seed + 33, 0)
    y0t = ref.normal(cols, 0.0, 1.0, seed + 34, 0)
    v["gemv_a"], v["gemv_xn"], v["gemv_xt"], v["gemv_y0n"], v["gemv_y0t"] = a, xn, xt, y0n, y0t
    v["gemv_n"] = ref.gemv(a, xn, 2.0, y0n, 0.5, trans=False)
    v["gemv_t"] = ref.gemv(a, xt, 2.0, y0t, 0.5, trans=True)
    v["matvec"] = ref.matvec(a, xn)

    # gelu on a grid plus special values.
    grid = np.concatenate([
        np.linspace(-12.0, 12.0, 2401, dtype=np.float32),
        np.array([0.0, -0.0, 1e-30, -1e-30, 3.4e38, -3.4e38, np.inf, -np.inf, np.nan,
                  1e-8, -1e-8, 50.0, -50.0], dtype=np.float32),
    ]).astype(np.float32)
    v["gelu_x"] = grid
    v["gelu_tanh"] = ref.gelu(grid, approximate=True)
    v["gelu_erf"] = ref.gelu(grid, approximate=False)

    # softmax lines: ordinary, fully masked, partly masked, NaN, +inf, and an inner axis.
    sm = ref.normal(8 * 37, 0.0, 3.0, seed + 40, 0).reshape(8, 37)
    sm[1, :] = -np.inf
    sm[2, 10:] = -np.inf
    sm[3, 5] = np.nan
    sm[4, 7] = np.inf
    v["softmax_x"] = sm
    v["softmax_last"] = ref.softmax(sm, axis=-1)
    sm3 = ref.normal(3 * 5 * 7, 0.0, 2.0, seed + 41, 0).reshape(3, 5, 7)
    v["softmax3_x"] = sm3
    v["softmax3_axis1"] = ref.softmax(sm3, axis=1)

    # argmax: ties, signed zeros, NaN.
    am = ref.uniform(6 * 9, -1.0, 1.0, seed + 50, 0).reshape(6, 9)
    am[1, :] = 0.25
    am[2, 2], am[2, 6] = -0.0, 0.0
    am[2, :2], am[2, 3:6], am[2, 7:] = -1.0, -1.0, -1.0
    am[3, 4] = np.nan
    am[4, 0] = np.nan
    am[5, 8] = 2.0
    v["argmax_x"] = am
    v["argmax_out"] = ref.argmax(am)

    # bias_add and where.
    x = ref.normal(7 * 11, 0.0, 1.0, seed + 60, 0).reshape(7, 11)
    bias = ref.uniform(11, -0.1, 0.1, seed + 61, 0)
    v["bias_x"], v["bias_b"] = x, bias
    v["bias_out"] = ref.bias_add(x, bias)
    cond = (ref.uniform(77, 0.0, 1.0, seed + 62, 0) > 0.5).astype(np.uint8)
    y = ref.normal(77, 0.0, 1.0, seed + 63, 0)
    v["where_c"], v["where_x"], v["where_y"] = cond, x.reshape(-1), y
    v["where_out"] = ref.where(cond, x.reshape(-1), y)

    # mensurflow::gemm's alpha/beta chain after the product (mul, scal, add; src/ops/blas.cpp:
    # 246-257), on values that separate one rounding from two (an fma would differ), overflow,
    # signed zeros, subnormals, infinities and NaN.
    prod = ref.normal(4 * 97, 0.0, 30.0, seed + 70, 0)
    c0 = ref.normal(4 * 97, 0.0, 30.0, seed + 71, 0)
    specials = np.array([0.0, -0.0, 1e-40, -1e-40, 3.0e38, -3.0e38, np.inf, -np.inf, np.nan,
                         1.0, -1.0, 2.5e-38], dtype=np.float32)
    prod[:12], c0[:12] = specials, specials[::-1]
    prod[12:24], c0[12:24] = specials, specials
    v["axpby_x"], v["axpby_c0"] = prod, c0
    v["axpby_cases"] = np.array(AXPBY_CASES, dtype=np.float32)
    for i, (alpha, beta) in enumerate(AXPBY_CASES):
        v[f"axpby_out{i}"] = ref.gemm_composition(prod, alpha, c0, beta)
        v[f"axpby_out{i}_noc0"] = ref.gemm_composition(prod, alpha, None, 0.0)

    # gemm_strided_batched's CPU kernel with its finish pass: 3 matrices, A broadcast over the
    # batch (every offset 0), B read transposed, alpha 1/8 without C0 (attention's scores) and
    # alpha 1.5, beta 0.5 with C0.
    bm, bn, bk, batch = 21, 19, 37, 3
    ba = ref.uniform(bm * bk, -1.0, 1.0, seed + 80, 0)
    bb = ref.uniform(batch * bn * bk, -1.0, 1.0, seed + 81, 0)  # [batch, n, k], read as B^T
    bc0 = ref.normal(batch * bm * bn, 0.0, 1.0, seed + 82, 0).reshape(batch, bm, bn)
    a_off = np.zeros(batch, np.int64)
    b_off = np.arange(batch, dtype=np.int64) * bn * bk
    v["batched_a"], v["batched_b"], v["batched_c0"] = ba, bb, bc0
    v["batched_scores"] = ref.gemm_batched(ba, bb, a_off, b_off, bm, bn, bk, bk, 1, 1, bk,
                                           alpha=0.125)
    v["batched_ab"] = ref.gemm_batched(ba, bb, a_off, b_off, bm, bn, bk, bk, 1, 1, bk,
                                       alpha=1.5, c0=bc0, beta=0.5)

    np.savez_compressed(OUT, **v)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(v)} arrays)")


if __name__ == "__main__":
    main()
