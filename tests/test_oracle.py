"""Pins the CPU oracle (oracle/oracle.c) before any GPU result is compared with it.

Three kinds of evidence, so that a plausible mistake in the restatement (a dropped term, a
transposed operand, a wrong rounding step, a wrong depth blocking) fails at least one check:

1. known answers held by the reference's own tests (tests/golden/reference_known_answers.json);
2. vectors written by the reference's own kernels compiled from its sources
   (tests/golden/ref_vectors.npz via oracle/_ref), compared bit for bit, and a live comparison
   with oracle/_ref where it is built;
3. closed forms: quarter-integer inputs make every fp32 sum exact, so the packed GEMM must equal
   the exact (float64) product in every bit, whatever its summation order.

A few tests plant a mistake in an oracle result and check that the pinning catches it.
"""
import json
import os

import numpy as np
import pytest

from helpers import quarter_input, quarter_matrix, same_bits

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def known():
    with open(os.path.join(GOLDEN, "reference_known_answers.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def vectors():
    with np.load(os.path.join(GOLDEN, "ref_vectors.npz"), allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


# ---- 1. known answers of the reference's tests ---------------------------------------------------


def test_philox_known_answers(oracle, known):
    for case in known["philox4x32_10"]["cases"]:
        got = oracle.philox(case["counter"], case["key"])
        assert got.tolist() == case["out"]


def test_matmul_known_values(oracle, known):
    case = known["matmul_2x3x2"]
    a = np.array(case["a"], dtype=np.float32)
    b = np.array(case["b"], dtype=np.float32)
    assert oracle.matmul(a, b).tolist() == case["c"]
    # A x I == A exactly (tests/ops/matmul_test.cpp:113-122)
    values = quarter_input(5 * 7, 3).reshape(5, 7)
    assert same_bits(oracle.matmul(values, np.eye(7, dtype=np.float32)), values)


def test_gemv_known_values(oracle, known):
    case = known["gemv"]
    a = np.array(case["a"], dtype=np.float32)
    p = case["plain"]
    assert oracle.gemv(a, np.array(p["x"], np.float32)).tolist() == p["y"]
    ab = case["alpha_beta"]
    got = oracle.gemv(a, np.array(ab["x"], np.float32), ab["alpha"],
                      np.array(ab["y0"], np.float32), ab["beta"])
    assert got.tolist() == ab["y"]
    t = case["transposed"]
    assert oracle.gemv(a, np.array(t["x"], np.float32), trans=True).tolist() == t["y"]


def test_gelu_known_value(oracle, known):
    case = known["gelu"]
    got = oracle.gelu(np.array([case["x"]], np.float32), approximate=False)[0]
    assert abs(float(got) - case["exact"]) < case["tolerance"]


# ---- 2. vectors of the compiled reference --------------------------------------------------------


def test_rng_matches_reference_vectors(oracle, vectors):
    seed = 0x5EED
    assert same_bits(oracle.uniform(1003, -1.0, 1.0, seed, 3), vectors["uniform_out"])
    assert same_bits(oracle.normal(1003, 0.0, 1.0, seed + 1, 5), vectors["normal_out"])


@pytest.mark.parametrize("idx", [0, 1, 2])
@pytest.mark.parametrize("kc", [256, 768])
def test_packed_gemm_matches_reference_vectors(oracle, vectors, idx, kc):
    a, b = vectors[f"gemm{idx}_a"], vectors[f"gemm{idx}_b"]
    assert same_bits(oracle.matmul(a, b, kc=kc), vectors[f"gemm{idx}_c_kc{kc}"])


def test_gemv_matches_reference_vectors(oracle, vectors):
    v = vectors
    assert same_bits(oracle.gemv(v["gemv_a"], v["gemv_xn"], 2.0, v["gemv_y0n"], 0.5), v["gemv_n"])
    assert same_bits(oracle.gemv(v["gemv_a"], v["gemv_xt"], 2.0, v["gemv_y0t"], 0.5, trans=True),
                     v["gemv_t"])
    assert same_bits(oracle.matvec(v["gemv_a"], v["gemv_xn"]), v["matvec"])


def test_elementwise_matches_reference_vectors(oracle, vectors):
    v = vectors
    assert same_bits(oracle.gelu(v["gelu_x"], True), v["gelu_tanh"])
    assert same_bits(oracle.gelu(v["gelu_x"], False), v["gelu_erf"])
    assert same_bits(oracle.bias_add(v["bias_x"], v["bias_b"]), v["bias_out"])
    assert same_bits(oracle.where(v["where_c"], v["where_x"], v["where_y"]), v["where_out"])


def test_softmax_argmax_match_reference_vectors(oracle, vectors):
    v = vectors
    assert same_bits(oracle.softmax(v["softmax_x"], -1), v["softmax_last"])
    assert same_bits(oracle.softmax(v["softmax3_x"], 1), v["softmax3_axis1"])
    assert oracle.argmax(v["argmax_x"]).tolist() == v["argmax_out"].tolist()


def test_live_reference_packed_gemm(oracle, reference):
    """Where oracle/_ref is built: more shapes and layouts, bit for bit."""
    rng = np.random.default_rng(7)
    saved = reference.get_kc()
    try:
        for m, n, k in [(1, 300, 700), (23, 16, 1537), (128, 96, 64), (200, 100, 1000)]:
            a = rng.standard_normal((m, k)).astype(np.float32)
            b = rng.standard_normal((k, n)).astype(np.float32)
            bt = np.ascontiguousarray(b.T)
            at = np.ascontiguousarray(a.T)
            for kc in (256, 768):
                reference.set_kc(kc)
                assert same_bits(oracle.matmul(a, b, kc), reference.matmul(a, b))
                assert same_bits(oracle.matmul(at.T, bt.T, kc), reference.matmul(at.T, bt.T))
    finally:
        reference.set_kc(saved)


def test_live_reference_gemv_softmax(oracle, reference):
    rng = np.random.default_rng(8)
    a = rng.standard_normal((300, 517)).astype(np.float32)
    x = rng.standard_normal(517).astype(np.float32)
    xt = rng.standard_normal(300).astype(np.float32)
    assert same_bits(oracle.gemv(a, x, 1.5), reference.gemv(a, x, 1.5))
    assert same_bits(oracle.gemv(a, xt, 1.5, trans=True), reference.gemv(a, xt, 1.5, trans=True))
    s = rng.standard_normal((64, 1024)).astype(np.float32) * 4
    assert same_bits(oracle.softmax(s), reference.softmax(s))


def test_dot_sub_known_answers_and_live_reference(oracle, reference):
    """dot and sub, the two ops the reference's CUDA backend registers besides add and mul: the
    known answers of tests/ops/dot_test.cpp:50-57, and the reference's own dot_f32 and sub_f32
    (single thread, so its order is the restatement's) on random inputs, bit for bit."""
    a = np.array([1, 2, 3], np.float32)
    b = np.array([4, -5, 6], np.float32)
    assert oracle.dot(a, b) == np.float32(12.0) and oracle.dot(a, a) == np.float32(14.0)
    assert oracle.dot(a[:0], b[:0]) == np.float32(0.0)
    rng = np.random.default_rng(21)
    reference.set_threads(1)
    try:
        for n in (1, 7, 1000, 300001):
            x = rng.standard_normal(n).astype(np.float32)
            y = rng.standard_normal(n).astype(np.float32)
            assert same_bits(np.array([oracle.dot(x, y)]), np.array([reference.dot(x, y)])), n
            assert same_bits(oracle.sub(x, y), reference.sub(x, y)), n
    finally:
        reference.set_threads(reference.max_threads())


def test_dot_closed_form_and_planted_float_accumulation(oracle):
    """The products are summed in double: quarter-integer inputs give the exact sum's float, and
    a cancellation that a float accumulator loses (1e8 + 1 - 1e8) keeps its 1."""
    x = quarter_input(4097, 22)
    y = quarter_input(4097, 23)
    exact = np.float32(np.dot(x.astype(np.float64), y.astype(np.float64)))
    assert oracle.dot(x, y) == exact
    big = np.array([1e8, 1.0, -1e8], np.float32)
    ones = np.ones(3, np.float32)
    assert oracle.dot(big, ones) == np.float32(1.0)
    float_sum = np.float32(0.0)
    for v in big * ones:
        float_sum = np.float32(float_sum + v)
    assert float_sum != oracle.dot(big, ones), "a float accumulator must be told apart"


# ---- 3. closed forms -------------------------------------------------------------------------------


@pytest.mark.parametrize("m,n,k", [(33, 47, 129), (64, 64, 1024), (5, 300, 2000)])
def test_packed_gemm_exact_on_quarter_integers(oracle, m, n, k):
    a = quarter_matrix(m, k, 1)
    b = quarter_matrix(k, n, 2)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert same_bits(oracle.matmul(a, b), exact.astype(np.float32))
    # transposed storage of both operands gives the same exact product
    at = np.ascontiguousarray(a.T)
    bt = np.ascontiguousarray(b.T)
    assert same_bits(oracle.matmul(at.T, bt.T), exact.astype(np.float32))


def test_gemv_exact_on_quarter_integers(oracle):
    a = quarter_matrix(300, 700, 3)
    x = quarter_matrix(1, 700, 4)[0]
    xt = quarter_matrix(1, 300, 5)[0]
    assert same_bits(oracle.gemv(a, x), (a.astype(np.float64) @ x).astype(np.float32))
    assert same_bits(oracle.gemv(a, xt, trans=True),
                     (a.T.astype(np.float64) @ xt).astype(np.float32))


def test_gemm_composition_rounding(oracle):
    """gemm = fl(fl(alpha*AB) + fl(beta*C0)) (src/ops/blas.cpp:246-257)."""
    rng = np.random.default_rng(9)
    a = rng.standard_normal((20, 30)).astype(np.float32)
    b = rng.standard_normal((30, 10)).astype(np.float32)
    c0 = rng.standard_normal((20, 10)).astype(np.float32)
    ab = oracle.matmul(a, b)
    want = (np.float32(1.5) * ab) + (np.float32(0.5) * c0)
    assert same_bits(oracle.gemm(a, b, 1.5, c0, 0.5), want.astype(np.float32))
    assert same_bits(oracle.gemm(np.ascontiguousarray(a.T), b, 1.5, c0, 0.5, trans_a=True),
                     want.astype(np.float32))


def test_gemm_composition_matches_reference_vectors(oracle, vectors):
    """orc_axpby_f32 against the reference's own mul -> scal -> add chain of mensurflow::gemm
    (src/ops/blas.cpp:246-257), bit for bit, with and without C0, on values that separate one
    rounding from two and on overflow, signed zeros, subnormals, infinities and NaN."""
    x, c0 = vectors["axpby_x"], vectors["axpby_c0"]
    for i, (alpha, beta) in enumerate(vectors["axpby_cases"].tolist()):
        assert same_bits(oracle.axpby(x, alpha, c0, beta), vectors[f"axpby_out{i}"]), (alpha, beta)
        assert same_bits(oracle.axpby(x, alpha, None, 0.0), vectors[f"axpby_out{i}_noc0"]), alpha


def test_batched_composition_matches_reference_vectors(oracle, vectors):
    """The oracle's batched GEMM (packed product per matrix, then orc_axpby_f32) against the
    reference's gemm_batched_f32_parallel with its finish pass (gemm_batched.cpp:12-28,58-70):
    A broadcast over the batch, B read transposed, alpha alone and alpha with beta * C0."""
    m, n, k, batch = 21, 19, 37, 3
    a = vectors["batched_a"].reshape(m, k)
    b = vectors["batched_b"].reshape(batch, n, k)
    c0 = vectors["batched_c0"]
    for i in range(batch):
        product = oracle.matmul(a, b[i].T, kc=768)
        assert same_bits(oracle.axpby(product, 0.125, None, 0.0), vectors["batched_scores"][i])
        assert same_bits(oracle.axpby(product, 1.5, c0[i], 0.5), vectors["batched_ab"][i])


def test_planted_fused_composition_is_caught(vectors):
    """An epilogue that fused alpha*x + beta*c0 into one rounding (an fma) would not match the
    reference's chain on these vectors."""
    x = vectors["axpby_x"].astype(np.float64)
    scaled_c0 = (np.float32(0.5) * vectors["axpby_c0"]).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        fused = (1.5 * x + scaled_c0).astype(np.float32)  # 1.5 * x is exact in float64
    assert not same_bits(fused, vectors["axpby_out0"])


def test_live_reference_composition(oracle, reference):
    """Where oracle/_ref is built: more alpha/beta values and a larger batched case, live."""
    rng = np.random.default_rng(21)
    x = (rng.standard_normal(5000) * 100).astype(np.float32)
    c0 = (rng.standard_normal(5000) * 100).astype(np.float32)
    for alpha, beta in [(0.3, 0.7), (-1.25, 2.0), (1.0, -3.0), (7.0, 0.0)]:
        assert same_bits(oracle.axpby(x, alpha, c0, beta),
                         reference.gemm_composition(x, alpha, c0, beta)), (alpha, beta)
    m, n, k, batch = 70, 45, 300, 4
    a = rng.uniform(-1, 1, (batch, k, m)).astype(np.float32)  # read transposed
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)  # broadcast over the batch
    cz = rng.standard_normal((batch, m, n)).astype(np.float32)
    saved = reference.get_kc()
    try:
        reference.set_kc(768)
        got = reference.gemm_batched(a, b, np.arange(batch) * k * m, np.zeros(batch), m, n, k,
                                     1, m, n, 1, alpha=0.25, c0=cz, beta=-2.0)
    finally:
        reference.set_kc(saved)
    for i in range(batch):
        want = oracle.axpby(oracle.matmul(a[i].T, b, kc=768), 0.25, cz[i], -2.0)
        assert same_bits(got[i], want), i


def test_softmax_special_lines(oracle):
    x = np.array([[0.0, 1.0, 2.0], [-np.inf] * 3, [1.0, np.nan, 0.0]], dtype=np.float32)
    out = oracle.softmax(x)
    e = np.exp(np.array([0.0, 1.0, 2.0]) - 2.0)
    np.testing.assert_allclose(out[0], e / e.sum(), rtol=1e-6)
    assert np.all(out[1] == 0.0)
    assert np.all(np.isnan(out[2]))


def test_argmax_semantics(oracle):
    x = np.array([[1, 3, 3, 2], [0, np.nan, 5, np.nan], [-0.0, 0.0, -1, -1]], dtype=np.float32)
    assert oracle.argmax(x).tolist() == [1, 1, 0]


# ---- planted mistakes: the checks above have teeth --------------------------------------------------


def test_planted_dropped_term_is_caught(oracle):
    a = quarter_matrix(16, 65, 11)
    b = quarter_matrix(65, 16, 12)
    exact = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    dropped = oracle.matmul(a[:, :-1], b[:-1, :])  # the last depth term left out
    assert not same_bits(dropped, exact)


def test_planted_transposed_operand_is_caught(oracle):
    a = quarter_matrix(24, 24, 13)
    b = quarter_matrix(24, 24, 14)
    exact = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    assert not same_bits(oracle.matmul(a, b.T), exact)


def test_planted_wrong_blocking_is_caught(oracle, vectors):
    a, b = vectors["gemm2_a"], vectors["gemm2_b"]
    # k = 1000 with KC = 768 stored vs a single chain: the last bits must differ somewhere.
    assert not same_bits(oracle.matmul(a, b, kc=0), vectors["gemm2_c_kc768"])


def test_planted_gemv_float_accumulation_is_caught(oracle, vectors):
    v = vectors
    a, x = v["gemv_a"].astype(np.float32), v["gemv_xn"]
    float_sum = np.zeros(a.shape[0], dtype=np.float32)
    for j in range(a.shape[1]):
        float_sum = float_sum + a[:, j] * x[j]
    assert not same_bits(float_sum, v["matvec"])
