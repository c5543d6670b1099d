"""GPU parity of mfr_sgemv / mfr_smatvec against the oracle (double accumulation, one rounding,
as src/backends/cpu/ops/blas/blas.cpp:55-79).

The GPU adds the same exact double products in a different fixed order, so after the single
rounding to fp32 nearly every output has the reference's bits; the bar is the north-star one
(1e-5*sqrt(K) relative to sum|a*x|), and the share of bit-identical outputs is reported."""
import numpy as np
import pytest

import mensurflow_amd as mf
from helpers import normal, quarter_matrix, record_parity, same_bits, tolerance, uniform

pytestmark = pytest.mark.gpu


def dev(x, stream):
    return mf.DeviceArray.from_numpy(np.ascontiguousarray(x), stream)


def assert_gemv_parity(got, want, a, x, alpha, y0, beta, trans, what):
    mag = (np.abs(a.T if trans else a).astype(np.float64) @ np.abs(x).astype(np.float64))
    scale = abs(alpha) * mag + (abs(beta) * np.abs(y0) if y0 is not None else 0.0)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    k = a.shape[0] if trans else a.shape[1]
    rel = float(np.max(err / (scale + 1e-30)))
    assert rel <= tolerance(k), f"{what}: rel err {rel:.3e} > {tolerance(k):.3e}"
    return rel, float(np.mean(got.view(np.uint32) == want.view(np.uint32)))


def test_known_values(stream):
    a = dev(np.array([[1, 2, 3], [4, 5, 6]], np.float32), stream)
    ones3 = dev(np.ones(3, np.float32), stream)
    assert mf.sgemv(a, ones3).numpy().tolist() == [6, 15]
    y0 = dev(np.array([2, 3], np.float32), stream)
    assert mf.sgemv(a, ones3, alpha=2.0, y0=y0, beta=0.5).numpy().tolist() == [13, 31.5]
    assert mf.sgemv(a, dev(np.ones(2, np.float32), stream), trans=True).numpy().tolist() == [5, 7, 9]
    assert mf.matvec(a, ones3).numpy().tolist() == [6, 15]


@pytest.mark.parametrize("trans", [False, True])
def test_config2_full_size(stream, oracle, trans):
    """A[16384,16384] and x uniform[-1,1] from a seed, y0 ~ N(0,1),
    y = 2*op(A)*x + 0.5*y0, for A and A^T."""
    n = 16384
    seed = 11
    a = uniform(oracle, (n, n), -1.0, 1.0, seed, 0)
    x = uniform(oracle, (n,), -1.0, 1.0, seed, n * n)
    y0 = normal(oracle, (n,), 0.0, 1.0, seed + 1, 0)
    got = mf.sgemv(dev(a, stream), dev(x, stream), alpha=2.0, y0=dev(y0, stream), beta=0.5,
                   trans=trans).numpy()
    want = oracle.gemv(a, x, 2.0, y0, 0.5, trans=trans)
    rel, same = assert_gemv_parity(got, want, a, x, 2.0, y0, 0.5, trans, f"cfg2 trans={trans}")
    print(f"cfg2 trans={trans}: rel err {rel:.3e}, bit-identical outputs {same:.6f}")
    record_parity(f"cfg2_gemv_16384_{'t' if trans else 'n'}", rel_err_vs_magnitude=rel,
                  bar=tolerance(n), bit_identical_share=same,
                  differing_outputs=int(np.sum(got.view(np.uint32) != want.view(np.uint32))))
    assert same > 0.999


# 16-byte paths too (cols % 4 == 0): a partial last 256-column strip of the T form, row counts
# around its 16-row step and chunking, and a partial last group of 8 rows in the N form.
@pytest.mark.parametrize("rows,cols", [(1, 1), (1, 1000), (1000, 1), (37, 53), (255, 257),
                                       (513, 4099), (4093, 130), (3, 70000), (1029, 1024),
                                       (300, 260), (2050, 772), (17, 4096), (5, 4096),
                                       (4111, 516)])
@pytest.mark.parametrize("trans", [False, True])
def test_exact_shapes(stream, oracle, rows, cols, trans):
    a = quarter_matrix(rows, cols, rows + cols)
    x = quarter_matrix(1, rows if trans else cols, 7)[0]
    y0 = quarter_matrix(1, cols if trans else rows, 8)[0]
    got = mf.sgemv(dev(a, stream), dev(x, stream), alpha=2.0, y0=dev(y0, stream), beta=0.5,
                   trans=trans).numpy()
    assert same_bits(got, oracle.gemv(a, x, 2.0, y0, 0.5, trans=trans)), (rows, cols, trans)


@pytest.mark.parametrize("trans", [False, True])
def test_padded_rows(stream, oracle, trans):
    """A [rows, cols] view with a leading dimension larger than cols (and not a multiple of 4)."""
    rows, cols, ld = 300, 500, 509
    stored = uniform(oracle, (rows, ld), -1.0, 1.0, 21, 0)
    a_view = dev(stored, stream).slice(1, 0, cols)
    a = stored[:, :cols]
    x = uniform(oracle, (rows if trans else cols,), -1.0, 1.0, 22, 0)
    got = mf.sgemv(a_view, dev(x, stream), trans=trans).numpy()
    want = oracle.gemv(np.ascontiguousarray(a), x, trans=trans)
    assert_gemv_parity(got, want, a, x, 1.0, None, 0.0, trans, "padded")


@pytest.mark.parametrize("trans", [False, True])
def test_no_products_gives_beta_y0(stream, trans):
    rows, cols = (0, 7) if trans else (7, 0)
    a = mf.DeviceArray.empty((rows, cols), stream)
    x = mf.DeviceArray.empty((0,), stream)
    y0 = np.arange(7, dtype=np.float32) - 3
    got = mf.sgemv(a, x, alpha=2.0, y0=dev(y0, stream), beta=0.5, trans=trans).numpy()
    assert same_bits(got, (np.float32(0.5) * y0).astype(np.float32))


def test_deterministic_and_matvec(stream, oracle):
    a = uniform(oracle, (2000, 3000), -1.0, 1.0, 31, 0)
    x = uniform(oracle, (3000,), -1.0, 1.0, 32, 0)
    xt = uniform(oracle, (2000,), -1.0, 1.0, 33, 0)
    a_d, x_d, xt_d = dev(a, stream), dev(x, stream), dev(xt, stream)
    assert same_bits(mf.sgemv(a_d, x_d).numpy(), mf.sgemv(a_d, x_d).numpy())
    assert same_bits(mf.sgemv(a_d, xt_d, trans=True).numpy(),
                     mf.sgemv(a_d, xt_d, trans=True).numpy())
    got = mf.matvec(a_d, x_d).numpy()
    assert_gemv_parity(got, oracle.matvec(a, x), a, x, 1.0, None, 0.0, False, "matvec")


def test_beta_without_y0_is_invalid(stream):
    a = dev(np.ones((4, 4), np.float32), stream)
    x = dev(np.ones(4, np.float32), stream)
    with pytest.raises(ValueError):
        mf.sgemv(a, x, beta=1.0)


# ---- dot (mfr_sdot) ------------------------------------------------------------------------------

@pytest.mark.parametrize("n", [0, 1, 3, 4, 1000, 16383, 16384, 16385, 1_000_003])
@pytest.mark.parametrize("offset", [0, 1])
def test_dot_exact_on_quarter_integers(stream, n, offset):
    """Quarter-integer inputs: every product and partial sum is exact in double, so the result is
    the exact sum rounded once, whatever the order; around the 16384-element chunks, at aligned
    (16-byte loads) and unaligned starts, and n = 0 (0)."""
    rng = np.random.default_rng(n + 7 * offset)
    xs = (rng.integers(-16, 17, n + offset) / 4).astype(np.float32)
    ys = (rng.integers(-16, 17, n + offset) / 4).astype(np.float32)
    x = dev(xs, stream).slice(0, offset, offset + n)
    y = dev(ys, stream).slice(0, offset, offset + n)
    # The reference's sum starts at +0.0 (blas.cpp:15), so an exact -0 sum comes out +0.
    want = np.float32(0.0 + np.dot(xs[offset:].astype(np.float64), ys[offset:].astype(np.float64)))
    got = mf.dot(x, y).numpy()
    assert got.shape == () and same_bits(np.array([got]), np.array([want])), (n, offset)


@pytest.mark.parametrize("n", [5, 100_003, 1 << 24])
def test_dot_matches_oracle_bits(stream, oracle, n):
    """Normal inputs: the double sums in two orders round to the same float (the oracle adds in
    index order as the reference's single-thread dot_f32 does); repeated calls give the same
    bits."""
    x = normal(oracle, (n,), 0.0, 1.0, 41, 0)
    y = normal(oracle, (n,), 0.0, 1.0, 42, 0)
    x_d, y_d = dev(x, stream), dev(y, stream)
    got = mf.dot(x_d, y_d).numpy()
    assert same_bits(np.array([got]), np.array([oracle.dot(x, y)])), n
    assert same_bits(np.array([mf.dot(x_d, y_d).numpy()]), np.array([got]))


def test_dot_lengths_must_agree(stream):
    with pytest.raises(ValueError):
        mf.dot(dev(np.ones(3, np.float32), stream), dev(np.ones(4, np.float32), stream))
