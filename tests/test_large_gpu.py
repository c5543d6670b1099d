"""Index arithmetic past 2^31 elements: element offsets that overflow int32 and byte offsets past
2^32, in gemv N and T over A [3, 2^30 + 4] (3.2 G elements, 12.9 GB), in a GEMM whose output
has more than 2^31 elements, and with a 2.4 G-element operand (GEMM tiles in both orientations,
the thin path, argmax, broadcast strided copies, elementwise add). Inputs are built on the device (row-wise constants, quarter
integers), so every expected value has a closed form and is exact in double before the one
rounding to fp32."""
import numpy as np
import pytest

import mensurflow_amd as mf
from helpers import quarter_matrix, same_bits

pytestmark = pytest.mark.gpu

ROWS, COLS = 3, (1 << 30) + 4


def dev(x, stream):
    return mf.DeviceArray.from_numpy(np.ascontiguousarray(x), stream)


def test_gemv_past_2_31_elements(stream):
    a = mf.DeviceArray.empty((ROWS, COLS), stream)
    for r in range(ROWS):
        mf.fill(a.slice(0, r, r + 1), 0.25 * (r + 1))
    x = mf.DeviceArray.empty((COLS,), stream)
    mf.fill(x, 1.0)
    # N: y[r] = 0.25 (r + 1) * COLS, exact in double, then rounded once to fp32.
    y = mf.sgemv(a, x).numpy()
    want = np.array([0.25 * (r + 1) * COLS for r in range(ROWS)], np.float64).astype(np.float32)
    assert same_bits(y, want)
    # T: y[j] = sum_r A[r][j] x[r] = 0.25 (1*1 + 2*2 + 3*3) = 3.5 for every column, including the
    # columns whose element offsets in rows 1 and 2 are past 2^31.
    yt = mf.sgemv(a, dev(np.array([1, 2, 3], np.float32), stream), trans=True)
    piece = 1 << 20
    for lo in (0, COLS // 2, COLS - piece):
        assert np.all(yt.slice(0, lo, lo + piece).numpy() == np.float32(3.5)), lo
    a.close()
    yt.close()


def test_gemm_output_past_2_31_elements(stream):
    m, n, k = 65536, 32772, 8  # m * n = 2^31 + 2^18 outputs
    av = quarter_matrix(m, k, 101)
    bv = quarter_matrix(k, n, 102)
    c = mf.DeviceArray.empty((m, n), stream)
    mf.gemm(dev(av, stream), dev(bv, stream), alpha=1.5, out=c)
    for lo in (0, m // 2, m - 4):
        rows = slice(lo, lo + 4)
        want = (np.float32(1.5) * (av[rows].astype(np.float64) @ bv.astype(np.float64))
                .astype(np.float32))
        assert same_bits(c.slice(0, lo, lo + 4).numpy(), want), lo
    c.close()


def test_operands_past_2_31_elements(stream):
    """A[60000, 40000] (2.4 G elements, 9.6 GB) as an operand: A(i, j) = r[i] + c[j] with small
    integers, built on the device by two broadcast strided copies and an elementwise add over
    2.4 G elements. Then A B and A^T B2 on the MFMA tiles, A x on the thin path and a row argmax,
    each against its closed form (integer sums below 2^24: exact in fp32 in any order)."""
    m, k, n = 60000, 40000, 64
    rng = np.random.default_rng(7)
    r = rng.integers(0, 4, m).astype(np.float32)
    c = rng.integers(0, 4, k).astype(np.float32)
    c[rng.integers(0, k)] = 5.0  # a single column maximum: every row's argmax
    rows = mf.strided_copy(dev(r, stream).view((m, 1)).expand((m, k)))
    cols = mf.strided_copy(dev(c, stream).view((1, k)).expand((m, k)))
    a = mf.elementwise(mf.abi.EW_ADD, rows, cols)
    rows.close()
    cols.close()
    # Spot checks of the built matrix, including its last elements (offset > 2^31).
    for lo in (0, m // 2, m - 2):
        assert np.array_equal(a.slice(0, lo, lo + 2).numpy(), r[lo:lo + 2, None] + c[None, :]), lo

    b = rng.integers(0, 2, (k, n)).astype(np.float32)
    want = (r.astype(np.float64)[:, None] * b.sum(0)[None, :] + (c.astype(np.float64) @ b))
    got = mf.gemm(a, dev(b, stream)).numpy()
    assert same_bits(got, want.astype(np.float32))

    b2 = rng.integers(0, 2, (m, n)).astype(np.float32)
    want_t = ((r.astype(np.float64) @ b2)[None, :] + c.astype(np.float64)[:, None] * b2.sum(0))
    got_t = mf.gemm(a.T, dev(b2, stream)).numpy()
    assert same_bits(got_t, want_t.astype(np.float32))

    x = rng.integers(0, 2, (k, 1)).astype(np.float32)
    plan = mf.gemm_plan(a, dev(x, stream), mf.DeviceArray.empty((m, 1), stream))
    assert plan[0] == mf.abi.TILE_THIN
    want_x = r.astype(np.float64) * x.sum() + float(c.astype(np.float64) @ x[:, 0])
    assert same_bits(mf.gemm(a, dev(x, stream)).numpy()[:, 0], want_x.astype(np.float32))

    assert np.all(mf.argmax(a).numpy() == int(np.argmax(c)))
    a.close()


def test_streamed_output_past_last_level_cache(stream):
    """An output over 256 MiB whose rows start on 128-byte lines is written with non-temporal
    stores (8192 x 8448 floats, 277 MB): sampled rows equal the exact product; a padded row
    stride (off the lines) takes ordinary stores and gives the same bits."""
    m, n, k = 8192, 8448, 12
    av = quarter_matrix(m, k, 111)
    bv = quarter_matrix(k, n, 112)
    a_d, b_d = dev(av, stream), dev(bv, stream)
    c = mf.DeviceArray.empty((m, n), stream)
    mf.gemm(a_d, b_d, alpha=0.5, out=c)
    wide = mf.DeviceArray.empty((m, n + 1), stream)
    mf.gemm(a_d, b_d, alpha=0.5, out=wide.slice(1, 0, n))
    for lo in (0, 4096, m - 3):
        rows = slice(lo, lo + 3)
        want = (np.float32(0.5) * (av[rows].astype(np.float64) @ bv.astype(np.float64))
                .astype(np.float32))
        assert same_bits(c.slice(0, lo, lo + 3).numpy(), want), lo
        assert same_bits(wide.slice(0, lo, lo + 3).numpy()[:, :n], want), lo
    c.close()
    wide.close()
