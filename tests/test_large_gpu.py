"""Index arithmetic past 2^31 elements: element offsets that overflow int32 and byte offsets past
2^32, in gemv N and T over A [3, 2^30 + 4] (3.2 G elements, 12.9 GB) and in a GEMM whose output
has more than 2^31 elements. Inputs are built on the device (row-wise constants, quarter
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
