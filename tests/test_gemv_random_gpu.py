"""Seeded random sweep of mfr_sgemv and mfr_smatvec: N and T forms, ragged sizes (around the N
form's 8-row groups and the T form's 256-column strips and row chunks), leading dimensions wider
than cols (multiples of 4 or not), A, x, y0 and y starting off a 16-byte boundary (views one
element into their storage), alpha, beta with and without y0. Quarter-integer inputs make every
double sum exact, so the result must equal the oracle's (double accumulation, one rounding) in
every bit; y sits between poisoned guard elements, which must survive."""
import numpy as np
import pytest

import mensurflow_amd as mf
from helpers import same_bits

pytestmark = pytest.mark.gpu

CASES = 150
POISON = np.float32(123.0)


def quarters(rng, shape):
    return (rng.integers(-16, 17, size=shape).astype(np.float32) / 4).astype(np.float32)


def vector(rng, stream, values):
    """A device vector view, one element into its storage half of the time."""
    shift = int(rng.integers(0, 2))
    stored = np.concatenate([np.full(shift, -77.0, np.float32), values])
    return mf.DeviceArray.from_numpy(stored, stream).slice(0, shift, shift + values.size)


@pytest.mark.parametrize("index", range(CASES))
def test_random_gemv_exact(stream, oracle, index):
    rng = np.random.default_rng(3000 + index)
    big = index % 10 == 9
    rows = int(rng.integers(1, 6000 if big else 700))
    cols = int(rng.integers(1, 6000 if big else 700))
    if index % 7 == 3:
        rows = int(rng.integers(1, 9))  # short T sums / a few N rows
    trans = bool(rng.random() < 0.5)
    pad = int(rng.choice([0, 0, 1, 3, 4, 8]))
    shift = int(rng.integers(0, 2))
    alpha = float(rng.choice([1.0, 2.0, -0.5]))
    beta = float(rng.choice([0.0, 0.5, -1.0]))
    use_y0 = beta != 0.0 or rng.random() < 0.5
    matvec = not trans and alpha == 1.0 and beta == 0.0 and rng.random() < 0.5
    what = (f"case {index}: {rows}x{cols} trans={trans} ld={cols + pad} shift={shift} "
            f"alpha={alpha} beta={beta} y0={use_y0} matvec={matvec}")

    a = quarters(rng, (rows, cols))
    stored = np.full((rows * (cols + pad) + shift,), -77.0, np.float32)
    stored[shift:].reshape(rows, cols + pad)[:, :cols] = a
    a_d = (mf.DeviceArray.from_numpy(stored, stream).slice(0, shift, stored.size)
           .view((rows, cols + pad)).slice(1, 0, cols))
    n_in, n_out = (rows, cols) if trans else (cols, rows)
    x = quarters(rng, (n_in,))
    y0 = quarters(rng, (n_out,)) if use_y0 else None
    y_buf = mf.DeviceArray.from_numpy(np.full(n_out + 2, POISON, np.float32), stream)
    y_d = y_buf.slice(0, 1, 1 + n_out)

    if matvec:
        mf.matvec(a_d, vector(rng, stream, x), out=y_d)
        want = oracle.matvec(a, x)
    else:
        mf.sgemv(a_d, vector(rng, stream, x), alpha=alpha,
                 y0=None if y0 is None else vector(rng, stream, y0), beta=beta, trans=trans,
                 out=y_d)
        want = oracle.gemv(a, x, alpha, y0, beta if y0 is not None else 0.0, trans=trans)
    got = y_buf.numpy()
    assert got[0] == POISON and got[-1] == POISON, what + ": write outside y"
    assert same_bits(got[1:-1], want), what
