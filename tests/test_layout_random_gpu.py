"""Seeded random sweeps of the layout and elementwise kernels:

- mfr_strided_copy on random views: up to 6 dimensions taken in a random order out of a
  contiguous allocation, sliced, some broadcast (stride 0), element sizes 1, 2, 4 and 8 bytes,
  against numpy's view of the same bytes; the packed destination sits between guard elements;
- mfr_where, mfr_elementwise (add, mul, scal) and mfr_bias_act (none, gelu-tanh) over random
  sizes with inputs and outputs starting off a 16-byte boundary, bit-exact against the oracle;
- mfr_softmax along a random axis (rows with -inf and NaN entries) within 4 ulp, and mfr_argmax
  (ties, NaN rows, -inf) bit-exact, against the oracle."""
import numpy as np
import pytest

import mensurflow_amd as mf
from helpers import same_bits

pytestmark = pytest.mark.gpu

DTYPES = [np.uint8, np.uint16, np.float32, np.uint64]


def ulp_diff(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.where(both_nan, 0, np.abs(ia - ib))


def shifted(stream, values, shift):
    """values on the device as a contiguous view `shift` elements into its allocation."""
    stored = np.concatenate([np.zeros(shift, values.dtype), values.ravel()])
    return (mf.DeviceArray.from_numpy(stored, stream).slice(0, shift, shift + values.size)
            .view(values.shape))


@pytest.mark.parametrize("index", range(80))
def test_random_strided_copy(stream, index):
    rng = np.random.default_rng(4000 + index)
    dtype = DTYPES[index % 4]
    ndim = int(rng.integers(1, 7))
    base_shape = tuple(int(x) for x in rng.integers(1, 10, size=ndim))
    total = int(np.prod(base_shape))
    host = rng.integers(0, 250, size=total).astype(dtype)
    base = mf.DeviceArray.from_numpy(host, stream)
    # Strides of the contiguous base, its dimensions permuted, then each dimension sliced or
    # (where it has extent 1 after slicing) broadcast.
    contiguous = np.cumprod((1,) + base_shape[::-1])[:-1][::-1]
    order = rng.permutation(ndim)
    shape, strides, offset = [], [], 0
    for dim in order:
        extent = base_shape[dim]
        start = int(rng.integers(0, extent))
        length = int(rng.integers(1, extent - start + 1))
        offset += start * int(contiguous[dim])
        if length == 1 and rng.random() < 0.5:
            shape.append(int(rng.integers(1, 6)))
            strides.append(0)
        else:
            shape.append(length)
            strides.append(int(contiguous[dim]))
    view = base._view(tuple(shape), tuple(strides), offset)
    want = np.lib.stride_tricks.as_strided(
        host[offset:], shape=tuple(shape),
        strides=tuple(s * host.itemsize for s in strides)).copy()
    n = int(np.prod(shape))
    out_buf = mf.DeviceArray.from_numpy(np.full(n + 2, 251, dtype), stream)
    out = out_buf.slice(0, 1, 1 + n).view(tuple(shape))
    mf.strided_copy(view, out=out)
    got = out_buf.numpy()
    what = f"case {index}: {np.dtype(dtype).name} shape {shape} strides {strides} offset {offset}"
    assert got[0] == 251 and got[-1] == 251, what + ": write outside the destination"
    assert np.array_equal(got[1:-1].reshape(shape), want), what


@pytest.mark.parametrize("index", range(40))
def test_random_elementwise(stream, oracle, index):
    rng = np.random.default_rng(5000 + index)
    n = int(rng.integers(1, 200000 if index % 4 == 3 else 3000))
    s = [int(x) for x in rng.integers(0, 4, size=4)]  # element shifts off 16-byte alignment
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    cond = (rng.random(n) > 0.5).astype(np.uint8)
    a_d, b_d = shifted(stream, a, s[0]), shifted(stream, b, s[1])
    what = f"case {index}: n={n} shifts {s}"

    def out_view():
        buf = mf.DeviceArray.from_numpy(np.full(n + s[3] + 1, 123.0, np.float32), stream)
        return buf, buf.slice(0, s[3], s[3] + n)

    buf, out = out_view()
    mf.where(shifted(stream, cond, s[2]), a_d, b_d, out=out)
    got = buf.numpy()
    assert got[-1] == 123.0 and same_bits(got[s[3]:s[3] + n], oracle.where(cond, a, b)), what
    alpha = np.float32(rng.uniform(-3, 3))
    for op, want in ((mf.abi.EW_ADD, a + b), (mf.abi.EW_MUL, a * b), (mf.abi.EW_SCAL, alpha * a)):
        buf, out = out_view()
        mf.elementwise(op, a_d, None if op == mf.abi.EW_SCAL else b_d, alpha=float(alpha),
                       out=out)
        got = buf.numpy()
        assert got[-1] == 123.0 and same_bits(got[s[3]:s[3] + n], want), (what, op)

    cols = min(n, int(rng.integers(1, 600)))
    rows = n // cols
    x = a[:rows * cols].reshape(rows, cols)
    bias = rng.uniform(-0.1, 0.1, cols).astype(np.float32)
    x_d = shifted(stream, x, s[0])
    bias_d = shifted(stream, bias, s[1])
    for act in (mf.ACT_NONE, mf.ACT_GELU_TANH):
        y_buf = mf.DeviceArray.from_numpy(np.full(rows * cols + s[3] + 1, 123.0, np.float32),
                                          stream)
        y = y_buf.slice(0, s[3], s[3] + rows * cols).view((rows, cols))
        mf.bias_act(x_d, bias_d, act, out=y)
        want = oracle.bias_add(x, bias)
        if act == mf.ACT_GELU_TANH:
            want = oracle.gelu(want, approximate=True)
        got = y_buf.numpy()
        assert got[-1] == 123.0, (what, act)
        assert same_bits(got[s[3]:s[3] + rows * cols].reshape(rows, cols), want), (what, act)


@pytest.mark.parametrize("index", range(40))
def test_random_softmax_and_argmax(stream, oracle, index):
    rng = np.random.default_rng(6000 + index)
    ndim = int(rng.integers(1, 4))
    shape = tuple(int(x) for x in rng.integers(1, 40 if ndim == 3 else 300, size=ndim))
    if index % 5 == 4:
        shape = shape[:-1] + (int(rng.integers(1000, 6000)),)  # long rows
    x = (rng.standard_normal(shape) * rng.uniform(0.5, 8)).astype(np.float32)
    flat = x.reshape(-1)
    picks = rng.integers(0, flat.size, size=max(1, flat.size // 50))
    flat[picks[: len(picks) // 2]] = -np.inf
    if index % 3 == 0:
        flat[picks[-1]] = np.nan
    axis = int(rng.integers(-ndim, ndim))
    what = f"case {index}: shape {shape} axis {axis}"
    got = mf.softmax(shifted(stream, x, int(rng.integers(0, 4))), axis=axis).numpy()
    assert int(ulp_diff(got, oracle.softmax(x, axis)).max(initial=0)) <= 4, what

    # argmax over the last axis: ties (values rounded to a few levels), -inf and NaN rows.
    y = np.round(x * 0.5).astype(np.float32)
    got_arg = mf.argmax(shifted(stream, y, int(rng.integers(0, 4)))).numpy()
    assert np.array_equal(got_arg, oracle.argmax(y)), what
