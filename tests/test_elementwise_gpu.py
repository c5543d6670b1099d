"""GPU parity of the elementwise, softmax, argmax and layout kernels against the vectors the
reference's own kernels wrote (tests/golden/ref_vectors.npz) and the oracle.

bias_add, where, argmax and the tanh gelu must match bit for bit (the tanh gelu's exp and
division are this library's own, checked on the CPU over every float input). The erf gelu and
softmax call the device library's erfc and exp, which may differ from glibc in the last bit
before the final rounding, so they are held to a few ulps and must be bit-identical on almost
every element."""
import os

import numpy as np
import pytest

import mensurflow_amd as mf
from helpers import normal, same_bits, uniform

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def vectors():
    with np.load(os.path.join(GOLDEN, "ref_vectors.npz"), allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def dev(x, stream):
    return mf.DeviceArray.from_numpy(np.ascontiguousarray(x), stream)


def ulp_diff(a, b):
    """Distance in units in the last place between float32 arrays (NaN == NaN)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    d = np.abs(ia - ib)
    return np.where(both_nan, 0, d)


def test_bias_add_and_where_bit_exact(stream, vectors):
    v = vectors
    got = mf.bias_act(dev(v["bias_x"], stream), dev(v["bias_b"], stream)).numpy()
    assert same_bits(got, v["bias_out"])
    got = mf.where(dev(v["where_c"], stream), dev(v["where_x"], stream),
                   dev(v["where_y"], stream)).numpy()
    assert same_bits(got, v["where_out"])


@pytest.mark.parametrize("rows,cols", [(7, 11), (4093, 4099), (64, 256)])
def test_bias_add_shapes(stream, oracle, rows, cols):
    x = normal(oracle, (rows, cols), 0.0, 1.0, 3, 0)
    b = uniform(oracle, (cols,), -0.1, 0.1, 4, 0)
    got = mf.bias_act(dev(x, stream), dev(b, stream)).numpy()
    assert same_bits(got, oracle.bias_add(x, b))


@pytest.mark.parametrize("act,key", [(mf.ACT_GELU_TANH, "gelu_tanh"), (mf.ACT_GELU_ERF, "gelu_erf")])
def test_gelu_against_reference_vectors(stream, vectors, act, key):
    x = vectors["gelu_x"]
    got = mf.bias_act(dev(x, stream), None, act).numpy()
    want = vectors[key]
    if act == mf.ACT_GELU_TANH:
        assert same_bits(got, want)
        return
    d = ulp_diff(got, want)
    assert int(d.max()) <= 2, f"max ulp difference {int(d.max())}"
    assert float(np.mean(d == 0)) > 0.995
    # the special values exactly: +-inf, NaN, signed zeros
    special = ~np.isfinite(x) | (x == 0)
    assert same_bits(got[special], want[special])


def test_gelu_tanh_every_61st_float(stream, oracle):
    """Every 61st float bit pattern (70 M inputs: all exponents, signs, subnormals, infinities
    and NaNs) through the device's tanh gelu: the oracle's bits on every one (NaN for NaN)."""
    bits = (np.arange(0, 1 << 32, 61, dtype=np.uint64)).astype(np.uint32)
    x = bits.view(np.float32)
    got = mf.bias_act(dev(x, stream), None, mf.ACT_GELU_TANH).numpy()
    want = oracle.gelu(x, approximate=True)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_gelu_known_value(stream):
    got = mf.bias_act(dev(np.array([1.0], np.float32), stream), None, mf.ACT_GELU_ERF).numpy()
    assert abs(float(got[0]) - 0.841344746) < 1e-7


def test_fused_bias_gelu_matches_chain(stream, oracle):
    x = normal(oracle, (300, 257), 0.0, 2.0, 5, 0)
    b = uniform(oracle, (257,), -0.1, 0.1, 6, 0)
    got = mf.bias_act(dev(x, stream), dev(b, stream), mf.ACT_GELU_TANH).numpy()
    want = oracle.gelu(oracle.bias_add(x, b), approximate=True)
    assert same_bits(got, want)


def test_softmax_against_reference_vectors(stream, vectors):
    v = vectors
    got = mf.softmax(dev(v["softmax_x"], stream)).numpy()
    want = v["softmax_last"]
    assert int(ulp_diff(got, want).max()) <= 4
    assert np.all(got[1] == 0.0)           # fully masked line
    assert np.all(np.isnan(got[3]))        # a NaN poisons its line
    got3 = mf.softmax(dev(v["softmax3_x"], stream), axis=1).numpy()
    assert int(ulp_diff(got3, v["softmax3_axis1"]).max()) <= 4


@pytest.mark.parametrize("length", [1, 63, 64, 257, 1024, 2048, 5000])
def test_softmax_rows(stream, oracle, length):
    x = normal(oracle, (33, length), 0.0, 4.0, length, 0)
    x[5, : length // 2] = -np.inf
    got = mf.softmax(dev(x, stream)).numpy()
    want = oracle.softmax(x)
    assert int(ulp_diff(got, want).max()) <= 4
    np.testing.assert_allclose(got.sum(axis=1, dtype=np.float64), 1.0, rtol=1e-5)


def test_argmax_bit_exact(stream, vectors, oracle):
    got = mf.argmax(dev(vectors["argmax_x"], stream)).numpy()
    assert got.tolist() == vectors["argmax_out"].tolist()
    x = normal(oracle, (1000, 4099), 0.0, 1.0, 77, 0)
    x[3, 100] = np.nan
    x[4, :] = 1.0
    assert mf.argmax(dev(x, stream)).numpy().tolist() == oracle.argmax(x).tolist()


@pytest.mark.parametrize("n", [1, 3, 4, 5, 8, 1023, 4096, 4099, (1 << 20) + 3])
@pytest.mark.parametrize("offset", [0, 1, 3])
def test_where_and_binary_sizes_and_alignment(stream, n, offset):
    """where, add, sub, mul and scal bit for bit against numpy on every size class (multiples of 4 go
    through the 16-byte streaming kernels, the rest of n through the scalar ones) and on views
    starting 1 or 3 elements into their buffers (misaligned: the scalar kernels only)."""
    rng = np.random.default_rng(n + offset)
    xs = rng.standard_normal(n + offset).astype(np.float32)
    ys = rng.standard_normal(n + offset).astype(np.float32)
    cs = (rng.random(n + offset) < 0.5).astype(np.uint8)
    x = dev(xs, stream).slice(0, offset, offset + n)
    y = dev(ys, stream).slice(0, offset, offset + n)
    c = dev(cs, stream).slice(0, offset, offset + n)
    xv, yv, cv = xs[offset:], ys[offset:], cs[offset:]
    assert same_bits(mf.where(c, x, y).numpy(), np.where(cv != 0, xv, yv))
    abi = mf.abi
    assert same_bits(mf.elementwise(abi.EW_ADD, x, y).numpy(), xv + yv)
    assert same_bits(mf.elementwise(abi.EW_MUL, x, y).numpy(), xv * yv)
    assert same_bits(mf.elementwise(abi.EW_SUB, x, y).numpy(), xv - yv)
    assert same_bits(mf.elementwise(abi.EW_SCAL, x, alpha=-1.5).numpy(), np.float32(-1.5) * xv)


def test_strided_copy_views(stream, oracle):
    base = uniform(oracle, (6, 7, 9), -1.0, 1.0, 88, 0)
    d = dev(base, stream)
    assert same_bits(d.transpose(0, 2).numpy(), np.ascontiguousarray(base.transpose(2, 1, 0)))
    assert same_bits(d.slice(1, 2, 6).numpy(), np.ascontiguousarray(base[:, 2:6, :]))
    row = dev(base[0, 0], stream).expand((4, 9))
    assert same_bits(row.numpy(), np.broadcast_to(base[0, 0], (4, 9)).copy())
    mask = dev(np.tril(np.ones((5, 5), np.uint8)), stream).expand((2, 3, 5, 5))
    assert same_bits(mask.numpy(), np.broadcast_to(np.tril(np.ones((5, 5), np.uint8)),
                                                   (2, 3, 5, 5)).copy())


def test_strided_copy_fast_paths(stream, oracle):
    """The two fast paths of the strided copy, against numpy: a source whose strides are all 0
    (a broadcast scalar), and rows with a unit stride, copied in 16-byte units when every row
    start and length allow it (a slice of a 304-wide matrix, an expanded byte mask) and element
    by element otherwise (odd strides and lengths, a middle broadcast dimension)."""
    for value, dtype in ((3.5, np.float32), (7, np.uint8), (-2, np.int64)):
        scalar = dev(np.array([value], dtype), stream)
        got = scalar.view((1, 1)).expand((3, 1000)).numpy()
        assert got.dtype == dtype and np.all(got == dtype(value))
    base = uniform(oracle, (50, 304), -1.0, 1.0, 91, 0)
    d = dev(base, stream)
    assert same_bits(d.slice(1, 4, 260).numpy(), np.ascontiguousarray(base[:, 4:260]))
    assert same_bits(d.slice(1, 3, 259).numpy(), np.ascontiguousarray(base[:, 3:259]))
    mask = (np.arange(100 * 100).reshape(100, 100) % 3 == 0).astype(np.uint8)
    expanded = dev(mask, stream).expand((2, 3, 100, 100)).numpy()
    assert same_bits(expanded, np.broadcast_to(mask, (2, 3, 100, 100)).copy())
    wide_bytes = (np.arange(7 * 2000) % 251).astype(np.uint8).reshape(7, 2000)
    assert same_bits(dev(wide_bytes, stream).slice(1, 5, 1006).numpy(),
                     np.ascontiguousarray(wide_bytes[:, 5:1006]))
    x = uniform(oracle, (4, 1, 300), -1.0, 1.0, 92, 0)
    assert same_bits(dev(x, stream).expand((4, 5, 300)).numpy(),
                     np.broadcast_to(x, (4, 5, 300)).copy())


def test_strided_copy_transposes(stream, oracle):
    """Transposed views (a strided last dimension, an earlier one contiguous) go through LDS
    tiles: 2-D with ragged edges, a batch of transposes, a transpose of a slice, one-byte,
    four-byte and eight-byte elements, and a broadcast last dimension; all against numpy."""
    base = uniform(oracle, (1000, 777), -1.0, 1.0, 93, 0)
    assert same_bits(dev(base, stream).T.numpy(), np.ascontiguousarray(base.T))
    batch = uniform(oracle, (3, 67, 130), -1.0, 1.0, 94, 0)
    got = dev(batch, stream).transpose(-2, -1).numpy()
    assert same_bits(got, np.ascontiguousarray(batch.transpose(0, 2, 1)))
    got = dev(batch, stream).transpose(0, 2).numpy()          # (130, 67, 3) from (3, 67, 130)
    assert same_bits(got, np.ascontiguousarray(batch.transpose(2, 1, 0)))
    wide = uniform(oracle, (90, 300), -1.0, 1.0, 95, 0)
    got = dev(wide, stream).slice(1, 17, 281).T.numpy()      # a slice, then transposed
    assert same_bits(got, np.ascontiguousarray(wide[:, 17:281].T))
    mask = (np.arange(300 * 200).reshape(300, 200) % 7 == 0).astype(np.uint8)
    assert same_bits(dev(mask, stream).T.numpy(), np.ascontiguousarray(mask.T))
    ints = np.arange(64 * 100, dtype=np.int64).reshape(64, 100)
    got = dev(ints, stream).T.numpy()
    assert got.dtype == np.int64 and np.array_equal(got, np.ascontiguousarray(ints.T))
    col = uniform(oracle, (200, 1), -1.0, 1.0, 96, 0)
    got = dev(col, stream).expand((200, 40)).numpy()           # last dimension broadcast
    assert same_bits(got, np.broadcast_to(col, (200, 40)).copy())


@pytest.mark.parametrize("count", [4, 1000, 2048 * 4 + 4, 4096 * 2048 * 4 + 12, 3, 8191])
def test_contiguous_copy_sizes(stream, count):
    """The contiguous fast path (16-byte units, one chunk per workgroup): a single unit, tails
    after the unrolled steps, more chunks than workgroups, and byte counts that are not
    multiples of 16 (the runtime's copy); output between guard bands."""
    src = np.arange(count, dtype=np.float32) * np.float32(0.5) - np.float32(7.0)
    buf = mf.DeviceArray.empty((count + 64,), stream)
    mf.fill(buf, 99.0)
    out = buf.slice(0, 32, 32 + count)
    mf.strided_copy(dev(src, stream), out=out)
    host = buf.numpy()
    assert same_bits(host[32:32 + count], src)
    assert np.all(host[:32] == 99.0) and np.all(host[32 + count:] == 99.0)


def test_fill(stream):
    buf = mf.DeviceArray.empty((1001,), stream)
    mf.fill(buf, -np.inf)
    assert np.all(buf.numpy() == -np.inf)
    ints = mf.DeviceArray.empty((77,), stream, np.int64)
    mf.fill(ints, -5)
    assert np.all(ints.numpy() == -5)


@pytest.mark.parametrize("case", range(12))
def test_where_nd_broadcast_views(stream, oracle, case):
    """mfr_where_nd reads each operand through its strides (0 where it broadcasts): seeded shapes
    with broadcast, sliced and transposed operands, rows that do and do not take 16-byte
    accesses, against the oracle's where on the packed operands, bit for bit."""
    rng = np.random.default_rng(900 + case)
    nd = int(rng.integers(1, 5))
    shape = tuple(int(rng.integers(1, 9)) for _ in range(nd - 1)) + (int(rng.choice([1, 3, 4, 8, 64, 130, 1024])),)
    print(f"where_nd case {case}: shape {shape}", flush=True)

    def operand(dtype, seed):
        kind = case % 3 if seed != 2 else (case // 3) % 3
        if kind == 0:  # full, packed
            host = rng.standard_normal(shape).astype(dtype) if dtype == np.float32 else \
                (rng.random(shape) > 0.5).astype(np.uint8)
            return host, dev(host, stream)
        if kind == 1:  # broadcast: extent 1 in random dimensions, then expanded
            small = tuple(1 if rng.random() < 0.5 else s for s in shape)
            host = rng.standard_normal(small).astype(dtype) if dtype == np.float32 else \
                (rng.random(small) > 0.5).astype(np.uint8)
            return np.broadcast_to(host, shape), dev(host, stream).expand(shape)
        # a slice of a wider array (row stride past the row length)
        wide = shape[:-1] + (shape[-1] + 3,)
        host = rng.standard_normal(wide).astype(dtype) if dtype == np.float32 else \
            (rng.random(wide) > 0.5).astype(np.uint8)
        return host[..., 1:1 + shape[-1]], dev(host, stream).slice(len(shape) - 1, 1, 1 + shape[-1])

    x_host, x = operand(np.float32, 0)
    y_host, y = operand(np.float32, 1)
    c_host, c = operand(np.uint8, 2)
    out = mf.where_nd(c, x, y, out=mf.DeviceArray.empty(shape, stream))
    want = oracle.where(np.ascontiguousarray(c_host), np.ascontiguousarray(x_host),
                        np.ascontiguousarray(y_host))
    assert same_bits(out.numpy(), want.reshape(shape))


def test_where_nd_attention_mask_shape(stream):
    """The composed attention's call: scores [2, 3, 64, 96], a -inf scalar and a [64, 96] mask
    expanded over the batch."""
    rng = np.random.default_rng(7)
    scores = rng.standard_normal((2, 3, 64, 96)).astype(np.float32)
    keep = np.tril(np.ones((64, 96), np.uint8))
    s_d = dev(scores, stream)
    minus_inf = dev(np.array([-np.inf], np.float32), stream)
    out = mf.where_nd(dev(keep, stream).expand(scores.shape), s_d, minus_inf.expand(scores.shape),
                      out=s_d)
    want = np.where(np.broadcast_to(keep, scores.shape) != 0, scores, np.float32(-np.inf))
    assert same_bits(out.numpy(), want.astype(np.float32))


@pytest.mark.parametrize("case", range(8))
def test_where_nd_in_place(stream, oracle, case):
    """where_nd with out being x or y itself (the same packed array): only the elements that take
    the other operand are written, so the result must equal the oracle's where on the operands as
    they were. Masks dense or broadcast (a lower triangle over the last two dimensions), the other
    operand a broadcast scalar or a full array; rows of a multiple of 4 (the quad kernel) and not
    (the generic one)."""
    shapes = [(2, 3, 64, 96), (5, 130), (4, 1024), (3, 7, 8), (2, 2, 6, 3), (1, 4), (16, 256),
              (3, 5, 12)]
    shape = shapes[case]
    rng = np.random.default_rng(950 + case)
    alias_x = case % 2 == 0
    print(f"where_nd in place case {case}: shape {shape}, out is {'x' if alias_x else 'y'}",
          flush=True)
    base = rng.standard_normal(shape).astype(np.float32)
    if case % 3 == 0 and len(shape) >= 2:
        keep = np.tril(np.ones(shape[-2:], np.uint8))
        c_host, c = np.broadcast_to(keep, shape), dev(keep, stream).expand(shape)
    else:
        c_host = (rng.random(shape) > 0.5).astype(np.uint8)
        c = dev(c_host, stream)
    if case % 4 < 2:
        scalar = np.array([-np.inf], np.float32)
        o_host, other = np.broadcast_to(scalar, shape), dev(scalar, stream).expand(shape)
    else:
        o_host = rng.standard_normal(shape).astype(np.float32)
        other = dev(o_host, stream)
    out = dev(base, stream)
    if alias_x:
        got = mf.where_nd(c, out, other, out=out)
        want = oracle.where(np.ascontiguousarray(c_host), base, np.ascontiguousarray(o_host))
    else:
        got = mf.where_nd(c, other, out, out=out)
        want = oracle.where(np.ascontiguousarray(c_host), np.ascontiguousarray(o_host), base)
    assert same_bits(got.numpy(), want.reshape(shape))
