"""The C ABI's smaller entry points on the device, called through ctypes as a C caller would:
mfr_sgemm_rm (BLAS-style row-major form, every transpose pair, leading dimensions wider than the
matrices, C0 in place), mfr_stream_wrap (a wrapped HIP stream runs work and is left alive by
mfr_stream_destroy), mfr_stream_device, mfr_memcpy_d2d and the events."""
import ctypes

import numpy as np
import pytest

import mensurflow_amd as mf
from mensurflow_amd import abi
from helpers import quarter_matrix, same_bits

pytestmark = pytest.mark.gpu


def dev(x, stream):
    return mf.DeviceArray.from_numpy(np.ascontiguousarray(x), stream)


@pytest.mark.parametrize("trans_a,trans_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_rm_every_transpose(stream, trans_a, trans_b):
    m, n, k = 130, 75, 97
    av = quarter_matrix(m, k, 11)
    bv = quarter_matrix(k, n, 12)
    c0v = quarter_matrix(m, n, 13)
    # Stored operands: A [m, k] or A^T [k, m], rows padded by 3; B likewise; C rows padded by 5.
    a_st = np.ascontiguousarray(av.T if trans_a else av)
    b_st = np.ascontiguousarray(bv.T if trans_b else bv)
    lda, ldb, ldc = a_st.shape[1] + 3, b_st.shape[1] + 3, n + 5
    a_pad = np.zeros((a_st.shape[0], lda), np.float32)
    a_pad[:, :a_st.shape[1]] = a_st
    b_pad = np.zeros((b_st.shape[0], ldb), np.float32)
    b_pad[:, :b_st.shape[1]] = b_st
    c_pad = np.full((m, ldc), 123.0, np.float32)
    c_pad[:, :n] = c0v
    a_d, b_d, c_d = dev(a_pad, stream), dev(b_pad, stream), dev(c_pad, stream)
    lib = abi.load()
    status = lib.mfr_sgemm_rm(stream.handle, trans_a, trans_b, m, n, k, ctypes.c_float(1.5),
                              ctypes.c_void_p(a_d.ptr), lda, ctypes.c_void_p(b_d.ptr), ldb,
                              ctypes.c_float(0.5), ctypes.c_void_p(c_d.ptr),
                              ctypes.c_void_p(c_d.ptr), ldc)
    abi.check(status, "mfr_sgemm_rm")
    got = c_d.numpy()
    exact = (av.astype(np.float64) @ bv.astype(np.float64)).astype(np.float32)
    want = (np.float32(1.5) * exact + np.float32(0.5) * c0v).astype(np.float32)
    assert same_bits(got[:, :n], want)
    assert np.all(got[:, n:] == 123.0), "write into the padding columns"


def test_stream_wrap_device_memcpy_and_events(stream):
    lib = abi.load()
    assert lib.mfr_stream_device(stream.handle) == stream.device
    wrapped = ctypes.c_void_p()
    abi.check(lib.mfr_stream_wrap(stream.device, ctypes.c_void_p(stream.hip_stream()),
                                  ctypes.byref(wrapped)), "mfr_stream_wrap")
    try:
        src = dev(np.arange(1000, dtype=np.float32), stream)
        dst = mf.DeviceArray.empty((1000,), stream)
        start, end = mf.Event(), mf.Event()
        abi.check(lib.mfr_event_record(start.handle, wrapped), "mfr_event_record")
        abi.check(lib.mfr_memcpy_d2d(wrapped, ctypes.c_void_p(dst.ptr), ctypes.c_void_p(src.ptr),
                                     4000), "mfr_memcpy_d2d")
        # A product on the wrapped stream (the same HIP stream), then the events.
        a = dev(quarter_matrix(40, 30, 21), stream)
        b = dev(quarter_matrix(30, 20, 22), stream)
        c = mf.DeviceArray.empty((40, 20), stream)
        desc = mf._gemm_desc(a, b, c, 1.0, None, 0.0, None, mf.ACT_NONE, 0, 0)
        abi.check(lib.mfr_sgemm(wrapped, ctypes.byref(desc)), "mfr_sgemm")
        abi.check(lib.mfr_event_record(end.handle, wrapped), "mfr_event_record")
        abi.check(lib.mfr_stream_sync(wrapped), "mfr_stream_sync")
        assert np.array_equal(dst.numpy(), np.arange(1000, dtype=np.float32))
        want = (quarter_matrix(40, 30, 21).astype(np.float64) @
                quarter_matrix(30, 20, 22).astype(np.float64)).astype(np.float32)
        assert same_bits(c.numpy(), want)
        assert start.elapsed_ms(end) >= 0.0
    finally:
        abi.check(lib.mfr_stream_destroy(wrapped), "mfr_stream_destroy")
    # The wrapped HIP stream belongs to `stream`, which still works.
    x = dev(np.ones(8, np.float32), stream)
    mf.fill(x, 2.0)
    assert np.all(x.numpy() == 2.0)


@pytest.mark.parametrize("nbytes", [1, 4093, (1 << 20) - 1, 1 << 20, (16 << 20) - 3, 16 << 20,
                                    (16 << 20) + 5, (32 << 20) + 1, (41 << 20) + 7])
def test_host_copies_every_size_around_the_staging_chunks(stream, nbytes):
    """mfr_memcpy_h2d and mfr_memcpy_d2h from and to pageable memory: 1 MiB and more go through
    the stream's two pinned staging slots in 16 MiB chunks, less goes directly. Every size around
    the chunk edges, from and to odd host addresses, comes back byte for byte; the device bytes
    are also read back through a device-to-device copy into a second buffer, and a second upload
    of other bytes overwrites the first completely (the slots are reused across calls)."""
    lib = abi.load()
    rng = np.random.default_rng(nbytes)
    first = rng.integers(0, 256, nbytes + 3, dtype=np.uint8)[3:]   # an odd host address
    second = rng.integers(0, 256, nbytes + 1, dtype=np.uint8)[1:]
    buf = mf.DeviceArray.empty((nbytes,), stream, dtype=np.uint8)
    other = mf.DeviceArray.empty((nbytes,), stream, dtype=np.uint8)
    for want in (first, second):
        abi.check(lib.mfr_memcpy_h2d(stream.handle, ctypes.c_void_p(buf.ptr),
                                     want.ctypes.data, nbytes), "mfr_memcpy_h2d")
        back = np.empty(nbytes + 5, np.uint8)
        view = back[5:]                                                  # an odd host address
        back[:5] = 7
        abi.check(lib.mfr_memcpy_d2h(stream.handle, view.ctypes.data, ctypes.c_void_p(buf.ptr),
                                     nbytes), "mfr_memcpy_d2h")
        assert np.array_equal(view, want)
        assert np.all(back[:5] == 7), "the copy wrote before its destination"
        abi.check(lib.mfr_memcpy_d2d(stream.handle, ctypes.c_void_p(other.ptr),
                                     ctypes.c_void_p(buf.ptr), nbytes), "mfr_memcpy_d2d")
        assert np.array_equal(other.numpy(), want)
    buf.close()
    other.close()


def test_released_blocks_serve_later_arrays_in_stream_order(stream):
    """A released array's block goes back to its stream without a wait and serves the stream's
    next array of the same size class. Work queued before the release still reads the old bytes:
    a 2048^3 GEMM reading A is queued, A is released, and a new array taking A's block is
    filled by an upload queued behind the GEMM; the product is exact and the new array holds
    the upload. A slightly smaller array takes the same block, and release_idle gives every idle
    block back to the device."""
    n = 2048
    av, bv = quarter_matrix(n, n, 21), quarter_matrix(n, n, 22)
    a, b = dev(av, stream), dev(bv, stream)
    c = mf.gemm(a, b)
    block = a._ptr
    a.close()
    again = dev(np.full((n, n), 3.0, np.float32), stream)
    assert again._ptr == block
    exact = (av.astype(np.float64) @ bv.astype(np.float64)).astype(np.float32)
    assert same_bits(c.numpy(), exact)
    assert np.all(again.numpy() == 3.0)
    again.close()
    smaller = mf.DeviceArray.empty((n * n - 1000,), stream)
    assert smaller._ptr == block
    smaller.close()
    assert stream._idle_bytes >= n * n * 4
    stream.release_idle()
    assert stream._idle_bytes == 0 and not stream._idle
