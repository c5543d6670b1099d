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
