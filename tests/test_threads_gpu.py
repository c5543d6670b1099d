"""Several host threads calling one stream at once.

A backend hands every thread the same stream of a device, and gemv's transposed form and the
GEMM's split-K and staging put partial results in that stream's workspace, which a call grows
(freeing the old buffer) when it needs more. These tests start threads whose calls need growing
workspace sizes on a fresh stream, all at once, and check every result against the same calls
made one at a time on another fresh stream (gemv and a fixed split count are deterministic, so
the bits must match).
"""
import threading

import numpy as np
import pytest

import mensurflow_amd as mf
from helpers import same_bits, uniform

pytestmark = pytest.mark.gpu

THREADS = 8
ROUNDS = 4


def _run_threads(work):
    barrier = threading.Barrier(len(work))
    errors = []

    def body(fn):
        try:
            barrier.wait()
            for _ in range(ROUNDS):
                fn()
        except Exception as exc:  # reported below; a thread cannot raise into pytest
            errors.append(exc)

    threads = [threading.Thread(target=body, args=(fn,)) for fn in work]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


def test_gemv_t_from_many_threads(oracle):
    cols = 4096
    cases = [(1024 * (i + 1), cols) for i in range(THREADS)]  # workspace grows with the rows
    host = [(uniform(oracle, (r, c), -1.0, 1.0, 300 + i), uniform(oracle, (r,), -1.0, 1.0, 400 + i))
            for i, (r, c) in enumerate(cases)]
    results = {}
    for mode in ("threads", "serial"):
        print(f"threads: gemv T, {mode}", flush=True)
        with mf.Stream(0) as s:
            dev = [(mf.DeviceArray.from_numpy(a, s), mf.DeviceArray.from_numpy(x, s))
                   for a, x in host]
            outs = [mf.DeviceArray.empty((cols,), s) for _ in cases]
            work = [lambda i=i: mf.sgemv(dev[i][0], dev[i][1], alpha=2.0, trans=True, out=outs[i])
                    for i in range(len(cases))]
            if mode == "threads":
                _run_threads(work)
            else:
                for fn in work:
                    fn()
            results[mode] = [o.numpy() for o in outs]
    for i, (got, want) in enumerate(zip(results["threads"], results["serial"])):
        assert same_bits(got, want), f"gemv T case {i} differs when called from threads"


def test_split_gemm_from_many_threads(oracle):
    # Fixed split counts, growing partial-sum sizes; odd row strides are staged as well.
    cases = [(128 + 64 * i, 96 + 32 * i, 2048 + 1) for i in range(THREADS)]
    host = [(uniform(oracle, (m, k), -1.0, 1.0, 500 + i), uniform(oracle, (k, n), -1.0, 1.0, 600 + i))
            for i, (m, n, k) in enumerate(cases)]
    results = {}
    for mode in ("threads", "serial"):
        print(f"threads: split gemm, {mode}", flush=True)
        with mf.Stream(0) as s:
            dev = [(mf.DeviceArray.from_numpy(a, s), mf.DeviceArray.from_numpy(b, s))
                   for a, b in host]
            outs = [mf.DeviceArray.empty((m, n), s) for m, n, _ in cases]
            work = [lambda i=i: mf.gemm(dev[i][0], dev[i][1], out=outs[i], splits=4, stage=2)
                    for i in range(len(cases))]
            if mode == "threads":
                _run_threads(work)
            else:
                for fn in work:
                    fn()
            results[mode] = [o.numpy() for o in outs]
    for i, (got, want) in enumerate(zip(results["threads"], results["serial"])):
        assert same_bits(got, want), f"split gemm case {i} differs when called from threads"


def test_large_copies_from_several_threads():
    """Host threads each moving a little over 24 MiB to the device and back, at once, each on a
    stream of its own. The CPU side of a staged copy is split over the library's helper threads
    when they are free and done by the calling thread alone when another copy holds them; either
    way every byte comes back, from and to odd host addresses, in every round."""
    streams = [mf.Stream(0) for _ in range(THREADS)]
    rngs = [np.random.default_rng(100 + t) for t in range(THREADS)]
    try:
        def copier(t):
            def fn():
                n = (24 << 20) + 4093 * t
                data = rngs[t].integers(0, 256, n + 1, dtype=np.uint8)[1:]  # an odd address
                buf = mf.DeviceArray.empty((n,), streams[t], dtype=np.uint8)
                buf.upload(data)
                back = buf.numpy()
                assert np.array_equal(back, data), f"thread {t}"
            return fn

        _run_threads([copier(t) for t in range(THREADS)])
    finally:
        for s in streams:
            s.close()
