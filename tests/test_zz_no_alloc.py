"""mfr_sgemm_noalloc: the GEMM entry point that allocates no device memory.

Called through the C ABI, it must give exactly mfr_sgemm's bits on products that use its fixed
scratch array (staged operands, split-K partial sums), on consecutive calls whose second input is
smaller (the array keeps the first call's contents), and refuse a product whose plan needs more
than MFR_SGEMM_SCRATCH_BYTES before launching anything. Automatic staging and splits that would
need more take the fallbacks mfr_sgemm takes without workspace memory (operands read in place,
one depth range) instead of a refusal.
"""
import ctypes

import numpy as np
import pytest

import mensurflow_amd as mf
from mensurflow_amd import abi
from helpers import normal, quarter_matrix, same_bits, uniform

pytestmark = pytest.mark.gpu


def _dev(x, stream):
    return mf.DeviceArray.from_numpy(np.ascontiguousarray(x, dtype=np.float32), stream)


def _run(entry, stream, desc):
    fn = getattr(abi.load(), entry)
    abi.check(fn(stream.handle, ctypes.byref(desc)), entry)


def _both(stream, a, b, c0=None, bias=None, *, alpha=1.0, beta=0.0, act=abi.ACT_NONE,
          splits=0, stage=abi.STAGE_AUTO, poison=np.float32(123.0)):
    """(mfr_sgemm's C, mfr_sgemm_noalloc's C, plan) for one product, each into a poisoned C."""
    m, n = a.shape[0], b.shape[1]
    outs = []
    for entry in ("mfr_sgemm", "mfr_sgemm_noalloc"):
        c = _dev(np.full((m, n), poison, np.float32), stream)
        desc = mf._gemm_desc(a, b, c, alpha, c0, beta, bias, act, 0, stage, splits)
        print(f"no_alloc: {entry} m={m} n={n} k={a.shape[1]} splits={splits}", flush=True)
        _run(entry, stream, desc)
        outs.append(c.numpy())
    plan = mf.gemm_plan(a, b, c, splits=splits, stage=stage, c0=c0, beta=beta)
    return outs[0], outs[1], plan


def test_noalloc_matches_sgemm_on_two_calls(stream, oracle):
    # Call 1: configs[3]'s MLP layer with staging asked for. X [4093, 1023] and W [1023, 4099]
    # are copied (their rows are not 16-byte multiples): 2 x ~16.8 MB of the scratch array.
    x = normal(oracle, (4093, 1023), 0.0, 1.0, 41)
    w = normal(oracle, (1023, 4099), 0.0, float(1.0 / np.sqrt(1023.0)), 42)
    bias = uniform(oracle, (4099,), -0.1, 0.1, 43)
    dx, dw, db = _dev(x, stream), _dev(w, stream), _dev(bias, stream)
    want, got, plan = _both(stream, dx, dw, bias=db, act=abi.ACT_GELU_TANH,
                            stage=abi.STAGE_ALWAYS)
    assert plan[1] == abi.STAGE_ALWAYS, plan
    assert same_bits(got, want), "call 1 (staged MLP layer) differs from mfr_sgemm"

    # Call 2, smaller: a split-K product over odd strides (staged, plus partial sums in front of
    # the staged copies), with alpha, beta * C0 in a second buffer, and a bias.
    m, n, k = 300, 260, 4100
    a = _dev(uniform(oracle, (m, k + 3), -1.0, 1.0, 51), stream).slice(1, 0, k)
    b = _dev(uniform(oracle, (k, n + 1), -1.0, 1.0, 52), stream).slice(1, 0, n)
    c0 = _dev(normal(oracle, (m, n), 0.0, 1.0, 53), stream)
    bias2 = _dev(uniform(oracle, (n,), -0.1, 0.1, 54), stream)
    want2, got2, plan2 = _both(stream, a, b, c0=c0, bias=bias2, alpha=1.5, beta=0.5, splits=4,
                               stage=abi.STAGE_ALWAYS)
    assert plan2[2] == 4, plan2
    assert plan2[1] == abi.STAGE_ALWAYS, plan2
    assert same_bits(got2, want2), "call 2 (split-K, staged, smaller) differs from mfr_sgemm"

    # Call 3: automatic splits on a long depth (partial sums only, no staging).
    a3 = _dev(uniform(oracle, (256, 16384), -1.0, 1.0, 61), stream)
    b3 = _dev(uniform(oracle, (16384, 256), -1.0, 1.0, 62), stream)
    want3, got3, plan3 = _both(stream, a3, b3)
    assert plan3[2] > 1, plan3
    assert same_bits(got3, want3), "call 3 (automatic split-K) differs from mfr_sgemm"


def test_noalloc_refuses_a_plan_above_the_maximum(stream, oracle):
    # 64 ranges of 1024 x 512 partial sums are 128 MiB, twice the scratch array.
    m, n, k = 1024, 512, 64 * 256
    a = _dev(uniform(oracle, (m, k), -1.0, 1.0, 71), stream)
    b = _dev(uniform(oracle, (k, n), -1.0, 1.0, 72), stream)
    poison = np.full((m, n), np.float32(123.0), np.float32)
    c = _dev(poison, stream)
    desc = mf._gemm_desc(a, b, c, 1.0, None, 0.0, None, abi.ACT_NONE, 0, 0, 64)
    status = abi.load().mfr_sgemm_noalloc(stream.handle, ctypes.byref(desc))
    assert status == abi.MFR_E_INVALID
    message = abi.last_error()
    assert "sgemm_noalloc" in message and str(abi.SGEMM_SCRATCH_BYTES) in message, message
    assert same_bits(c.numpy(), poison), "a refused call wrote C"
    # The same product still runs through mfr_sgemm (the stream's own workspace).
    _run("mfr_sgemm", stream, desc)
    assert np.all(np.isfinite(c.numpy()))


def test_noalloc_without_scratch_use(stream, oracle):
    # Aligned operands, no split: the plan needs no scratch at all.
    a = _dev(uniform(oracle, (512, 256), -1.0, 1.0, 81), stream)
    b = _dev(uniform(oracle, (256, 384), -1.0, 1.0, 82), stream)
    want, got, plan = _both(stream, a, b, splits=1)
    assert plan[1] == abi.STAGE_NEVER and plan[2] == 1, plan
    assert same_bits(got, want)


def test_noalloc_falls_back_to_in_place_reads_over_the_maximum(stream):
    """AUTO staging (and AUTO splits) that would need more than the scratch array: the no-alloc
    entry point reads the operands in place in one depth range instead, as mfr_sgemm does when
    its workspace cannot be had. Quarter-integer inputs make every sum exact in any order, so both
    entry points must give the exact product."""
    m, n, k = 4096, 256, 4097
    a = quarter_matrix(m, k, 91)  # rows of 4097 floats, which 16-byte loads cannot take
    b = quarter_matrix(k, n, 92)
    da, db = _dev(a, stream), _dev(b, stream)
    probe = mf.DeviceArray.empty((m, n), stream)
    plan = mf.gemm_plan(da, db, probe)
    # mfr_sgemm stages A: 4096 rows of 4100 floats, 67,174,400 bytes, just over the maximum.
    assert plan[1] == abi.STAGE_ALWAYS, plan
    assert 4 * m * 4100 > abi.SGEMM_SCRATCH_BYTES
    want = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    for entry in ("mfr_sgemm", "mfr_sgemm_noalloc"):
        c = _dev(np.full((m, n), np.float32(123.0), np.float32), stream)
        desc = mf._gemm_desc(da, db, c, 1.0, None, 0.0, None, abi.ACT_NONE, 0, abi.STAGE_AUTO, 0)
        print(f"no_alloc: {entry} m={m} n={n} k={k} over the maximum", flush=True)
        _run(entry, stream, desc)
        assert same_bits(c.numpy(), want), entry
