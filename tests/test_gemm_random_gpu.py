"""Seeded random sweep of mfr_sgemm: shapes (empty, thin, ragged, medium), operand layouts (row-
major, transposed, sliced out of wider storage), batch dimensions with broadcast operands, the
epilogue (alpha, beta with a separate or in-place C0, a bias, gelu in both forms) and the plan
settings (AUTO, every fixed tile, the thin path, staging modes, split counts).

Inputs are quarter integers, so every product sum is exact in fp32 in any order and the
pre-activation values are exact: the output must equal the exact result in every bit (the tanh
gelu is bit-exact against the oracle for every float input; the erf form, which uses the device
library's erfc, is held to 2 ulp). The output sits in a poisoned buffer with guard bands and, in
some cases, poisoned padding columns, which must survive. A point the ABI refuses
(NotImplementedError: the thin or panel path where it does not apply or with a split) must leave
the output untouched.

test_random_panel_exact draws products the panel path takes (k <= 64, a multiple of 4, both
operands read along k with aligned strides) on the fixed PANEL point and on AUTO."""
import numpy as np
import pytest

import mensurflow_amd as mf
from helpers import same_bits

pytestmark = pytest.mark.gpu

POISON = np.float32(123.0)
GUARD = 64
CASES = 400
A = mf.abi


def quarters(rng, shape):
    return (rng.integers(-16, 17, size=shape).astype(np.float32) / 4).astype(np.float32)


def ulp_diff(a, b):
    ia = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def device_operand(rng, stream, values, batch):
    """values [*b', rows, cols] (b' = 1 where the operand is broadcast) as a device view of
    shape [*batch, rows, cols] in one of four layouts; returns (view, description)."""
    rows, cols = values.shape[-2:]
    kind = int(rng.integers(0, 4))
    lead = values.shape[:-2]
    if kind in (0, 1):
        pad_r, pad_c = (0, 0) if kind == 0 else (int(rng.integers(1, 3)), int(rng.integers(1, 6)))
        stored = np.full(lead + (rows + pad_r, cols + pad_c), -77.0, np.float32)
        stored[..., :rows, :cols] = values
        view = mf.DeviceArray.from_numpy(stored, stream)
        view = view.slice(-2, 0, rows).slice(-1, 0, cols)
    else:
        pad_r, pad_c = (0, 0) if kind == 2 else (int(rng.integers(1, 6)), int(rng.integers(1, 3)))
        stored = np.full(lead + (cols + pad_c, rows + pad_r), -77.0, np.float32)
        stored[..., :cols, :rows] = np.swapaxes(values, -1, -2)
        view = mf.DeviceArray.from_numpy(stored, stream)
        view = view.slice(-2, 0, cols).slice(-1, 0, rows).transpose(-2, -1)
    if lead != batch:
        view = view.expand(batch + (rows, cols))
    return view, ["rows", "sliced", "transposed", "transposed+sliced"][kind]


def make_case(index):
    rng = np.random.default_rng(1000 + index)
    medium = index % 8 == 7
    if medium:
        m, n, k = (int(x) for x in rng.integers(300, 2200, size=3))
        batch = ()
    else:
        m, n = (int(x) for x in rng.integers(1, 300, size=2))
        k = int(rng.integers(0, 400))
        if index % 5 == 0:
            n = int(rng.integers(1, 9))  # thin candidates
        elif index % 5 == 1:
            m = int(rng.integers(1, 9))
        dims = int(rng.integers(0, 3))
        batch = tuple(int(x) for x in rng.integers(1, 4, size=dims))
    return rng, m, n, k, batch


@pytest.mark.parametrize("index", range(CASES))
def test_random_gemm_exact(stream, oracle, index):
    rng, m, n, k, batch = make_case(index)
    # Operands: each batch dimension of A or B broadcast (stride 0) with probability 1/3.
    a_lead = tuple(1 if rng.random() < 1 / 3 else s for s in batch)
    b_lead = tuple(1 if rng.random() < 1 / 3 else s for s in batch)
    av = quarters(rng, a_lead + (m, k))
    bv = quarters(rng, b_lead + (k, n))
    a_d, a_kind = device_operand(rng, stream, av, batch)
    b_d, b_kind = device_operand(rng, stream, bv, batch)

    alpha = float(rng.choice([1.0, 0.5, 1.5, -2.0]))
    beta = float(rng.choice([0.0, 0.5, -1.0]))
    c0_mode = str(rng.choice(["none", "separate", "in-place"]))
    use_bias = bool(rng.random() < 0.5)
    act = int(rng.choice([A.ACT_NONE, A.ACT_NONE, A.ACT_GELU_TANH, A.ACT_GELU_ERF]))
    tile = int(rng.choice([A.TILE_AUTO] * 6 + list(range(1, A.TILE_COUNT))))
    stage = int(rng.choice([A.STAGE_AUTO] * 3 + [A.STAGE_NEVER, A.STAGE_ALWAYS]))
    splits = int(rng.choice([0] * 6 + [1, 2, 3, 4, 8, 16]))
    pad = int(rng.integers(0, 3))  # padding columns of the output
    what = (f"case {index}: m={m} n={n} k={k} batch={batch} A[{a_kind} {a_lead}] "
            f"B[{b_kind} {b_lead}] alpha={alpha} beta={beta} c0={c0_mode} bias={use_bias} "
            f"act={act} tile={tile} stage={stage} splits={splits} pad={pad}")

    c0v = quarters(rng, batch + (m, n))
    biasv = quarters(rng, (n,))
    # Output: [*batch, m, n + pad] inside guard bands, poisoned; in place, C0 sits in it.
    size = int(np.prod(batch + (m, n + pad), dtype=np.int64))
    image = np.full(size + 2 * GUARD, POISON, np.float32)
    inner = image[GUARD:GUARD + size].reshape(batch + (m, n + pad))
    if c0_mode == "in-place":
        inner[..., :n] = c0v
    buf = mf.DeviceArray.from_numpy(image, stream)
    c_d = buf.slice(0, GUARD, GUARD + size).view(batch + (m, n + pad)).slice(-1, 0, n)
    c0_d = None
    if c0_mode == "separate":
        c0_d = mf.DeviceArray.from_numpy(c0v, stream)
    elif c0_mode == "in-place":
        c0_d = c_d
    bias_d = mf.DeviceArray.from_numpy(biasv, stream) if use_bias else None

    try:
        mf.gemm_batched(a_d, b_d, c_d, alpha=alpha, c0=c0_d, beta=beta, bias=bias_d, act=act,
                        tile=tile, stage=stage, splits=splits)
    except NotImplementedError:
        assert same_bits(buf.numpy(), image), what + ": refused, but the output changed"
        assert tile in (A.TILE_THIN, A.TILE_PANEL), what + ": refused"
        return

    got_image = buf.numpy()
    assert np.all(got_image[:GUARD] == POISON) and np.all(got_image[-GUARD:] == POISON), (
        what + ": write outside C")
    got_inner = got_image[GUARD:GUARD + size].reshape(batch + (m, n + pad))
    assert np.all(got_inner[..., n:] == POISON), what + ": write into the padding columns"
    got = got_inner[..., :n]

    exact = np.matmul(np.broadcast_to(av, batch + (m, k)).astype(np.float64),
                      np.broadcast_to(bv, batch + (k, n)).astype(np.float64)) + 0.0
    pre = exact.astype(np.float32)
    if alpha != 1.0:
        pre = np.float32(alpha) * pre
    if c0_mode != "none" and beta != 0.0:
        pre = pre + np.float32(beta) * c0v
    if use_bias:
        pre = pre + biasv
    pre = np.ascontiguousarray(pre, np.float32)
    if act == A.ACT_NONE:
        assert same_bits(got, pre), what
    elif act == A.ACT_GELU_TANH:
        assert same_bits(got, oracle.gelu(pre, approximate=True)), what
    else:
        want = oracle.gelu(pre, approximate=False)
        assert int(ulp_diff(got, want).max(initial=0)) <= 2, what


PANEL_CASES = 60


@pytest.mark.parametrize("index", range(PANEL_CASES))
def test_random_panel_exact(stream, index):
    """The panel path on random shapes (ragged edges past every panel, tile and range), batch
    dimensions with broadcast operands, aligned row strides wider than k, alpha, beta with a
    separate or in-place C0, a bias and padding columns; bits equal the exact result."""
    rng = np.random.default_rng(5000 + index)
    m = int(rng.integers(1, 700)) if index % 3 else int(rng.integers(250, 1300))
    n = int(rng.integers(1, 700))
    k = 4 * int(rng.integers(1, 17))
    dims = int(rng.integers(0, 3))
    batch = tuple(int(x) for x in rng.integers(1, 4, size=dims))
    a_lead = tuple(1 if rng.random() < 1 / 3 else s for s in batch)
    b_lead = tuple(1 if rng.random() < 1 / 3 else s for s in batch)
    av = quarters(rng, a_lead + (m, k))
    btv = quarters(rng, b_lead + (n, k))  # B stored [n, k]: read along k
    a_pad = 4 * int(rng.integers(0, 3))
    b_pad = 4 * int(rng.integers(0, 3))
    a_store = np.full(a_lead + (m, k + a_pad), -77.0, np.float32)
    a_store[..., :k] = av
    b_store = np.full(b_lead + (n, k + b_pad), -77.0, np.float32)
    b_store[..., :k] = btv
    a_d = mf.DeviceArray.from_numpy(a_store, stream).slice(-1, 0, k)
    b_d = mf.DeviceArray.from_numpy(b_store, stream).slice(-1, 0, k).transpose(-2, -1)
    if a_lead != batch:
        a_d = a_d.expand(batch + (m, k))
    if b_lead != batch:
        b_d = b_d.expand(batch + (k, n))
    alpha = float(rng.choice([1.0, 0.125, 1.5, -2.0]))
    beta = float(rng.choice([0.0, 0.5, -1.0]))
    c0_mode = str(rng.choice(["none", "separate", "in-place"]))
    use_bias = bool(rng.random() < 0.5)
    tile = int(rng.choice([A.TILE_AUTO, A.TILE_PANEL, A.TILE_PANEL]))
    pad = int(rng.integers(0, 3))
    what = (f"panel case {index}: m={m} n={n} k={k} batch={batch} A{a_lead}+{a_pad} "
            f"B{b_lead}+{b_pad} alpha={alpha} beta={beta} c0={c0_mode} bias={use_bias} "
            f"tile={tile} pad={pad}")
    c0v = quarters(rng, batch + (m, n))
    biasv = quarters(rng, (n,))
    size = int(np.prod(batch + (m, n + pad), dtype=np.int64))
    image = np.full(size + 2 * GUARD, POISON, np.float32)
    inner = image[GUARD:GUARD + size].reshape(batch + (m, n + pad))
    if c0_mode == "in-place":
        inner[..., :n] = c0v
    buf = mf.DeviceArray.from_numpy(image, stream)
    c_d = buf.slice(0, GUARD, GUARD + size).view(batch + (m, n + pad)).slice(-1, 0, n)
    c0_d = None
    if c0_mode == "separate":
        c0_d = mf.DeviceArray.from_numpy(c0v, stream)
    elif c0_mode == "in-place":
        c0_d = c_d
    bias_d = mf.DeviceArray.from_numpy(biasv, stream) if use_bias else None
    if tile == A.TILE_PANEL:
        assert mf.gemm_plan(a_d, b_d, c_d, tile=tile, c0=c0_d, beta=beta)[0] == A.TILE_PANEL
    mf.gemm_batched(a_d, b_d, c_d, alpha=alpha, c0=c0_d, beta=beta, bias=bias_d, tile=tile)
    got_image = buf.numpy()
    assert np.all(got_image[:GUARD] == POISON) and np.all(got_image[-GUARD:] == POISON), (
        what + ": write outside C")
    got_inner = got_image[GUARD:GUARD + size].reshape(batch + (m, n + pad))
    assert np.all(got_inner[..., n:] == POISON), what + ": write into the padding columns"
    exact = np.matmul(np.broadcast_to(av, batch + (m, k)).astype(np.float64),
                      np.swapaxes(np.broadcast_to(btv, batch + (n, k)), -1, -2).astype(np.float64))
    pre = (exact + 0.0).astype(np.float32)
    if alpha != 1.0:
        pre = np.float32(alpha) * pre
    if c0_mode != "none" and beta != 0.0:
        pre = pre + np.float32(beta) * c0v
    if use_bias:
        pre = pre + biasv
    assert same_bits(got_inner[..., :n], np.ascontiguousarray(pre, np.float32)), what
