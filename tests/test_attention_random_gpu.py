"""Seeded random sweep of the fused attention kernel (mfr_attention) against the oracle's
restatement of the reference's composition (src/ops/attention.cpp:48-98: packed GEMM q k^T,
alpha pass, where(-inf), softmax, packed GEMM with v): every head size 16, 32, ..., 128, ragged and
empty key counts, one or two batch dimensions with k and v broadcast (512 entries in every 15th
case, which runs the 16-query kernel for causal d = 64), causal or not, no mask, a
[Lq, Lk] mask or a batched mask broadcast over heads, the default or an explicit scale, and row
strides wider than d (16-byte aligned) for q, k, v and the output. The bar is the GEMM's: max
relative error 1e-5*sqrt(Lk) of sum_j |p_ij v_jc| per output entry; rows whose keys are all
removed must be exactly zero, and padding columns of the output must stay untouched."""
import numpy as np
import pytest

import mensurflow_amd as mf
from helpers import assert_gemm_parity

pytestmark = pytest.mark.gpu

CASES = 120
POISON = np.float32(123.0)


def strided(rng, stream, values, batch):
    """values [*b', rows, d] as a device view [*batch, rows, d] whose rows are d + 4j apart."""
    rows, d = values.shape[-2:]
    pad = 4 * int(rng.integers(0, 3))
    stored = np.full(values.shape[:-1] + (d + pad,), -77.0, np.float32)
    stored[..., :d] = values
    view = mf.DeviceArray.from_numpy(stored, stream).slice(-1, 0, d)
    if values.shape[:-2] != batch:
        view = view.expand(batch + (rows, d))
    return view


@pytest.mark.parametrize("index", range(CASES))
def test_random_fused_attention(stream, oracle, index):
    rng = np.random.default_rng(2000 + index)
    d = int(rng.choice([16, 32, 48, 64, 80, 96, 112, 128]))
    batch = tuple(int(x) for x in rng.integers(1, 4, size=int(rng.integers(1, 3))))
    lq = int(rng.integers(1, 300))
    lk = 0 if index % 23 == 22 else int(rng.integers(1, 300))
    causal = bool(rng.random() < 0.5)
    mask_kind = str(rng.choice(["none", "2d", "batched"]))
    scale = 0.0 if rng.random() < 0.5 else float(np.float32(rng.uniform(0.05, 0.5)))
    if index % 15 == 14:
        # 512 batch entries, causal, d = 64, no mask: a grid large enough for the 16-query
        # kernel (one 256-query workgroup per CU, longest first).
        d, batch, causal, mask_kind, lk = 64, (32, 16), True, "none", max(lk, 1)
    kv_lead = tuple(1 if rng.random() < 1 / 3 else s for s in batch)
    what = (f"case {index}: d={d} batch={batch} lq={lq} lk={lk} causal={causal} "
            f"mask={mask_kind} scale={scale} kv={kv_lead}")

    q = rng.standard_normal(batch + (lq, d)).astype(np.float32)
    k = rng.standard_normal(kv_lead + (lk, d)).astype(np.float32)
    v = rng.standard_normal(kv_lead + (lk, d)).astype(np.float32)
    mask = None
    if mask_kind == "2d":
        mask = (rng.random((lq, lk)) > 0.3).astype(np.uint8)
    elif mask_kind == "batched":
        mask = (rng.random(batch[:1] + (1,) * (len(batch) - 1) + (lq, lk)) > 0.3).astype(np.uint8)
    if mask is not None and lq > 1:
        mask[..., lq // 2, :] = 0  # a query that sees no key

    out_pad = 4 * int(rng.integers(0, 3))
    out_buf = mf.DeviceArray.from_numpy(np.full(batch + (lq, d + out_pad), POISON, np.float32),
                                        stream)
    out = out_buf.slice(-1, 0, d)
    mf.attention_fused(strided(rng, stream, q, batch), strided(rng, stream, k, batch),
                       strided(rng, stream, v, batch),
                       mask=None if mask is None else mf.DeviceArray.from_numpy(mask, stream),
                       causal=causal, scale=scale, out=out)
    image = out_buf.numpy()
    assert np.all(image[..., d:] == POISON), what + ": write into the padding columns"
    got = image[..., :d]

    s = np.float32(scale) if scale != 0.0 else np.float32(1.0 / np.sqrt(d))
    kf = np.broadcast_to(k, batch + (lk, d))
    vf = np.broadcast_to(v, batch + (lk, d))
    keep_all = np.ones(batch + (lq, lk), np.uint8)
    if mask is not None:
        keep_all &= np.broadcast_to(mask, batch + (lq, lk))
    if causal:
        keep_all &= np.tril(np.ones((lq, lk), np.uint8))
    want = np.zeros(batch + (lq, d), np.float32)
    mag = np.zeros(batch + (lq, d), np.float64)
    if lk > 0:
        for idx in np.ndindex(batch):
            sc = oracle.axpby(oracle.matmul(q[idx], np.ascontiguousarray(kf[idx].T)), s, None, 0.0)
            sc = oracle.where(keep_all[idx], sc, np.full_like(sc, -np.inf))
            p = oracle.softmax(sc, -1)
            want[idx] = oracle.matmul(p, np.ascontiguousarray(vf[idx]))
            mag[idx] = np.abs(p).astype(np.float64) @ np.abs(vf[idx]).astype(np.float64)
    dead = ~keep_all.any(axis=-1)  # queries with no key left
    assert np.all(got[dead] == 0.0), what + ": a query with no key is not zero"
    assert_gemm_parity(got, want, mag + 1e-6, lk, what)
