"""GPU parity of attention (q, k, v [8, 16, 1024, 64] ~ N(0,1), causal) built
from the batched GEMM, where and softmax kernels, against the oracle's restatement of the same
composition (src/ops/attention.cpp:48-98) and a float64 reference."""
import numpy as np
import pytest

import mensurflow_amd as mf
from helpers import assert_gemm_parity, normal

pytestmark = pytest.mark.gpu


def dev(x, stream):
    return mf.DeviceArray.from_numpy(np.ascontiguousarray(x), stream)


def oracle_attention(oracle, q, k, v, keep, scale):
    """The reference's composition per head: packed GEMM q k^T, alpha pass, where(-inf),
    softmax, packed GEMM with v. Returns (output, magnitude sum_j |p_ij v_jc|)."""
    out = np.empty(q.shape[:-1] + (v.shape[-1],), np.float32)
    mag = np.empty_like(out, dtype=np.float64)
    for idx in np.ndindex(q.shape[:-2]):
        s = oracle.axpby(oracle.matmul(q[idx], k[idx].T), np.float32(scale), None, 0.0)
        if keep is not None:
            s = oracle.where(keep, s, np.full_like(s, -np.inf))
        p = oracle.softmax(s, -1)
        out[idx] = oracle.matmul(p, v[idx])
        mag[idx] = np.abs(p).astype(np.float64) @ np.abs(v[idx]).astype(np.float64)
    return out, mag


@pytest.mark.parametrize("causal", [False, True])
def test_attention_small_with_mask(stream, oracle, causal):
    b, h, lq, lk, d = 2, 3, 100, 130, 64
    q = normal(oracle, (b, h, lq, d), 0.0, 1.0, 1)
    k = normal(oracle, (b, h, lk, d), 0.0, 1.0, 2)
    v = normal(oracle, (b, h, lk, d), 0.0, 1.0, 3)
    rng = np.random.default_rng(4)
    mask = (rng.random((lq, lk)) > 0.3).astype(np.uint8)
    mask[7, :] = 0  # a query that sees no key
    keep = mask.copy()
    if causal:
        keep &= np.tril(np.ones((lq, lk), np.uint8))
    got = mf.attention(dev(q, stream), dev(k, stream), dev(v, stream), mask=dev(mask, stream),
                       causal=causal).numpy()
    want, mag = oracle_attention(oracle, q, k, v, keep, np.float32(1.0 / 8.0))
    assert np.all(got[:, :, 7, :] == 0.0), "fully masked query gives zeros"
    assert_gemm_parity(got, want, mag + 1e-6, lk, "attention small")


def test_config5_attention_full(stream, oracle):
    """configs[4] at full size: B=8, H=16, S=1024, D=64, causal."""
    b, h, s, d = 8, 16, 1024, 64
    q = normal(oracle, (b, h, s, d), 0.0, 1.0, 11)
    k = normal(oracle, (b, h, s, d), 0.0, 1.0, 12)
    v = normal(oracle, (b, h, s, d), 0.0, 1.0, 13)
    got = mf.attention(dev(q, stream), dev(k, stream), dev(v, stream), causal=True).numpy()
    keep = np.tril(np.ones((s, s), np.uint8))
    want, mag = oracle_attention(oracle, q, k, v, keep, np.float32(0.125))
    rel_mag, rel_max = assert_gemm_parity(got, want, mag + 1e-6, s, "cfg5")
    print(f"cfg5 attention: rel err vs magnitude {rel_mag:.3e}, vs max|out| {rel_max:.3e}")
    # float64 reference on two heads (as tests/reference/softmax_loss.hpp:149+): rel 1e-4
    for (bi, hi) in [(0, 0), (7, 15)]:
        sc = (q[bi, hi].astype(np.float64) @ k[bi, hi].T.astype(np.float64)) * 0.125
        sc[keep == 0] = -np.inf
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        ref = p @ v[bi, hi].astype(np.float64)
        assert np.max(np.abs(got[bi, hi] - ref) / (1.0 + np.abs(ref))) < 1e-4
