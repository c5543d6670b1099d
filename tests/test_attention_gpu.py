"""GPU parity of attention (q, k, v [8, 16, 1024, 64] ~ N(0,1), causal), both
the composition of the batched GEMM, where and softmax kernels and the fused kernel
(mfr_attention), against the oracle's restatement of the reference's composition
(src/ops/attention.cpp:48-98) and a float64 reference. The bar is the GEMM's: max relative error
1e-5*sqrt(Lk) of sum_j |p_ij v_jc| per output entry."""
import numpy as np
import pytest

import mensurflow_amd as mf
from helpers import assert_gemm_parity, normal, record_parity

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


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_small_with_mask(stream, oracle, causal, fused):
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
                       causal=causal, fused=fused).numpy()
    want, mag = oracle_attention(oracle, q, k, v, keep, np.float32(1.0 / 8.0))
    assert np.all(got[:, :, 7, :] == 0.0), "fully masked query gives zeros"
    assert_gemm_parity(got, want, mag + 1e-6, lk, "attention small")


def test_composed_calls_reuse_stream_scratch(oracle):
    """The composition keeps its scores, packed mask and -inf operand as its stream's scratch
    arrays, reused from call to call: a masked causal call, a smaller unmasked causal one, and a
    masked non-causal one of the first shape, on one fresh stream, each match the oracle."""
    with mf.Stream(0) as stream:
        rng = np.random.default_rng(61)
        for index, (lq, lk, use_mask, causal) in enumerate(
                [(90, 120, True, True), (40, 50, False, True), (90, 120, True, False)]):
            d = 40
            q = normal(oracle, (2, lq, d), 0.0, 1.0, 70 + index)
            k = normal(oracle, (2, lk, d), 0.0, 1.0, 80 + index)
            v = normal(oracle, (2, lk, d), 0.0, 1.0, 90 + index)
            mask = (rng.random((lq, lk)) > 0.4).astype(np.uint8) if use_mask else None
            keep = None if mask is None else mask.copy()
            if causal:
                lower = np.tril(np.ones((lq, lk), np.uint8))
                keep = lower if keep is None else keep & lower
            got = mf.attention(dev(q, stream), dev(k, stream), dev(v, stream),
                               mask=None if mask is None else dev(mask, stream), causal=causal,
                               fused=False).numpy()
            want, mag = oracle_attention(oracle, q, k, v, keep, np.float32(1.0 / np.sqrt(d)))
            assert_gemm_parity(got, want, mag + 1e-6, lk, f"composed call {index}")


def test_composed_causal_where_fallback(stream, oracle):
    """d = 18: q's rows (72 bytes) cannot take the panel path's 16-byte loads, so the scores
    GEMM refuses the causal flag and the composition masks with where() over the lower triangle
    instead; the result matches the oracle either way."""
    b, h, lq, lk, d = 2, 2, 70, 90, 18
    q = normal(oracle, (b, h, lq, d), 0.0, 1.0, 21)
    k = normal(oracle, (b, h, lk, d), 0.0, 1.0, 22)
    v = normal(oracle, (b, h, lk, d), 0.0, 1.0, 23)
    q_d, k_d, v_d = dev(q, stream), dev(k, stream), dev(v, stream)
    scores = mf.DeviceArray.empty((b, h, lq, lk), stream)
    with pytest.raises(NotImplementedError):
        mf.gemm_batched(q_d, k_d.transpose(-2, -1), scores, alpha=0.25, causal=True)
    got = mf.attention(q_d, k_d, v_d, causal=True, fused=False).numpy()
    keep = np.tril(np.ones((lq, lk), np.uint8))
    want, mag = oracle_attention(oracle, q, k, v, keep, np.float32(1.0 / np.sqrt(d)))
    assert_gemm_parity(got, want, mag + 1e-6, lk, "composed causal, where fallback")


def test_config5_attention_full(stream, oracle):
    """configs[4] at full size: B=8, H=16, S=1024, D=64, causal -- the composition and the fused
    kernel against one oracle run."""
    b, h, s, d = 8, 16, 1024, 64
    q = normal(oracle, (b, h, s, d), 0.0, 1.0, 11)
    k = normal(oracle, (b, h, s, d), 0.0, 1.0, 12)
    v = normal(oracle, (b, h, s, d), 0.0, 1.0, 13)
    q_d, k_d, v_d = dev(q, stream), dev(k, stream), dev(v, stream)
    keep = np.tril(np.ones((s, s), np.uint8))
    want, mag = oracle_attention(oracle, q, k, v, keep, np.float32(0.125))
    for fused in (False, True):
        got = mf.attention(q_d, k_d, v_d, causal=True, fused=fused).numpy()
        rel_mag, rel_max = assert_gemm_parity(got, want, mag + 1e-6, s, f"cfg5 fused={fused}")
        print(f"cfg5 attention fused={fused}: rel err vs magnitude {rel_mag:.3e}, "
              f"vs max|out| {rel_max:.3e}")
        worst64 = 0.0
        # float64 reference on two heads (as tests/reference/softmax_loss.hpp:149+): rel 1e-4
        for (bi, hi) in [(0, 0), (7, 15)]:
            sc = (q[bi, hi].astype(np.float64) @ k[bi, hi].T.astype(np.float64)) * 0.125
            sc[keep == 0] = -np.inf
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            ref = p @ v[bi, hi].astype(np.float64)
            err64 = float(np.max(np.abs(got[bi, hi] - ref) / (1.0 + np.abs(ref))))
            assert err64 < 1e-4
            worst64 = max(worst64, err64)
        record_parity(f"cfg5_attention_{'fused' if fused else 'composed'}",
                      rel_err_vs_magnitude=rel_mag, rel_err_vs_max=rel_max, bar=1e-5 * np.sqrt(s),
                      float64_rel_err_two_heads=worst64, float64_bar=1e-4)


@pytest.mark.parametrize("d", [16, 32, 48, 64, 80, 96, 112, 128])
@pytest.mark.parametrize("lq,lk", [(100, 130), (300, 200), (129, 1), (1, 257)])
@pytest.mark.parametrize("causal", [False, True])
def test_fused_shapes(stream, oracle, d, lq, lk, causal):
    """Every head size the fused kernel takes, ragged query and key counts around its 128-query
    and 64-key blocks, causal with lq != lk (top-left: query i keeps keys 0..i)."""
    b, h = 2, 2
    q = normal(oracle, (b, h, lq, d), 0.0, 1.0, 21)
    k = normal(oracle, (b, h, lk, d), 0.0, 1.0, 22)
    v = normal(oracle, (b, h, lk, d), 0.0, 1.0, 23)
    keep = np.tril(np.ones((lq, lk), np.uint8)) if causal else None
    got = mf.attention_fused(dev(q, stream), dev(k, stream), dev(v, stream),
                             causal=causal).numpy()
    scale = np.float32(1.0 / np.sqrt(d))
    want, mag = oracle_attention(oracle, q, k, v, keep, scale)
    assert_gemm_parity(got, want, mag + 1e-6, lk, f"fused d={d} lq={lq} lk={lk}")


@pytest.mark.parametrize("d", [64, 96, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_fused_many_batch_entries(stream, oracle, d, causal):
    """Enough batch entries for two workgroups of 8 wavefronts per CU (512 entries of 100
    queries), the form config 5 runs; smaller grids (test_fused_shapes) run 4 per workgroup."""
    b, h, lq, lk = 32, 16, 100, 100
    q = normal(oracle, (b, h, lq, d), 0.0, 1.0, 31)
    k = normal(oracle, (b, h, lk, d), 0.0, 1.0, 32)
    v = normal(oracle, (b, h, lk, d), 0.0, 1.0, 33)
    keep = np.tril(np.ones((lq, lk), np.uint8)) if causal else None
    got = mf.attention_fused(dev(q, stream), dev(k, stream), dev(v, stream),
                             causal=causal).numpy()
    scale = np.float32(1.0 / np.sqrt(d))
    want, mag = oracle_attention(oracle, q, k, v, keep, scale)
    assert_gemm_parity(got, want, mag + 1e-6, lk, f"fused d={d} many entries")


def test_fused_broadcast_batch_and_batched_mask(stream, oracle):
    """k and v shared over the first batch dimension (stride 0), a [B, 1, Lq, Lk] mask, an
    explicit scale."""
    b, h, lq, lk, d = 3, 2, 70, 90, 64
    q = normal(oracle, (b, h, lq, d), 0.0, 1.0, 31)
    k = normal(oracle, (1, h, lk, d), 0.0, 1.0, 32)
    v = normal(oracle, (1, h, lk, d), 0.0, 1.0, 33)
    rng = np.random.default_rng(34)
    mask = (rng.random((b, 1, lq, lk)) > 0.5).astype(np.uint8)
    shape = (b, h, lk, d)
    got = mf.attention_fused(dev(q, stream), dev(k, stream).expand(shape),
                             dev(v, stream).expand(shape), mask=dev(mask, stream),
                             scale=0.3).numpy()
    want = np.empty_like(got)
    mag = np.empty(got.shape, np.float64)
    for i in range(b):
        for hh in range(h):
            s = oracle.axpby(oracle.matmul(q[i, hh], k[0, hh].T), np.float32(0.3), None, 0.0)
            s = oracle.where(mask[i, 0], s, np.full_like(s, -np.inf))
            p = oracle.softmax(s, -1)
            want[i, hh] = oracle.matmul(p, v[0, hh])
            mag[i, hh] = np.abs(p).astype(np.float64) @ np.abs(v[0, hh]).astype(np.float64)
    assert_gemm_parity(got, want, mag + 1e-6, lk, "fused broadcast")


def test_fused_nan_row_and_empty_keys(stream, oracle):
    """A NaN in a query poisons that query's row (the reference's softmax takes a float maximum
    over the row); no keys at all gives zeros."""
    lq, lk, d = 40, 50, 64
    q = normal(oracle, (1, lq, d), 0.0, 1.0, 41)
    k = normal(oracle, (1, lk, d), 0.0, 1.0, 42)
    v = normal(oracle, (1, lk, d), 0.0, 1.0, 43)
    q[0, 5, 3] = np.nan
    got = mf.attention_fused(dev(q, stream), dev(k, stream), dev(v, stream)).numpy()
    assert np.all(np.isnan(got[0, 5]))
    assert np.all(np.isfinite(np.delete(got[0], 5, axis=0)))
    empty = mf.DeviceArray.empty((1, 0, d), stream)
    zeros = mf.attention_fused(dev(q, stream), empty, empty).numpy()
    assert zeros.shape == (1, lq, d) and np.all(zeros == 0.0)


def test_fused_unsupported_falls_back(stream, oracle):
    """d = 40 (not a multiple of 16) and a q view starting off a 16-byte boundary are not the
    fused kernel's: fused=True raises NotImplementedError, the default composes the op instead."""
    lq, lk = 33, 47
    for d, offset in ((40, 0), (64, 1)):
        store = normal(oracle, (lq * d + offset,), 0.0, 1.0, 51)
        q = store[offset:].reshape(1, lq, d)
        k = normal(oracle, (1, lk, d), 0.0, 1.0, 52)
        v = normal(oracle, (1, lk, d), 0.0, 1.0, 53)
        q_d = dev(store, stream).slice(0, offset, offset + lq * d).view((1, lq, d))
        with pytest.raises(NotImplementedError):
            mf.attention(q_d, dev(k, stream), dev(v, stream), fused=True)
        got = mf.attention(q_d, dev(k, stream), dev(v, stream)).numpy()
        want, mag = oracle_attention(oracle, q, k, v, None, np.float32(1.0 / np.sqrt(d)))
        assert_gemm_parity(got, want, mag + 1e-6, lk, f"fallback d={d}")
