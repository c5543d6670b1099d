"""GPU parity of mfr_sgemm (fp32 MFMA GEMM with fused epilogue) against the oracle.

Bit-exact cases use quarter-integer inputs (the reference tests' generator): every partial sum
is exact in fp32, so the GPU result must equal the exact product in every bit whatever the
summation order -- this pins indexing, edges, transposes, strides, batching and the epilogue.
Realistic cases (Philox uniform/normal inputs, the BASELINE configs) are held to the north-star
bar: max relative error 1e-5*sqrt(K) against the per-entry magnitude sum|a*b| and against
max|C| (helpers.assert_gemm_parity). Outputs start poisoned and sit between guard bands.
"""
import numpy as np
import pytest

import mensurflow_amd as mf
from helpers import (assert_gemm_parity, magnitude, normal, quarter_input, quarter_matrix,
                     record_parity, same_bits, same_elements, tolerance, uniform)

pytestmark = pytest.mark.gpu

POISON = np.float32(123.0)


def dev(x, stream):
    return mf.DeviceArray.from_numpy(np.ascontiguousarray(x), stream)


def guarded_output(stream, shape, guard=64):
    """A [rows, cols] output in the middle of a poisoned buffer; returns (view, buffer)."""
    rows, cols = shape
    buf = mf.DeviceArray.empty((rows * cols + 2 * guard,), stream)
    mf.fill(buf, POISON)
    view = buf.slice(0, guard, guard + rows * cols).view((rows, cols))
    return view, buf


def check_guards(buf, guard=64):
    host = buf.numpy()
    assert np.all(host[:guard] == POISON) and np.all(host[-guard:] == POISON), "stray write"


def make_view(stream, values, kind):
    """The reference's matmul layouts (tests/ops/matmul_test.cpp:189-214): 0 contiguous,
    1 sliced out of a wider matrix, 2 transposed storage, 3 transposed and sliced."""
    rows, cols = values.shape
    if kind == 0:
        return dev(values, stream)
    if kind == 1:
        stored = np.full((rows + 2, cols + 9), -77.0, np.float32)
        stored[1:1 + rows, 3:3 + cols] = values
        return dev(stored, stream).slice(0, 1, 1 + rows).slice(1, 3, 3 + cols)
    if kind == 2:
        return dev(np.ascontiguousarray(values.T), stream).T
    stored = np.full((cols + 3, rows + 5), -77.0, np.float32)
    stored[2:2 + cols, 4:4 + rows] = values.T
    return dev(stored, stream).slice(0, 2, 2 + cols).slice(1, 4, 4 + rows).T


def exact_product(a, b):
    return (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)


def test_known_values(stream):
    a = dev(np.array([[1, 2, 3], [4, 5, 6]], np.float32), stream)
    b = dev(np.array([[7, 8], [9, 10], [11, 12]], np.float32), stream)
    assert mf.gemm(a, b).numpy().tolist() == [[58, 64], [139, 154]]
    values = quarter_input(5 * 7, 3).reshape(5, 7)
    ident = mf.gemm(dev(values, stream), dev(np.eye(7, dtype=np.float32), stream)).numpy()
    assert same_bits(ident, values)


# Sizes around the 128x128x32 tile and the reference's block edges.
SHAPES = [(1, 1, 1), (1, 5, 1), (5, 1, 3), (3, 5, 7), (16, 16, 16), (17, 31, 13), (64, 64, 64),
          (65, 129, 130), (100, 300, 50), (200, 100, 300), (2, 1000, 3), (1000, 2, 3),
          (257, 129, 257), (127, 128, 31), (128, 128, 32), (129, 255, 33), (256, 256, 256),
          (300, 77, 1000)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_exact_shapes(stream, m, n, k):
    a = quarter_matrix(m, k, m + 1)
    b = quarter_matrix(k, n, n + 2)
    c, buf = guarded_output(stream, (m, n))
    mf.gemm(dev(a, stream), dev(b, stream), out=c)
    assert same_bits(c.numpy(), exact_product(a, b)), f"{m}x{n}x{k}"
    check_guards(buf)


@pytest.mark.parametrize("m,n,k", [(70, 60, 90), (130, 200, 150), (300, 300, 300)])
def test_exact_strided_layouts(stream, m, n, k):
    a = quarter_matrix(m, k, 21)
    b = quarter_matrix(k, n, 22)
    want = exact_product(a, b)
    for kind_a in range(4):
        for kind_b in range(4):
            c, buf = guarded_output(stream, (m, n))
            mf.gemm(make_view(stream, a, kind_a), make_view(stream, b, kind_b), out=c)
            assert same_bits(c.numpy(), want), f"A{kind_a} B{kind_b}"
            check_guards(buf)


@pytest.mark.parametrize("trans_a,trans_b", [(False, False), (False, True), (True, False),
                                             (True, True)])
def test_exact_alpha_beta_in_place(stream, trans_a, trans_b):
    m, n, k = 190, 133, 300
    a = quarter_matrix(k if trans_a else m, m if trans_a else k, 31)
    b = quarter_matrix(n if trans_b else k, k if trans_b else n, 32)
    c0 = quarter_matrix(m, n, 33)
    left = a.T if trans_a else a
    right = b.T if trans_b else b
    want = (np.float32(1.5) * exact_product(left, right)) + np.float32(0.5) * c0
    c = dev(c0, stream)
    # c0 == c: the epilogue reads and writes the same element in place.
    mf.gemm(dev(a, stream), dev(b, stream), alpha=1.5, c0=c, beta=0.5, trans_a=trans_a,
            trans_b=trans_b, out=c)
    assert same_bits(c.numpy(), want.astype(np.float32))


TILES = list(range(1, mf.abi.TILE_THIN))  # the MFMA tiles


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("m,n,k", [(300, 260, 1000), (257, 129, 257), (1, 300, 64),
                                   (513, 7, 96), (64, 64, 2000), (129, 65, 36), (2100, 2100, 64)])
def test_exact_every_tile(stream, tile, m, n, k):
    """Every workgroup tile on edge shapes and all four layouts: bits equal the exact product.
    2100^2 has more tiles than CUs for the 128x128 tile, so both of its launch forms (8
    wavefronts at one workgroup per CU, 4 beyond) are covered. With staging off, the 256x256
    tile reads operands that 16-byte loads cannot take with 4-byte direct-to-LDS loads."""
    a = quarter_matrix(m, k, 71)
    b = quarter_matrix(k, n, 72)
    c0 = quarter_matrix(m, n, 73)
    bias = quarter_matrix(1, n, 74)[0]
    want = (np.float32(1.5) * exact_product(a, b)) + np.float32(0.5) * c0
    want = (want + bias).astype(np.float32)
    for trans_a in (False, True):
        for trans_b in (False, True):
            a_st = np.ascontiguousarray(a.T) if trans_a else a
            b_st = np.ascontiguousarray(b.T) if trans_b else b
            c, buf = guarded_output(stream, (m, n))
            mf.gemm(dev(a_st, stream), dev(b_st, stream), alpha=1.5, c0=dev(c0, stream), beta=0.5,
                    trans_a=trans_a, trans_b=trans_b, bias=dev(bias, stream), out=c, tile=tile,
                    stage=mf.abi.STAGE_NEVER)
            assert same_bits(c.numpy(), want), (tile, trans_a, trans_b)
            check_guards(buf)


@pytest.mark.parametrize("tile", TILES)
def test_exact_batched_every_tile(stream, tile):
    bsz, heads, m, n, k = 2, 3, 100, 68, 64
    a = quarter_matrix(bsz * heads * m, k, 81).reshape(bsz, heads, m, k)
    bt = quarter_matrix(heads * n, k, 82).reshape(1, heads, n, k)
    out = mf.DeviceArray.empty((bsz, heads, m, n), stream)
    b_d = dev(bt, stream).expand((bsz, heads, n, k)).transpose(-2, -1)
    mf.gemm_batched(dev(a, stream), b_d, out, alpha=0.5, tile=tile)
    got = out.numpy()
    for i in range(bsz):
        for h in range(heads):
            want = (np.float32(0.5) * exact_product(a[i, h], bt[0, h].T)).astype(np.float32)
            assert same_bits(got[i, h], want), (tile, i, h)


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("m,n,k", [(300, 261, 1023), (257, 129, 257), (5, 300, 63),
                                   (129, 66, 35)])
def test_exact_staged_every_tile(stream, tile, m, n, k):
    """Operands copied to the aligned workspace first (stage ALWAYS), on every tile and every
    pair of the reference's matmul layouts -- sliced views start at unaligned addresses with odd
    strides: bits equal the exact product."""
    a = quarter_matrix(m, k, 91)
    b = quarter_matrix(k, n, 92)
    c0 = quarter_matrix(m, n, 93)
    bias = quarter_matrix(1, n, 94)[0]
    want = (np.float32(1.5) * exact_product(a, b)) + np.float32(0.5) * c0
    want = (want + bias).astype(np.float32)
    c0_d, bias_d = dev(c0, stream), dev(bias, stream)
    for kind_a in range(4):
        for kind_b in range(4):
            c, buf = guarded_output(stream, (m, n))
            mf.gemm(make_view(stream, a, kind_a), make_view(stream, b, kind_b), alpha=1.5,
                    c0=c0_d, beta=0.5, bias=bias_d, out=c, tile=tile,
                    stage=mf.abi.STAGE_ALWAYS)
            assert same_bits(c.numpy(), want), (tile, kind_a, kind_b)
            check_guards(buf)


def test_exact_staged_batched_broadcast(stream):
    """Staging a batched operand copies each distinct matrix once: a broadcast batch dimension
    (stride 0) stays broadcast in the staged copy."""
    bsz, heads, m, n, k = 3, 2, 70, 45, 63
    a = quarter_matrix(heads * m, k, 95).reshape(1, heads, m, k)
    b = quarter_matrix(bsz * heads * k, n, 96).reshape(bsz, heads, k, n)
    out = mf.DeviceArray.empty((bsz, heads, m, n), stream)
    a_d = dev(a, stream).expand((bsz, heads, m, k))
    for tile in TILES:
        mf.gemm_batched(a_d, dev(b, stream), out, alpha=0.5, tile=tile,
                        stage=mf.abi.STAGE_ALWAYS)
        got = out.numpy()
        for i in range(bsz):
            for h in range(heads):
                want = (np.float32(0.5) * exact_product(a[0, h], b[i, h])).astype(np.float32)
                assert same_bits(got[i, h], want), (tile, i, h)


def test_stage_modes_agree_bitwise(stream, oracle):
    """Staging changes only where operands are read from: with the same tile, realistic inputs
    give the same bits staged and unstaged (the zero padding adds +0 to each sum). For the
    256x256 tile that compares the register-staged 16-byte kernel with the direct-to-LDS one."""
    m, n, k = 1021, 515, 1023
    x = oracle.normal(m * k, 0.0, 1.0, 11, 0).reshape(m, k)
    w = oracle.normal(k * n, 0.0, 1.0 / np.sqrt(k), 12, 0).reshape(k, n)
    x_d, w_d = dev(x, stream), dev(w, stream)
    for tile in TILES:
        plain = mf.gemm(x_d, w_d, tile=tile, stage=mf.abi.STAGE_NEVER).numpy()
        staged = mf.gemm(x_d, w_d, tile=tile, stage=mf.abi.STAGE_ALWAYS).numpy()
        assert np.array_equal(plain.view(np.uint32), staged.view(np.uint32)), tile
    got = mf.gemm(x_d, w_d, tile=mf.abi.TILE_256x256, stage=mf.abi.STAGE_ALWAYS).numpy()
    assert_gemm_parity(got, oracle.gemm(x, w), magnitude(oracle, x, w), k, "staged 256x256")


TILE_BN = {1: 256, 2: 128, 3: 64, 4: 128, 5: 64}  # output columns per tile, by abi.TILE_* id


@pytest.mark.parametrize("m, n, k, b_kmajor", [
    (4093, 4099, 1023, False),  # configs[3]: 4093 x 4096 on the 256x256 tile, a 3-column strip
    (2045, 2053, 1023, False),  # a 5-column strip (the 8-column kernel)
    (2045, 2049, 1021, True),   # B read along k through a transposed view, staged as well
    (2045, 2049, 1023, False),  # one column (the 1-column kernel)
    (2045, 2050, 999, False),   # two columns, an odd depth (the copy's line padded by one zero)
    (2045, 2051, 2101, False),  # rows loaded in three chunks of 1024 depths, the last partial
])
def test_strip_stages_a_in_one_launch(stream, oracle, m, n, k, b_kmajor):
    """AUTO stages a K-major A whose rows 16-byte loads cannot take; when a peeled strip of at
    most 8 columns covers all of A's rows, the strip's launch writes that copy as it reads A.

    The strip's columns must be the thin path's bits on A read in place (tile THIN, staging off),
    and the main rectangle's the same tile's bits with A copied by the staging kernel, so the
    copy (with its zero padding) is the staging kernel's. Both parts within the parity bar."""
    x = normal(oracle, (m, k), 0.0, 1.0, 21, 0)
    w = normal(oracle, (k, n), 0.0, float(1.0 / np.sqrt(k)), 22, 0)
    bias = uniform(oracle, (n,), -0.1, 0.1, 23, 0)
    x_d, b_d = dev(x, stream), dev(bias, stream)
    w_d = dev(np.ascontiguousarray(w.T), stream).T if b_kmajor else dev(w, stream)
    out_d = mf.DeviceArray.empty((m, n), stream)
    tile, stage, splits, regions = mf.gemm_plan(x_d, w_d, out_d)
    assert stage == mf.abi.STAGE_ALWAYS and splits == 1 and regions == 2, (tile, stage, regions)
    main_n = n - n % TILE_BN[tile]
    assert 0 < n - main_n <= 8
    got = mf.gemm(x_d, w_d, bias=b_d, act=mf.ACT_GELU_TANH, out=out_d).numpy()
    strip = mf.gemm(x_d, w_d.slice(1, main_n, n), bias=b_d.slice(0, main_n, n),
                    act=mf.ACT_GELU_TANH, tile=mf.abi.TILE_THIN, stage=mf.abi.STAGE_NEVER).numpy()
    main = mf.gemm(x_d, w_d.slice(1, 0, main_n), bias=b_d.slice(0, 0, main_n),
                   act=mf.ACT_GELU_TANH, tile=tile, stage=mf.abi.STAGE_ALWAYS).numpy()
    assert same_bits(got[:, main_n:], strip)
    assert same_bits(got[:, :main_n], main)
    if m * n * k < 2**33:
        want = oracle.gelu(oracle.bias_add(oracle.matmul(x, w), bias), approximate=True)
        scale = 1.13 * (magnitude(oracle, x, w) + np.abs(bias))
        assert_gemm_parity(got, want, scale, k, f"strip staging {m}x{n}x{k}")


def test_strip_staging_with_alpha_beta_c0(stream, oracle):
    """The strip's launch that copies A also runs the full epilogue: alpha, beta * C0 and the
    bias (no activation), bit for bit the thin path's on A read in place, and the main rectangle
    the staged tile's; both within the parity bar."""
    m, n, k = 2045, 2051, 1023
    alpha, beta = 1.5, 0.5
    x = normal(oracle, (m, k), 0.0, 1.0, 31, 0)
    w = normal(oracle, (k, n), 0.0, float(1.0 / np.sqrt(k)), 32, 0)
    c0 = normal(oracle, (m, n), 0.0, 1.0, 33, 0)
    bias = uniform(oracle, (n,), -0.1, 0.1, 34, 0)
    x_d, w_d, c0_d, b_d = dev(x, stream), dev(w, stream), dev(c0, stream), dev(bias, stream)
    out_d = mf.DeviceArray.empty((m, n), stream)
    tile, stage, splits, regions = mf.gemm_plan(x_d, w_d, out_d, c0=c0_d, beta=beta)
    assert stage == mf.abi.STAGE_ALWAYS and splits == 1 and regions == 2, (tile, stage, regions)
    main_n = n - n % TILE_BN[tile]
    got = mf.gemm(x_d, w_d, alpha=alpha, beta=beta, c0=c0_d, bias=b_d, out=out_d).numpy()
    strip = mf.gemm(x_d, w_d.slice(1, main_n, n), alpha=alpha, beta=beta,
                    c0=c0_d.slice(1, main_n, n), bias=b_d.slice(0, main_n, n),
                    tile=mf.abi.TILE_THIN, stage=mf.abi.STAGE_NEVER).numpy()
    main = mf.gemm(x_d, w_d.slice(1, 0, main_n), alpha=alpha, beta=beta,
                   c0=c0_d.slice(1, 0, main_n), bias=b_d.slice(0, 0, main_n), tile=tile,
                   stage=mf.abi.STAGE_ALWAYS).numpy()
    assert same_bits(got[:, main_n:], strip)
    assert same_bits(got[:, :main_n], main)
    want = oracle.bias_add(oracle.gemm(x, w, alpha=alpha, c0=c0, beta=beta), bias)
    scale = alpha * magnitude(oracle, x, w) + beta * np.abs(c0) + np.abs(bias)
    assert_gemm_parity(got, want, scale, k, "strip staging, alpha beta C0")


def test_plan_on_baseline_shapes(stream):
    """mfr_sgemm_plan reports what AUTO runs: the 256x256 tile in place for configs[2], staged
    operands for configs[3] (whose rows 16-byte loads cannot take), the 256x256 tile reading them
    in place (straight into LDS) when staging is off, the panel path for the attention scores."""
    abi = mf.abi
    big = mf.DeviceArray.empty((4096, 4096), stream)
    assert mf.gemm_plan(big, big.T, big) == (abi.TILE_256x256, abi.STAGE_NEVER, 1, 1)
    x = mf.DeviceArray.empty((4093, 1023), stream)
    w = mf.DeviceArray.empty((1023, 4099), stream)
    out = mf.DeviceArray.empty((4093, 4099), stream)
    tile, stage, splits, regions = mf.gemm_plan(x, w, out)
    assert (tile, stage, splits) == (abi.TILE_256x256, abi.STAGE_ALWAYS, 1)
    assert mf.gemm_plan(x, w, out, stage=abi.STAGE_NEVER)[:2] == (abi.TILE_256x256,
                                                                  abi.STAGE_NEVER)
    q = mf.DeviceArray.empty((128, 1024, 64), stream)
    scores = mf.DeviceArray.empty((128, 1024, 1024), stream)
    assert mf.gemm_plan(q, q.transpose(-2, -1), scores) == (abi.TILE_PANEL, abi.STAGE_NEVER, 1, 1)
    # Small outputs, and operands the panel path cannot read, keep the short-depth tiles.
    assert mf.gemm_plan(q.slice(0, 0, 1).slice(1, 0, 128), q.slice(0, 0, 1).slice(1, 0, 128)
                        .transpose(-2, -1), scores.slice(0, 0, 1).slice(1, 0, 128)
                        .slice(2, 0, 128))[0] in (abi.TILE_128x64, abi.TILE_64x128)
    v = mf.DeviceArray.empty((128, 64, 1024), stream)
    assert mf.gemm_plan(q, v, scores)[0] in (abi.TILE_128x64, abi.TILE_64x128)
    assert mf.gemm_plan(x, w, out, tile=abi.TILE_256x256, stage=abi.STAGE_NEVER)[:2] == (
        abi.TILE_256x256, abi.STAGE_NEVER)
    assert mf.gemm_plan(x, w, out, tile=abi.TILE_256x256)[:2] == (abi.TILE_256x256,
                                                                  abi.STAGE_ALWAYS)
    empty = mf.DeviceArray.empty((0, 4099), stream)
    assert mf.gemm_plan(mf.DeviceArray.empty((0, 1023), stream), w, empty)[0] == abi.TILE_AUTO
    # The fixed 256x256 tile on odd operands runs staged, bit-exact.
    m, n, k = 130, 75, 67
    a = quarter_matrix(m, k, 97)
    b = quarter_matrix(k, n, 98)
    got = mf.gemm(dev(a, stream), dev(b, stream), tile=abi.TILE_256x256).numpy()
    assert same_bits(got, exact_product(a, b))


@pytest.mark.parametrize("m,n,k", [(256, 256, 4), (256, 256, 28), (256, 256, 32), (300, 260, 36),
                                   (256, 256, 64), (300, 260, 96), (256, 512, 100),
                                   (512, 200, 128), (260, 300, 160), (256, 256, 260)])
def test_held_back_slices_exact(stream, m, n, k):
    """The 256x256 tile with both operands read along k (A row-major, B a transposed view of an
    [n, k] array, 16-byte loads, in place) holds each 32-deep slice's last group of MFMAs back
    across the slice barrier and reads one group past the last slice. Depths of one to nine
    slices, odd and even counts and ragged last slices, on whole and ragged tiles: the exact
    product of quarter integers, and the same bits as the same product read N-major (the
    in-order loop); one case with alpha, beta and C0."""
    a = quarter_matrix(m, k, 300 + k)
    bt = quarter_matrix(n, k, 400 + k)
    a_d, bt_d = dev(a, stream), dev(bt, stream)
    view, buf = guarded_output(stream, (m, n))
    mf.gemm(a_d, bt_d, trans_b=True, tile=mf.abi.TILE_256x256, stage=mf.abi.STAGE_NEVER,
            out=view)
    got = view.numpy()
    check_guards(buf)
    want = exact_product(a, bt.T)
    assert same_bits(got, want), f"{m}x{n}x{k}"
    b_nmajor = dev(np.ascontiguousarray(bt.T), stream)
    other = mf.gemm(a_d, b_nmajor, tile=mf.abi.TILE_256x256, stage=mf.abi.STAGE_NEVER).numpy()
    assert same_bits(got, other), f"{m}x{n}x{k}: K-major and N-major B differ"
    if k == 100:
        c0 = quarter_matrix(m, n, 500)
        got = mf.gemm(a_d, bt_d, trans_b=True, alpha=1.5, c0=dev(c0, stream), beta=0.5,
                      tile=mf.abi.TILE_256x256, stage=mf.abi.STAGE_NEVER).numpy()
        want = (np.float32(1.5) * exact_product(a, bt.T) + np.float32(0.5) * c0).astype(np.float32)
        assert same_bits(got, want), "alpha, beta and C0"


# ---- the panel path ------------------------------------------------------------------------------

PANEL = mf.abi.TILE_PANEL


@pytest.mark.parametrize("m,n,k", [(1, 1, 4), (1, 300, 64), (255, 63, 64), (256, 64, 64),
                                   (257, 65, 60), (300, 200, 36), (513, 1000, 16), (1000, 129, 4),
                                   (129, 1, 8), (700, 777, 32), (2100, 1100, 64), (64, 4100, 12)])
def test_exact_panel(stream, m, n, k):
    """The panel path (B read along k) on shapes around its 256-row panels, 64-column tiles and
    depth groups: alpha, beta * C0 (separate and in place) and a bias; bits equal the exact
    product and the guard bands survive."""
    a = quarter_matrix(m, k, 101)
    bt = quarter_matrix(n, k, 102)
    c0 = quarter_matrix(m, n, 103)
    bias = quarter_matrix(1, n, 104)[0]
    a_d, b_d, bias_d = dev(a, stream), dev(bt, stream).T, dev(bias, stream)
    product = exact_product(a, bt.T)
    want = ((np.float32(1.5) * product) + np.float32(0.5) * c0 + bias).astype(np.float32)
    c, buf = guarded_output(stream, (m, n))
    assert mf.gemm_plan(a_d, b_d, c, tile=PANEL)[0] == PANEL
    mf.gemm_batched(a_d, b_d, c, alpha=1.5, c0=dev(c0, stream), beta=0.5, bias=bias_d, tile=PANEL)
    assert same_bits(c.numpy(), want), f"{m}x{n}x{k}"
    check_guards(buf)
    c_in = dev(c0, stream)
    mf.gemm_batched(a_d, b_d, c_in, alpha=1.5, c0=c_in, beta=0.5, bias=bias_d, tile=PANEL)
    assert same_bits(c_in.numpy(), want), f"{m}x{n}x{k} in place"
    plain, buf = guarded_output(stream, (m, n))
    mf.gemm_batched(a_d, b_d, plain, tile=PANEL)
    assert same_bits(plain.numpy(), product), f"{m}x{n}x{k} plain"
    check_guards(buf)


def test_exact_panel_batched_broadcast(stream):
    """Two batch dimensions, B broadcast over the first and A over the second; row strides wider
    than k; the output's rows wider than n (a padded row stride)."""
    bsz, heads, m, n, k = 2, 3, 300, 130, 40
    a = quarter_matrix(bsz * m, k, 111).reshape(bsz, 1, m, k)
    bt = quarter_matrix(heads * n, k, 112).reshape(1, heads, n, k)
    a_st = np.full((bsz, 1, m, k + 8), -5.0, np.float32)
    a_st[..., :k] = a
    a_d = dev(a_st, stream).slice(-1, 0, k).expand((bsz, heads, m, k))
    b_d = dev(bt, stream).expand((bsz, heads, n, k)).transpose(-2, -1)
    wide = mf.DeviceArray.empty((bsz, heads, m, n + 12), stream)
    mf.fill(wide, POISON)
    out = wide.slice(-1, 0, n)
    mf.gemm_batched(a_d, b_d, out, alpha=0.125, tile=PANEL)
    got = wide.numpy()
    assert np.all(got[..., n:] == POISON)
    for i in range(bsz):
        for h in range(heads):
            want = (np.float32(0.125) * exact_product(a[i, 0], bt[0, h].T)).astype(np.float32)
            assert same_bits(got[i, h, :, :n], want), (i, h)


def test_panel_matches_tiles_bitwise(stream, oracle):
    """Realistic inputs: the panel path sums in the MFMA tiles' order, so the scores of a causal
    attention-sized product come out bit for bit as on the 128x64 tile, AUTO picks the panel
    path, and the result is within the parity bar of the oracle."""
    bsz, m, n, k = 4, 1024, 1024, 64
    q = normal(oracle, (bsz, m, k), 0.0, 1.0, 121, 0)
    kk = normal(oracle, (bsz, n, k), 0.0, 1.0, 122, 0)
    q_d, k_d = dev(q, stream), dev(kk, stream).transpose(-2, -1)
    out = mf.DeviceArray.empty((bsz, m, n), stream)
    assert mf.gemm_plan(q_d, k_d, out)[0] == PANEL
    mf.gemm_batched(q_d, k_d, out, alpha=0.125)
    got = out.numpy()
    mf.gemm_batched(q_d, k_d, out, alpha=0.125, tile=mf.abi.TILE_128x64)
    assert np.array_equal(got.view(np.uint32), out.numpy().view(np.uint32))
    for b in range(bsz):
        want = oracle.gemm(q[b], kk[b], alpha=0.125, trans_b=True)
        scale = 0.125 * magnitude(oracle, q[b], kk[b].T)
        assert_gemm_parity(got[b], want, scale, k, f"panel scores batch {b}")


@pytest.mark.parametrize("case", ["depth 68", "depth 6", "B along n", "A along m",
                                  "activation", "split", "unaligned A"])
def test_panel_refusals(stream, case):
    """A fixed PANEL point it cannot take fails with MFR_E_UNSUPPORTED and leaves C untouched."""
    m, n, k = 300, 200, 68 if case == "depth 68" else 6 if case == "depth 6" else 32
    a = dev(quarter_matrix(m, k, 131), stream)
    bt = dev(quarter_matrix(n, k, 132), stream)
    b = bt.T
    kwargs = {}
    if case == "B along n":
        b = dev(quarter_matrix(k, n, 133), stream)
    elif case == "A along m":
        a = dev(quarter_matrix(k, m, 134), stream).T
    elif case == "activation":
        kwargs["act"] = mf.ACT_GELU_TANH
    elif case == "split":
        kwargs["splits"] = 2
    elif case == "unaligned A":
        a = dev(quarter_matrix(m, k + 1, 135), stream).slice(1, 1, k + 1)
    c = mf.DeviceArray.empty((m, n), stream)
    mf.fill(c, POISON)
    with pytest.raises(NotImplementedError):
        mf.gemm_batched(a, b, c, tile=PANEL, **kwargs)
    assert np.all(c.numpy() == POISON)


# ---- the causal flag (attention's scores, MFR_GEMM_CAUSAL) --------------------------------------

def causal_where(x):
    """where(keep, x, -inf) with keep(i, j) = j <= i over the last two dimensions (the reference's
    top-left causal mask, src/ops/attention.cpp:85-96)."""
    rows, cols = x.shape[-2:]
    keep = np.tril(np.ones((rows, cols), bool))
    return np.where(keep, x, np.float32(-np.inf)).astype(np.float32)


@pytest.mark.parametrize("m,n,k", [(1, 1, 4), (1, 300, 64), (64, 64, 4), (255, 63, 64),
                                   (256, 64, 64), (300, 200, 40), (513, 700, 20), (200, 900, 64),
                                   (900, 200, 8), (1024, 1024, 64), (2100, 1100, 60)])
def test_exact_causal_panel(stream, m, n, k):
    """-inf wherever column > row and the exact product elsewhere, with blocks wholly above the
    diagonal skipped and blocks across it masked lane by lane: bits equal where(tril, product,
    -inf), AUTO takes the flag to the panel path, and the guard bands survive."""
    a = quarter_matrix(m, k, 151)
    bt = quarter_matrix(n, k, 152)
    a_d, b_d = dev(a, stream), dev(bt, stream).T
    want = causal_where((np.float32(0.75) * exact_product(a, bt.T)).astype(np.float32))
    for tile in (0, PANEL):
        c, buf = guarded_output(stream, (m, n))
        assert mf.gemm_plan(a_d, b_d, c, tile=tile, causal=True)[0] == PANEL
        mf.gemm_batched(a_d, b_d, c, alpha=0.75, tile=tile, causal=True)
        assert same_bits(c.numpy(), want), f"{m}x{n}x{k} tile {tile}"
        check_guards(buf)


def test_causal_panel_batched_with_epilogue(stream):
    """Two broadcast batch dimensions, a padded output row stride, beta * C0 and a bias: the mask
    applies after the epilogue (the masked outputs are -inf whatever C0 and the bias hold)."""
    bsz, heads, m, n, k = 2, 3, 300, 280, 32
    a = quarter_matrix(bsz * m, k, 161).reshape(bsz, 1, m, k)
    bt = quarter_matrix(heads * n, k, 162).reshape(1, heads, n, k)
    c0 = quarter_matrix(bsz * heads * m, n, 163).reshape(bsz, heads, m, n)
    bias = quarter_matrix(1, n, 164)[0]
    a_d = dev(a, stream).expand((bsz, heads, m, k))
    b_d = dev(bt, stream).expand((bsz, heads, n, k)).transpose(-2, -1)
    wide = mf.DeviceArray.empty((bsz, heads, m, n + 12), stream)
    mf.fill(wide, POISON)
    out = wide.slice(-1, 0, n)
    mf.gemm_batched(a_d, b_d, out, alpha=0.5, c0=dev(c0, stream), beta=2.0,
                    bias=dev(bias, stream), causal=True)
    got = wide.numpy()
    assert np.all(got[..., n:] == POISON)
    for i in range(bsz):
        for h in range(heads):
            pre = ((np.float32(0.5) * exact_product(a[i, 0], bt[0, h].T)) +
                   np.float32(2.0) * c0[i, h] + bias).astype(np.float32)
            assert same_bits(got[i, h, :, :n], causal_where(pre)), (i, h)


def test_causal_matches_plain_then_where(stream, oracle):
    """Realistic inputs at attention's shape: the causal product is bit for bit the plain panel
    product followed by where(tril, scores, -inf), the composition's own steps."""
    bsz, m, n, k = 4, 1024, 1024, 64
    q = normal(oracle, (bsz, m, k), 0.0, 1.0, 171, 0)
    kk = normal(oracle, (bsz, n, k), 0.0, 1.0, 172, 0)
    q_d, k_d = dev(q, stream), dev(kk, stream).transpose(-2, -1)
    out = mf.DeviceArray.empty((bsz, m, n), stream)
    mf.gemm_batched(q_d, k_d, out, alpha=0.125)
    want = causal_where(out.numpy())
    mf.gemm_batched(q_d, k_d, out, alpha=0.125, causal=True)
    assert np.array_equal(out.numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("case", ["fixed 128x64", "depth 6", "depth 68", "activation", "split",
                                  "B along n"])
def test_causal_refusals(stream, case):
    """The causal flag on a point the panel path cannot take (or with a fixed tile of another
    path) fails with MFR_E_UNSUPPORTED and leaves C untouched; unknown flags are invalid."""
    m, n, k = 300, 200, 68 if case == "depth 68" else 6 if case == "depth 6" else 32
    a = dev(quarter_matrix(m, k, 181), stream)
    b = dev(quarter_matrix(n, k, 182), stream).T
    kwargs = {}
    if case == "fixed 128x64":
        kwargs["tile"] = mf.abi.TILE_128x64
    elif case == "activation":
        kwargs["act"] = mf.ACT_GELU_TANH
    elif case == "split":
        kwargs["splits"] = 2
    elif case == "B along n":
        b = dev(quarter_matrix(k, n, 183), stream)
    c = mf.DeviceArray.empty((m, n), stream)
    mf.fill(c, POISON)
    with pytest.raises(NotImplementedError):
        mf.gemm_batched(a, b, c, causal=True, **kwargs)
    assert np.all(c.numpy() == POISON)
    d = mf._gemm_desc(a, b, c, 1.0, None, 0.0, None, mf.ACT_NONE, 0, 0)
    d.flags = 2
    with pytest.raises(ValueError):
        mf.sgemm(c.stream, d)
    assert np.all(c.numpy() == POISON)


# ---- the paired 128x64 kernel (B read along n, at most 64 columns) ------------------------------

@pytest.mark.parametrize("m,n,k", [(1, 64, 4), (127, 64, 32), (128, 60, 36), (129, 32, 100),
                                   (300, 4, 1024), (1000, 16, 68), (513, 64, 257 * 4)])
def test_exact_pair_tile(stream, m, n, k):
    """The 128x64 tile on a K-major A and an N-major B of at most 64 columns (sgemm_pair_kernel,
    whose lanes hold column pairs): alpha, beta * C0, a bias and the tanh gelu, a split-K run, and
    rows, columns and depths past the tile edges. Bits equal the exact result."""
    a = quarter_matrix(m, k, 141)
    b = quarter_matrix(k, n, 142)
    c0 = quarter_matrix(m, n, 143)
    bias = quarter_matrix(1, n, 144)[0]
    a_d, b_d, c0_d, bias_d = dev(a, stream), dev(b, stream), dev(c0, stream), dev(bias, stream)
    tile = mf.abi.TILE_128x64
    pre = ((np.float32(1.5) * exact_product(a, b)) + np.float32(0.5) * c0 + bias).astype(
        np.float32)
    c, buf = guarded_output(stream, (m, n))
    mf.gemm_batched(a_d, b_d, c, alpha=1.5, c0=c0_d, beta=0.5, bias=bias_d, tile=tile, splits=1)
    assert same_bits(c.numpy(), pre), f"{m}x{n}x{k}"
    check_guards(buf)
    mf.gemm_batched(a_d, b_d, c, alpha=1.5, c0=c0_d, beta=0.5, bias=bias_d,
                    act=mf.ACT_GELU_TANH, tile=tile, splits=1)
    from oracle import Oracle
    assert same_bits(c.numpy(), Oracle().gelu(pre, approximate=True)), f"{m}x{n}x{k} gelu"
    if k >= 512:
        split, buf = guarded_output(stream, (m, n))
        mf.gemm_batched(a_d, b_d, split, alpha=1.5, c0=c0_d, beta=0.5, bias=bias_d, tile=tile,
                        splits=4)
        assert mf.gemm_plan(a_d, b_d, split, tile=tile, splits=4)[2] == 4
        assert same_bits(split.numpy(), pre), f"{m}x{n}x{k} split"
        check_guards(buf)


def test_pair_tile_attention_pv_bitwise(stream, oracle):
    """Attention's P V at 4 x [1024 x 1024] x [1024 x 64] on the 128x64 tile (the paired kernel,
    which AUTO picks at config 5's 128 batches) gives the 64x64 tile's bits (the tiles share one
    summation order) and is within the parity bar of the oracle."""
    bsz, m, n, k = 4, 1024, 64, 1024
    pm = uniform(oracle, (bsz, m, k), 0.0, 1.0 / 512.0, 151, 0)
    v = normal(oracle, (bsz, k, n), 0.0, 1.0, 152, 0)
    p_d, v_d = dev(pm, stream), dev(v, stream)
    out = mf.DeviceArray.empty((bsz, m, n), stream)
    scores = mf.DeviceArray.empty((128, m, k), stream)
    values = mf.DeviceArray.empty((128, k, n), stream)
    assert mf.gemm_plan(scores, values, mf.DeviceArray.empty((128, m, n), stream))[0] == (
        mf.abi.TILE_128x64)
    mf.gemm_batched(p_d, v_d, out, tile=mf.abi.TILE_128x64)
    got = out.numpy()
    mf.gemm_batched(p_d, v_d, out, tile=mf.abi.TILE_64x64)
    assert np.array_equal(got.view(np.uint32), out.numpy().view(np.uint32))
    for b in range(bsz):
        want = oracle.matmul(pm[b], v[b])
        assert_gemm_parity(got[b], want, magnitude(oracle, pm[b], v[b]), k, f"P V batch {b}")


# ---- split-K -----------------------------------------------------------------------------------

def ranges_run(k, splits):
    """Depth ranges mfr_sgemm runs when `splits` are asked for: each a multiple of 32 deep."""
    if splits <= 1 or k == 0:
        return 1
    per = -(-k // splits)           # ceil(k / splits)
    per = -(-per // 32) * 32        # rounded up to a multiple of 32
    return -(-k // per)


@pytest.mark.parametrize("splits", [2, 3, 5, 8, 64])
@pytest.mark.parametrize("tile", TILES)
def test_exact_split_k_every_tile(stream, tile, splits):
    """Split-K on every tile and all four layouts, with alpha, beta*C0 and a bias: the ranges'
    raw sums and their reduction are exact on quarter integers, so the bits equal the exact
    product. n is odd, so the fixed 256x256 tile also stages its operands into the same
    workspace as the partial sums."""
    m, n, k = 130, 97, 1000
    a = quarter_matrix(m, k, 171)
    b = quarter_matrix(k, n, 172)
    c0 = quarter_matrix(m, n, 173)
    bias = quarter_matrix(1, n, 174)[0]
    want = (np.float32(1.5) * exact_product(a, b)) + np.float32(0.5) * c0
    want = (want + bias).astype(np.float32)
    for trans_a in (False, True):
        for trans_b in (False, True):
            a_d = dev(np.ascontiguousarray(a.T) if trans_a else a, stream)
            b_d = dev(np.ascontiguousarray(b.T) if trans_b else b, stream)
            left = a_d.T if trans_a else a_d
            right = b_d.T if trans_b else b_d
            c, buf = guarded_output(stream, (m, n))
            plan = mf.gemm_plan(left, right, c, tile=tile, splits=splits)
            assert plan[0] == tile and plan[2] == ranges_run(k, splits), plan
            mf.gemm(left, right, alpha=1.5, c0=dev(c0, stream), beta=0.5,
                    bias=dev(bias, stream), out=c, tile=tile, splits=splits)
            assert same_bits(c.numpy(), want), (tile, splits, trans_a, trans_b)
            check_guards(buf)


def test_exact_split_k_batched_broadcast_in_place(stream):
    """Split-K over a [2,3] batch with B broadcast over the first dimension (stride 0) and read
    transposed, and C0 == C (the reduction reads and writes each element in place)."""
    bsz, heads, m, n, k = 2, 3, 70, 45, 777
    a = quarter_matrix(bsz * heads * m, k, 181).reshape(bsz, heads, m, k)
    bt = quarter_matrix(heads * n, k, 182).reshape(1, heads, n, k)
    c0 = quarter_matrix(bsz * heads * m, n, 183).reshape(bsz, heads, m, n)
    b_d = dev(bt, stream).expand((bsz, heads, n, k)).transpose(-2, -1)
    for splits in (4, 7):
        c = dev(c0, stream)
        mf.gemm_batched(dev(a, stream), b_d, c, alpha=0.25, c0=c, beta=-2.0, splits=splits)
        got = c.numpy()
        for i in range(bsz):
            for h in range(heads):
                prod = exact_product(a[i, h], bt[0, h].T)
                want = (np.float32(0.25) * prod) + (np.float32(-2.0) * c0[i, h])
                assert same_bits(got[i, h], want.astype(np.float32)), (splits, i, h)


def test_split_k_short_depths(stream):
    """More ranges asked for than the depth allows runs fewer (ranges are 32 deep at least);
    k == 0 runs no split and gives the epilogue of a zero product."""
    m, n = 33, 65
    for k in (1, 31, 33, 40, 95):
        a = quarter_matrix(m, k, 191 + k)
        b = quarter_matrix(k, n, 192 + k)
        a_d, b_d = dev(a, stream), dev(b, stream)
        c, buf = guarded_output(stream, (m, n))
        assert mf.gemm_plan(a_d, b_d, c, splits=8)[2] == ranges_run(k, 8)
        mf.gemm(a_d, b_d, out=c, splits=8)
        assert same_bits(c.numpy(), exact_product(a, b)), k
        check_guards(buf)
    c0 = quarter_matrix(m, n, 199)
    a = mf.DeviceArray.empty((m, 0), stream)
    b = mf.DeviceArray.empty((0, n), stream)
    c, _ = guarded_output(stream, (m, n))
    assert mf.gemm_plan(a, b, c, splits=4)[2] == 1
    mf.gemm(a, b, alpha=2.0, c0=dev(c0, stream), beta=0.5, out=c, splits=4)
    assert same_bits(c.numpy(), (np.float32(0.5) * c0).astype(np.float32))


def test_split_k_invalid_counts(stream):
    a = dev(np.ones((8, 64), np.float32), stream)
    b = dev(np.ones((64, 8), np.float32), stream)
    for splits in (-1, mf.abi.MAX_SPLITS + 1):
        with pytest.raises(ValueError):
            mf.gemm(a, b, splits=splits)
    assert np.all(mf.gemm(a, b, splits=mf.abi.MAX_SPLITS).numpy() == 64.0)


def test_split_k_gelu_same_bits_as_unsplit(stream, oracle):
    """The activation sees the same pre-activation value split or not (exact inputs), so the
    outputs agree in every bit, and equal the oracle's gelu of the exact pre-activation."""
    m, n, k = 96, 200, 2048
    av, bv = quarter_matrix(m, k, 201), quarter_matrix(k, n, 202)
    biasv = quarter_matrix(1, n, 203)[0]
    a, b, bias = dev(av, stream), dev(bv, stream), dev(biasv, stream)
    one = mf.gemm(a, b, bias=bias, act=mf.ACT_GELU_TANH, splits=1).numpy()
    want = oracle.gelu((exact_product(av, bv) + biasv).astype(np.float32), approximate=True)
    assert same_bits(one, want)
    for splits in (2, 16):
        got = mf.gemm(a, b, bias=bias, act=mf.ACT_GELU_TANH, splits=splits).numpy()
        assert same_bits(got, one), splits


@pytest.mark.parametrize("tile", TILES + [mf.abi.TILE_THIN])
def test_epilogue_gelu_bits_equal_oracle(stream, oracle, tile):
    """gelu-tanh in every tile's epilogue (and the thin path's) on exact pre-activation values
    (quarter integers, widely spread by alpha): the oracle's bits, element for element."""
    m, n, k = (300, 8, 77) if tile == mf.abi.TILE_THIN else (300, 260, 96)
    av, bv = quarter_matrix(m, k, 211), quarter_matrix(k, n, 212)
    biasv = quarter_matrix(1, n, 213)[0]
    for alpha in (0.03125, 1.0, 0.125):
        pre = (np.float32(alpha) * exact_product(av, bv) + biasv).astype(np.float32)
        got = mf.gemm(dev(av, stream), dev(bv, stream), alpha=alpha, bias=dev(biasv, stream),
                      act=mf.ACT_GELU_TANH, tile=tile).numpy()
        assert same_bits(got, oracle.gelu(pre, approximate=True)), alpha


@pytest.mark.parametrize("tile", TILES)
def test_gelu_row_edge_tiles_drop_rows_past_m(stream, oracle, tile):
    """Tiles whose columns are all inside C but whose rows run past m compute every row and
    store through a buffer resource of m rows, which drops the stores past m: C is an exact
    output inside a poisoned buffer (the rows past m would land in the guard after it), and the
    values are the oracle's bits."""
    m, n, k = 300, 256, 96
    av, bv = quarter_matrix(m, k, 221), quarter_matrix(k, n, 222)
    biasv = quarter_matrix(1, n, 223)[0]
    out, buf = guarded_output(stream, (m, n), guard=64 * 1024)
    mf.gemm(dev(av, stream), dev(bv, stream), bias=dev(biasv, stream), act=mf.ACT_GELU_TANH,
            tile=tile, out=out)
    check_guards(buf, guard=64 * 1024)
    pre = (exact_product(av, bv) + biasv).astype(np.float32)
    assert same_bits(out.numpy(), oracle.gelu(pre, approximate=True))


def test_split_k_automatic_choice(stream):
    """AUTO splits a product with few output tiles and a long depth, and leaves products that
    fill the device (4096^3, the MLP) or have a short depth unsplit."""
    def plan(m, n, k):
        return mf.gemm_plan(mf.DeviceArray.empty((m, k), stream),
                            mf.DeviceArray.empty((k, n), stream),
                            mf.DeviceArray.empty((m, n), stream))
    assert plan(256, 256, 16384)[2] > 1
    assert plan(512, 512, 8192)[2] > 1
    assert plan(4096, 4096, 4096)[2] == 1
    assert plan(4093, 4099, 1023)[2] == 1
    assert plan(256, 256, 256)[2] == 1


@pytest.mark.parametrize("m,n,k", [(256, 256, 16384), (128, 4096, 4096), (1000, 1000, 3000)])
def test_split_k_realistic(stream, oracle, m, n, k):
    """Split-K (as AUTO picks it, and fixed at 8) on normal inputs against the packed CPU GEMM,
    to the 1e-5*sqrt(K) bar; deterministic from call to call."""
    a = normal(oracle, (m, k), 0.0, 1.0, 11, 0)
    b = normal(oracle, (k, n), 0.0, 1.0, 12, 0)
    a_d, b_d = dev(a, stream), dev(b, stream)
    want = oracle.matmul(a, b)
    scale = magnitude(oracle, a, b)
    for splits in (0, 8):
        got = mf.gemm(a_d, b_d, splits=splits).numpy()
        assert_gemm_parity(got, want, scale, k, f"split {splits}")
        assert same_bits(got, mf.gemm(a_d, b_d, splits=splits).numpy())


@pytest.mark.parametrize("m,n,k,regions", [(4093, 4099, 1023, 2), (4099, 4093, 1023, 2),
                                           (4099, 4099, 2048, 4)])
def test_peeled_edges_exact(stream, m, n, k, regions):
    """AUTO peels edge strips a big tile would waste a wave on into launches of their own: the
    MLP's 3 extra columns, 3 extra rows, and both (main, right strip, bottom strip, corner).
    Quarter-integer inputs with alpha, beta*C0 and a bias: every region's bits equal the exact
    product, which pins each strip's offsets into A, B, C, C0 and the bias; no stray writes."""
    a = quarter_matrix(m, k, 211)
    b = quarter_matrix(k, n, 212)
    c0 = quarter_matrix(m, n, 213)
    bias = quarter_matrix(1, n, 214)[0]
    want = (np.float32(1.5) * exact_product(a, b)) + np.float32(0.5) * c0
    want = (want + bias).astype(np.float32)
    a_d, b_d, c0_d = dev(a, stream), dev(b, stream), dev(c0, stream)
    c, buf = guarded_output(stream, (m, n))
    assert mf.gemm_plan(a_d, b_d, c, c0=c0_d, beta=0.5)[3] == regions
    mf.gemm(a_d, b_d, alpha=1.5, c0=c0_d, beta=0.5, bias=dev(bias, stream), out=c)
    assert same_bits(c.numpy(), want)
    check_guards(buf)
    # A fixed tile or split count runs one region.
    assert mf.gemm_plan(a_d, b_d, c, tile=mf.abi.TILE_64x64)[3] == 1
    assert mf.gemm_plan(a_d, b_d, c, splits=1)[3] == 1


@pytest.mark.parametrize("bsz,m,n,k", [(2, 4093, 2051, 1023), (3, 2049, 2047, 2048)])
def test_peeled_edges_batched_broadcast_exact(stream, bsz, m, n, k):
    """Peeling on a batch, B broadcast over it (batch stride 0), with alpha, beta*C0 and a bias:
    the strips' offsets combine with every matrix's batch offsets."""
    a = quarter_matrix(bsz * m, k, 261).reshape(bsz, m, k)
    b = quarter_matrix(k, n, 262)
    c0 = quarter_matrix(bsz * m, n, 263).reshape(bsz, m, n)
    bias = quarter_matrix(1, n, 264)[0]
    a_d = dev(a, stream)
    b_d = dev(b.reshape(1, k, n), stream).expand((bsz, k, n))
    c0_d = dev(c0, stream)
    out = mf.DeviceArray.empty((bsz, m, n), stream)
    assert mf.gemm_plan(a_d, b_d, out, c0=c0_d, beta=0.5)[3] == 2
    mf.gemm_batched(a_d, b_d, out, alpha=1.5, c0=c0_d, beta=0.5, bias=dev(bias, stream))
    got = out.numpy()
    for i in range(bsz):
        want = (np.float32(1.5) * exact_product(a[i], b)) + np.float32(0.5) * c0[i]
        assert same_bits(got[i], (want + bias).astype(np.float32)), i


# ---- the thin path ------------------------------------------------------------------------------

THIN = mf.abi.TILE_THIN


@pytest.mark.parametrize("m,n,k", [(4093, 3, 1023), (4096, 8, 1024), (300, 1, 77), (17, 5, 2500),
                                   (1, 1, 1), (9, 8, 3), (257, 2, 515), (100, 4, 64), (33, 7, 9)])
def test_thin_exact_rows(stream, m, n, k):
    """n <= 8 with A read along k (4-byte loads for odd k, 16-byte for k % 4 == 0), with alpha,
    beta*C0 and a bias: the thin path's bits equal the exact product; no stray writes. The
    column counts cover every kernel width (1, 2, 4, 8 computed columns)."""
    a = quarter_matrix(m, k, 221)
    b = quarter_matrix(k, n, 222)
    c0 = quarter_matrix(m, n, 223)
    bias = quarter_matrix(1, n, 224)[0]
    want = (np.float32(1.5) * exact_product(a, b)) + np.float32(0.5) * c0
    want = (want + bias).astype(np.float32)
    for b_stored_t in (False, True):
        for stage in (mf.abi.STAGE_AUTO, mf.abi.STAGE_ALWAYS):
            # Staged, A's lines are padded to a multiple of 4 and read with 16-byte loads even
            # for odd k; B has no depth past k, which must not be read.
            b_d = dev(np.ascontiguousarray(b.T), stream).T if b_stored_t else dev(b, stream)
            c, buf = guarded_output(stream, (m, n))
            mf.gemm(dev(a, stream), b_d, alpha=1.5, c0=dev(c0, stream), beta=0.5,
                    bias=dev(bias, stream), out=c, tile=THIN, stage=stage)
            assert same_bits(c.numpy(), want), (b_stored_t, stage)
            check_guards(buf)


@pytest.mark.parametrize("m,n,k", [(3, 4099, 1023), (8, 4096, 1024), (1, 300, 77), (5, 17, 2500),
                                   (2, 600, 130)])
def test_thin_exact_transposed(stream, m, n, k):
    """m <= 8 with B read along k (B stored [n, k], read transposed): the thin path computes
    C^T = B^T A^T row by row of B^T; bits equal the exact product, bias per column of C."""
    a = quarter_matrix(m, k, 231)
    b_stored = quarter_matrix(n, k, 232)
    c0 = quarter_matrix(m, n, 233)
    bias = quarter_matrix(1, n, 234)[0]
    want = (np.float32(0.25) * exact_product(a, b_stored.T)) + np.float32(-2.0) * c0
    want = (want + bias).astype(np.float32)
    for a_stored_t in (False, True):
        a_d = dev(np.ascontiguousarray(a.T), stream).T if a_stored_t else dev(a, stream)
        c, buf = guarded_output(stream, (m, n))
        mf.gemm(a_d, dev(b_stored, stream), trans_b=True, alpha=0.25, c0=dev(c0, stream),
                beta=-2.0, bias=dev(bias, stream), out=c, tile=THIN)
        assert same_bits(c.numpy(), want), a_stored_t
        check_guards(buf)


def test_thin_batched_broadcast_gelu(stream):
    """A [2,3] batch with B broadcast over the first dimension; gelu on the thin path gives the
    bits an MFMA tile gives (the same exact pre-activation values)."""
    bsz, heads, m, n, k = 2, 3, 70, 5, 300
    a = quarter_matrix(bsz * heads * m, k, 241).reshape(bsz, heads, m, k)
    bv = quarter_matrix(heads * k, n, 242).reshape(1, heads, k, n)
    b_d = dev(bv, stream).expand((bsz, heads, k, n))
    bias = dev(quarter_matrix(1, n, 243)[0], stream)
    thin = mf.DeviceArray.empty((bsz, heads, m, n), stream)
    tiled = mf.DeviceArray.empty((bsz, heads, m, n), stream)
    mf.gemm_batched(dev(a, stream), b_d, thin, bias=bias, act=mf.ACT_GELU_TANH, tile=THIN)
    mf.gemm_batched(dev(a, stream), b_d, tiled, bias=bias, act=mf.ACT_GELU_TANH,
                    tile=mf.abi.TILE_64x64)
    assert same_bits(thin.numpy(), tiled.numpy())
    plain = mf.DeviceArray.empty((bsz, heads, m, n), stream)
    mf.gemm_batched(dev(a, stream), b_d, plain, tile=THIN)
    got = plain.numpy()
    for i in range(bsz):
        for h in range(heads):
            assert same_bits(got[i, h], exact_product(a[i, h], bv[0, h])), (i, h)


@pytest.mark.parametrize("n,pad", [(4, 0), (4, 2), (8, 0), (8, 4), (2, 0), (2, 1)])
def test_thin_b_pieces_and_batch_strides(stream, n, pad):
    """A batched product with 2, 4 or 8 columns and B's batches `pad` floats apart beyond their
    k*n. An even (2 columns) or multiple-of-4 batch stride lets the thin path read B's rows as
    8- or 16-byte pieces; an odd one, or 2 floats with 4 columns, makes it read one value at a
    time. Both give the exact product's bits."""
    batch, m, k = 3, 70, 130
    a = quarter_matrix(batch * m, k, 261).reshape(batch, m, k)
    bv = quarter_matrix(batch * k, n, 262).reshape(batch, k, n)
    per = k * n + pad
    stored = np.full((batch * per,), -5.0, np.float32)
    for i in range(batch):
        stored[i * per:i * per + k * n] = bv[i].reshape(-1)
    b_d = dev(stored, stream)._view((batch, k, n), (per, n, 1), 0)
    c = mf.DeviceArray.empty((batch, m, n), stream)
    mf.gemm_batched(dev(a, stream), b_d, c, tile=THIN)
    got = c.numpy()
    for i in range(batch):
        assert same_bits(got[i], exact_product(a[i], bv[i])), (n, pad, i)


@pytest.mark.parametrize("batch,m,n,k", [(1, 2000, 8, 1300), (3, 500, 8, 700), (1, 16, 8, 513),
                                         (2, 37, 6, 2049), (1, 1000, 7, 4096)])
def test_thin_lds_exact(stream, batch, m, n, k):
    """8 computed columns read as 16-byte pieces from 16 rows on: B' staged through LDS in groups
    of 512 depths (thin_dot_lds_kernel). Depths past the last group's end, a batch with B
    broadcast, 6 and 7 columns (B staged, its lines padded to 8), alpha, beta*C0 and a bias:
    bits equal the exact product, no stray writes."""
    a = quarter_matrix(batch * m, k, 291).reshape(batch, m, k)
    b = quarter_matrix(k, n, 292)
    c0 = quarter_matrix(batch * m, n, 293).reshape(batch, m, n)
    bias = quarter_matrix(1, n, 294)[0]
    want = np.stack([(np.float32(0.5) * exact_product(a[i], b)) + np.float32(2.0) * c0[i]
                     for i in range(batch)])
    want = (want + bias).astype(np.float32)
    # Staged, A's lines (odd k) take 16-byte loads and B's lines are padded to 8 columns.
    stage = mf.abi.STAGE_ALWAYS if n % 4 or k % 4 else mf.abi.STAGE_AUTO
    b_d = dev(b, stream).expand((batch, k, n))
    buf = mf.DeviceArray.empty((batch * m * n + 128,), stream)
    mf.fill(buf, POISON)
    c = buf.slice(0, 64, 64 + batch * m * n).view((batch, m, n))
    mf.gemm_batched(dev(a, stream), b_d, c, alpha=0.5, c0=dev(c0, stream), beta=2.0,
                    bias=dev(bias, stream), tile=THIN, stage=stage)
    assert same_bits(c.numpy(), want)
    check_guards(buf)


def test_thin_k_zero_and_refusals(stream):
    m, n = 33, 4
    c0 = quarter_matrix(m, n, 251)
    c, _ = guarded_output(stream, (m, n))
    mf.gemm(mf.DeviceArray.empty((m, 0), stream), mf.DeviceArray.empty((0, n), stream),
            alpha=2.0, c0=dev(c0, stream), beta=0.5, out=c, tile=THIN)
    assert same_bits(c.numpy(), (np.float32(0.5) * c0).astype(np.float32))
    wide = dev(np.ones((64, 64), np.float32), stream)
    with pytest.raises(NotImplementedError):        # n > 8 and m > 8
        mf.gemm(wide, wide, tile=THIN)
    a_t = dev(np.ones((64, 300), np.float32), stream).T  # [300, 64], unit stride along m
    with pytest.raises(NotImplementedError):        # n <= 8 but A not read along k
        mf.gemm(a_t, dev(np.ones((64, 3), np.float32), stream), tile=THIN)
    with pytest.raises(NotImplementedError):        # no split on the thin path
        mf.gemm(dev(np.ones((300, 64), np.float32), stream),
                dev(np.ones((64, 3), np.float32), stream), tile=THIN, splits=2)


def test_big_tile_slice_offset_limit(stream):
    """The 256x256 tile addresses each depth slice with 32-bit offsets below 2^30 bytes. An
    operand whose rows lie 2^22 floats apart (a slice of 256 such rows spans 4 GiB) makes a fixed
    256x256 tile refused, for 4-byte and 16-byte loads alike; AUTO takes another tile, and the
    bits are exact (quarter-integer inputs)."""
    far = 1 << 22
    for k in (5, 8):  # 4-byte loads (odd k), 16-byte loads
        m, n = 3, 40
        a = quarter_matrix(m, k, 271)
        b = quarter_matrix(k, n, 272)
        host = np.zeros((m, far), np.float32)
        host[:, :k] = a
        a_view = dev(host, stream).slice(1, 0, k)  # [m, k], rows 2^22 floats apart
        b_d = dev(b, stream)
        with pytest.raises(NotImplementedError):
            mf.gemm(a_view, b_d, tile=mf.abi.TILE_256x256, stage=mf.abi.STAGE_NEVER)
        assert mf.gemm_plan(a_view, b_d, mf.DeviceArray.empty((m, n), stream),
                            stage=mf.abi.STAGE_NEVER)[0] != mf.abi.TILE_256x256
        got = mf.gemm(a_view, b_d, stage=mf.abi.STAGE_NEVER).numpy()
        assert same_bits(got, exact_product(a, b).astype(np.float32)), k


def test_thin_automatic_choice(stream):
    """AUTO takes the thin path for a long product with a few columns (the MLP's 3-column edge
    strip, 4 aligned columns), and the MFMA tiles where the output fills them."""
    def plan(m, n, k, **kw):
        return mf.gemm_plan(mf.DeviceArray.empty((m, k), stream),
                            mf.DeviceArray.empty((k, n), stream),
                            mf.DeviceArray.empty((m, n), stream), **kw)
    assert plan(4093, 3, 1023)[0] == THIN
    assert plan(16384, 1, 16384)[0] == THIN
    # 4 aligned columns: B rows read as 16-byte pieces (51 us against 101 us on 64x64 tiles).
    assert plan(16384, 4, 4096)[0] == THIN
    # 8 aligned columns: B' staged in LDS (55.6 us against 101 us for 64x64 split 4).
    assert plan(16384, 8, 4096)[0] == THIN
    assert plan(4096, 4096, 4096)[0] == mf.abi.TILE_256x256


def test_unknown_stage_mode_is_invalid(stream):
    a = dev(np.ones((4, 4), np.float32), stream)
    with pytest.raises(ValueError):
        mf.gemm(a, a, stage=7)


def test_k_zero_gives_epilogue_of_zero_product(stream):
    m, n = 33, 17
    c0 = quarter_matrix(m, n, 41)
    a = mf.DeviceArray.empty((m, 0), stream)
    b = mf.DeviceArray.empty((0, n), stream)
    c, _ = guarded_output(stream, (m, n))
    mf.gemm(a, b, out=c)
    assert np.all(c.numpy() == 0.0)
    mf.gemm(a, b, alpha=2.0, c0=dev(c0, stream), beta=0.5, out=c)
    assert same_bits(c.numpy(), (np.float32(0.5) * c0).astype(np.float32))


def test_empty_outputs_touch_nothing(stream):
    c, buf = guarded_output(stream, (0, 5))
    mf.gemm(mf.DeviceArray.empty((0, 4), stream), dev(np.ones((4, 5), np.float32), stream), out=c)
    check_guards(buf)


def test_batched_broadcast_and_transposed(stream):
    """gemm_strided_batched semantics: a [2,3,m,k] batch times a b broadcast over the first
    batch dimension (stride 0), read transposed."""
    bsz, heads, m, n, k = 2, 3, 70, 45, 96
    a = quarter_matrix(bsz * heads * m, k, 51).reshape(bsz, heads, m, k)
    bt = quarter_matrix(heads * n, k, 52).reshape(1, heads, n, k)  # stored [.., n, k]
    c0 = quarter_matrix(bsz * heads * m, n, 53).reshape(bsz, heads, m, n)
    a_d = dev(a, stream)
    b_d = dev(bt, stream).expand((bsz, heads, n, k)).transpose(-2, -1)  # [2,3,k,n], batch stride 0
    c0_d = dev(c0, stream)
    out = mf.DeviceArray.empty((bsz, heads, m, n), stream)
    mf.gemm_batched(a_d, b_d, out, alpha=0.25, c0=c0_d, beta=-2.0)
    got = out.numpy()
    for i in range(bsz):
        for h in range(heads):
            prod = exact_product(a[i, h], bt[0, h].T)
            want = (np.float32(0.25) * prod) + (np.float32(-2.0) * c0[i, h])
            assert same_bits(got[i, h], want.astype(np.float32)), (i, h)


def test_config1_matmul_1024_realistic(stream, oracle):
    """A, B [1024,1024] uniform[-1,1] from seed 0 (A at offset 0, B after
    it), alpha 1, beta 0 -- against the packed CPU GEMM's arithmetic."""
    n = 1024
    a = uniform(oracle, (n, n), -1.0, 1.0, 0, 0)
    b = uniform(oracle, (n, n), -1.0, 1.0, 0, n * n)
    got = mf.gemm(dev(a, stream), dev(b, stream)).numpy()
    want = oracle.matmul(a, b)
    rel_mag, rel_max = assert_gemm_parity(got, want, magnitude(oracle, a, b), n, "cfg1")
    print(f"cfg1 1024^3: rel err vs magnitude {rel_mag:.3e}, vs max|C| {rel_max:.3e}")
    record_parity("cfg1_matmul_1024", rel_err_vs_magnitude=rel_mag, rel_err_vs_max=rel_max,
                  bar=tolerance(n), bit_identical_share=float(np.mean(same_elements(got, want))))


def test_config3_gemm_4096_nt_exact(stream):
    """BASELINE configs[2] shape and epilogue (transB, alpha 1.5, beta 0.5) at full size with
    quarter-integer inputs: exact in any order, so every bit must match."""
    n = 4096
    a = quarter_matrix(n, n, 61)
    b_stored = quarter_matrix(n, n, 62)  # B is read transposed
    c0 = quarter_matrix(n, n, 63)
    c = mf.gemm(dev(a, stream), dev(b_stored, stream), alpha=1.5, c0=dev(c0, stream), beta=0.5,
                trans_b=True).numpy()
    exact = a.astype(np.float64) @ b_stored.T.astype(np.float64)
    want = (np.float32(1.5) * exact.astype(np.float32)) + np.float32(0.5) * c0
    assert same_bits(c, want.astype(np.float32))


def test_config3_gemm_4096_nt_realistic(stream, oracle):
    """BASELINE configs[2] with its own inputs at full size: A, B uniform[-1,1], C0 ~ N(0,1),
    from a seed; against the packed CPU GEMM's arithmetic and mensurflow::gemm's roundings."""
    n = 4096
    seed = 3
    a = uniform(oracle, (n, n), -1.0, 1.0, seed, 0)
    b_stored = uniform(oracle, (n, n), -1.0, 1.0, seed, n * n)
    c0 = normal(oracle, (n, n), 0.0, 1.0, seed + 1, 0)
    got = mf.gemm(dev(a, stream), dev(b_stored, stream), alpha=1.5, c0=dev(c0, stream), beta=0.5,
                  trans_b=True).numpy()
    want = oracle.gemm(a, b_stored, 1.5, c0, 0.5, trans_b=True)
    scale = 1.5 * magnitude(oracle, a, b_stored.T) + 0.5 * np.abs(c0)
    rel_mag, rel_max = assert_gemm_parity(got, want, scale, n, "cfg3")
    print(f"cfg3 4096^3 NT: rel err vs magnitude {rel_mag:.3e}, vs max|C| {rel_max:.3e}")
    record_parity("cfg3_gemm_4096_nt", rel_err_vs_magnitude=rel_mag, rel_err_vs_max=rel_max,
                  bar=tolerance(n), bit_identical_share=float(np.mean(same_elements(got, want))))


def test_config4_fused_epilogue_equals_unfused_chain(stream, oracle):
    """BASELINE configs[3] at full size: the fused bias + gelu-tanh epilogue (exp table in LDS,
    interior and row-edge copies, the strip's launch with the copy of X) gives the bits of the
    unfused chain on the same device: the product without an epilogue, then mfr_bias_act's
    gelu (its own kernel, table read from global memory). Both sides run the same plan, so the
    pre-activation values are the same floats."""
    m, k, n = 4093, 1023, 4099
    x = normal(oracle, (m, k), 0.0, 1.0, 7, 0)
    w = normal(oracle, (k, n), 0.0, float(np.sqrt(1.0 / 1023.0)), 8, 0)
    bias = uniform(oracle, (n,), -0.1, 0.1, 9, 0)
    x_d, w_d, b_d = dev(x, stream), dev(w, stream), dev(bias, stream)
    fused = mf.gemm(x_d, w_d, bias=b_d, act=mf.ACT_GELU_TANH).numpy()
    chain = mf.bias_act(mf.gemm(x_d, w_d), b_d, mf.ACT_GELU_TANH).numpy()
    assert same_bits(fused, chain)


def test_config4_mlp_fused_bias_gelu(stream, oracle):
    """X[4093,1023] x W[1023,4099] + bias, gelu-tanh fused in the epilogue,
    against the reference's three-op chain gelu(bias_add(matmul(X, W), b), true).

    Row argmax is bit-exact, as the north star asks: the GPU's index equals the oracle's on every
    one of the 4093 rows (both sides are deterministic). The rows whose top two values lie within
    twice the error bar (near ties that another summation order could flip) are counted and
    recorded as a diagnostic, with the number of rows that differ (0)."""
    m, k, n = 4093, 1023, 4099
    x = normal(oracle, (m, k), 0.0, 1.0, 7, 0)
    w = normal(oracle, (k, n), 0.0, float(np.sqrt(1.0 / 1023.0)), 8, 0)
    bias = uniform(oracle, (n,), -0.1, 0.1, 9, 0)
    out_d = mf.gemm(dev(x, stream), dev(w, stream), bias=dev(bias, stream), act=mf.ACT_GELU_TANH)
    out = out_d.numpy()
    gpu_argmax = mf.argmax(out_d).numpy()
    want = oracle.gelu(oracle.bias_add(oracle.matmul(x, w), bias), approximate=True)
    # gelu'(v) <= 1.13, so the pre-activation scale bounds the output's error scale.
    scale = 1.13 * (magnitude(oracle, x, w) + np.abs(bias))
    rel_mag, rel_max = assert_gemm_parity(out, want, scale, k, "cfg4")
    want_arg = oracle.argmax(want)
    top2 = np.sort(want, axis=1)[:, -2:]
    margin = top2[:, 1] - top2[:, 0]
    bar = 1e-5 * np.sqrt(k) * scale.max(axis=1)
    decided = margin > 2 * bar
    differ = np.nonzero(gpu_argmax != want_arg)[0]
    print(f"cfg4: rel err vs magnitude {rel_mag:.3e}, vs max|C| {rel_max:.3e}; argmax: "
          f"{int(decided.sum())} decided rows, {int((~decided).sum())} near-tie rows, "
          f"{differ.size} rows differ")
    record_parity("cfg4_mlp_bias_gelu", rel_err_vs_magnitude=rel_mag, rel_err_vs_max=rel_max,
                  bar=tolerance(k), bit_identical_share=float(np.mean(same_elements(out, want))),
                  argmax_rows=m, argmax_decided_rows=int(decided.sum()),
                  argmax_near_tie_rows=int((~decided).sum()), argmax_differing_rows=int(differ.size),
                  argmax_differing_row_ids=[int(r) for r in differ])
    assert np.array_equal(gpu_argmax, want_arg), f"argmax differs on rows {differ.tolist()}"


def test_deterministic(stream):
    a = dev(np.random.default_rng(5).standard_normal((300, 500)).astype(np.float32), stream)
    b = dev(np.random.default_rng(6).standard_normal((500, 260)).astype(np.float32), stream)
    first = mf.gemm(a, b).numpy()
    second = mf.gemm(a, b).numpy()
    assert same_bits(first, second)


def test_unsupported_and_invalid(stream):
    a = dev(np.ones((8, 8), np.float32), stream)
    # a view with no unit stride (every other row and column)
    odd = dev(np.ones((16, 16), np.float32), stream)
    odd = mf.DeviceArray(odd.shape, np.float32, stream, _base=odd, _offset=0,
                         _strides=(32, 2), _ptr=odd._ptr)
    odd.shape = (8, 8)
    with pytest.raises(NotImplementedError):
        mf.gemm(odd, a)
    with pytest.raises(ValueError):
        mf.gemm(a, dev(np.ones((7, 8), np.float32), stream))


def test_repeated_shapes_with_new_operands(stream, oracle):
    """The same shapes called again (mfr_sgemm reuses its plan for them) with other buffers, an
    operand moved off a 16-byte boundary, other alpha/beta/bias/activation values and C0 present
    or absent: every call equals its exact result."""
    m, n, k = 300, 260, 516
    rng = np.random.default_rng(77)
    for trial in range(8):
        av = quarter_matrix(m, k, 300 + trial)
        bv = quarter_matrix(k, n, 400 + trial)
        shift = trial % 2  # odd trials read A one float into its storage (4-byte loads)
        store = np.zeros(m * k + shift, np.float32)
        store[shift:] = av.ravel()
        a_d = dev(store, stream).slice(0, shift, shift + m * k).view((m, k))
        alpha = float(rng.choice([1.0, 0.5, -2.0]))
        beta = float(rng.choice([0.0, 0.5]))
        c0v = quarter_matrix(m, n, 500 + trial)
        biasv = quarter_matrix(1, n, 600 + trial)[0]
        use_c0, use_bias = trial % 3 != 0, trial % 4 < 2
        act = [mf.ACT_NONE, mf.ACT_GELU_TANH][trial % 2]
        c, buf = guarded_output(stream, (m, n))
        mf.gemm(a_d, dev(bv, stream), alpha=alpha, c0=dev(c0v, stream) if use_c0 else None,
                beta=beta, bias=dev(biasv, stream) if use_bias else None, act=act, out=c)
        pre = np.float32(alpha) * exact_product(av, bv)
        if use_c0 and beta != 0.0:
            pre = pre + np.float32(beta) * c0v
        if use_bias:
            pre = pre + biasv
        pre = pre.astype(np.float32)
        want = oracle.gelu(pre, approximate=True) if act == mf.ACT_GELU_TANH else pre
        assert same_bits(c.numpy(), want), trial
        check_guards(buf)


@pytest.mark.parametrize("tile,k,line", [(mf.abi.TILE_64x64, 128, 2**22 + 2**18),
                                         (mf.abi.TILE_128x128, 64, 2**23 + 2**19)])
def test_deep_slices_with_long_lines(stream, tile, k, line):
    """The one-workgroup-per-CU 64x64 and 128x128 tiles read 128- and 64-deep slices straight
    into LDS through 32-bit byte offsets. An N-major B whose line stride puts such a slice past
    2^31 bytes (127 or 63 lines of ~17.8 or ~35.7 MB), while a 32-deep slice would stay inside,
    must not take that form: the product runs on the wavefront sets instead, exact."""
    size = 64 if tile == mf.abi.TILE_64x64 else 128
    a = quarter_matrix(size, k, 141)
    b = quarter_matrix(k, size, 142)
    stored = np.zeros((k, line), np.float32)  # ~2.3 GB, mostly untouched zero pages
    stored[:, :size] = b
    b_store = dev(stored, stream)
    del stored
    c, buf = guarded_output(stream, (size, size))
    mf.gemm(dev(a, stream), b_store.slice(1, 0, size), out=c, tile=tile, splits=1,
            stage=mf.abi.STAGE_NEVER)
    assert same_bits(c.numpy(), exact_product(a, b))
    check_guards(buf)
    b_store.close()


@pytest.mark.parametrize("tile,m,n,k", [
    (mf.abi.TILE_64x64, 1000, 1000, 1000), (mf.abi.TILE_64x64, 300, 260, 1023),
    (mf.abi.TILE_64x64, 64, 64, 2000), (mf.abi.TILE_64x64, 37, 100, 65),
    (mf.abi.TILE_64x64, 1024, 1024, 0), (mf.abi.TILE_128x128, 2000, 2048, 300),
    (mf.abi.TILE_128x128, 300, 260, 1023), (mf.abi.TILE_128x128, 129, 127, 70),
    (mf.abi.TILE_64x64, 1024, 1024, 1000), (mf.abi.TILE_64x64, 1024, 1024, 1023),
    (mf.abi.TILE_64x64, 512, 256, 36), (mf.abi.TILE_128x128, 2048, 2048, 300),
    (mf.abi.TILE_128x128, 1024, 2048, 1023), (mf.abi.TILE_128x128, 128, 128, 4),
    (mf.abi.TILE_128x128, 1500, 1460, 300), (mf.abi.TILE_64x64, 1000, 940, 68),
    (mf.abi.TILE_128x128, 4, 8, 40)])
def test_exact_sixteen_wave_set_forms(stream, tile, m, n, k):
    """Unsplit with at most one workgroup per CU, the 64x64 and 128x128 tiles run the
    direct-to-LDS kernel (one chain per lane) when both operands take 16-byte loads, edge tiles
    included (their rows outside the matrix load zeros through the fixed offsets); with a 4-byte
    operand the 64x64 tile runs 16 wavefronts in four sets and the 128x128 tile 16 in two, the
    sets sharing each depth slice and adding their accumulators through LDS. Either way bits
    equal the exact result in all four layouts (4-byte loads, so the sets, for odd k), with
    alpha, beta*C0 and a bias."""
    size = 64 if tile == mf.abi.TILE_64x64 else 128
    assert ((m + size - 1) // size) * ((n + size - 1) // size) <= mf.device_info(0).compute_units
    a = quarter_matrix(m, k, 91)
    b = quarter_matrix(k, n, 92)
    c0 = quarter_matrix(m, n, 93)
    bias = quarter_matrix(1, n, 94)[0]
    pre = (np.float32(0.5) * exact_product(a, b) + np.float32(1.5) * c0 + bias).astype(np.float32)
    for trans_a in (False, True):
        for trans_b in (False, True):
            a_st = np.ascontiguousarray(a.T) if trans_a else a
            b_st = np.ascontiguousarray(b.T) if trans_b else b
            c, buf = guarded_output(stream, (m, n))
            mf.gemm(dev(a_st, stream), dev(b_st, stream), alpha=0.5, c0=dev(c0, stream), beta=1.5,
                    trans_a=trans_a, trans_b=trans_b, bias=dev(bias, stream), out=c,
                    tile=tile, splits=1, stage=mf.abi.STAGE_NEVER)
            assert same_bits(c.numpy(), pre), (trans_a, trans_b)
            check_guards(buf)
