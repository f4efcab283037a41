"""The Q4_0 products against the oracle.

Integers: every per-block sum the GPU uses equals golem's dotQ4_0Go
accumulator minus 8*sum(q) (nn/dot_q4_0.go:58-63), bit for bit, exported by
the kernels that ship (gx_q4_0_block_dots: the SGPR-activation matrix-vector
kernel, the direct-to-LDS int8-MFMA product, the fp16-MFMA product and the
one-column LDS kernel in each of its tile shapes; gx_q4_0_fused_block_dots:
the fused norm products of the decode step).
Floats: golem's compareFloats bar (nn/quants_reference_test.go:96-120),
max |got - want| / RMS(want) <= 1e-5, against both of golem's generic forms
(row layout dotQ4_0Go and the 8-row packed dotPackedQ4_0Go) through
Matrix.rows.  Determinism: a column's result is bit-identical whatever the
batch (M = 1 .. 8 on the matrix-vector kernel, M > 8 on MFMA), golem's
"batch == one at a time" (nn/dot_q4_0.go:143-146).
"""
import numpy as np
import pytest

from golem_amd import capi, synth
from tests.gpu_util import log

pytestmark = pytest.mark.gpu

TOL = 1e-5


def setup(dev, orc, rows, cols, M, seed):
    g = synth.rng(seed)
    w = synth.q4_0_weights(g, rows, cols)
    x = synth.activations(g, M, cols)
    b = orc.Batch(x).quantize()
    wd = dev.weight(w, capi.Q4_0, rows, cols)
    act = dev.quantize_q8_0(x, with_corr=False)
    return w, b, wd, act


def test_dequantized_rows_cover_every_half(dev, orc):
    """Matrix.Row (dequantizeQ4_0Row, nn/matrix.go:175-190) bit for bit, over a
    matrix whose block scales run through every finite fp16 pattern: pins the
    device fp16 widening exhaustively."""
    halves = np.array([h for h in range(1 << 16) if (h >> 10) & 0x1F != 0x1F], dtype=np.uint16)
    cols = 256
    blocks_per_row = cols // 32
    rows = (len(halves) + blocks_per_row - 1) // blocks_per_row
    g = synth.rng(1)
    w = synth.q4_0_weights(g, rows, cols).reshape(-1, 18)
    d = np.resize(halves, rows * blocks_per_row)
    w[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    w = w.reshape(-1)
    wd = dev.weight(w, capi.Q4_0, rows, cols)
    ids = np.arange(rows, dtype=np.int32)
    got = dev.rows(wd, ids)
    want = np.stack([orc.dequantize_q4_0_row(w[r * blocks_per_row * 18:(r + 1) * blocks_per_row * 18], cols)
                     for r in range(rows)])
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,cols,M", [(64, 256, 1), (200, 2560, 3), (96, 704, 9), (130, 2816, 40),
                                         (300, 2560, 1)])
@pytest.mark.parametrize("path", [0, 1, 2, 3, 4, 5])
def test_block_integers_bit_exact(dev, orc, rows, cols, M, path):
    if path == 3 and M != 1:
        pytest.skip("the one-column kernel takes M = 1")
    if path == 5 and M > 16:
        pytest.skip("the few-column MFMA kernel takes at most 16 columns")
    log(f"q4_0 block dots rows={rows} cols={cols} M={M} path={path}")
    w, b, wd, act = setup(dev, orc, rows, cols, M, 100 + rows)
    start, end = (0, rows) if rows < 100 else (5, rows - 3)
    got = dev.q4_0_block_dots(wd, act, M, start, end, path)
    acc = orc.q4_0_block_acc(w, b, rows)[:, start:end, :]
    qsum = b.qsum_rows()[:, None, :]
    np.testing.assert_array_equal(got, acc - 8 * qsum)


@pytest.mark.parametrize("rows,cols,M,span", [
    (2560, 9728, 8, (0, 2560)),     # Down at 8 columns: two groups of 4 on quarter tiles
    (2560, 4096, 5, (17, 2500)),    # O: a group of 4 and one column, a range that cuts quarter tiles
    (6144, 2560, 8, (0, 6144)),     # Q|K|V: half tiles
    (19456, 2560, 3, (64, 19456)),  # Gate|Up: whole tiles
    (9728, 2560, 2, (0, 9728)),     # config 0's matrix
    (2560, 9728, 16, (3, 2557)),    # Down at 16 columns (path 4 in groups of 8)
    (200, 2816, 11, (0, 200)),      # a ragged last tile
    (300, 6144, 7, (0, 300)),       # 24 stretches: two a wavefront, weights in registers
    (100, 16640, 3, (2, 99)),       # 65 stretches: B operands straight from global memory
])
@pytest.mark.parametrize("path", [4, 5])
def test_multi_column_integers_every_shape(dev, orc, rows, cols, M, span, path):
    """Path 4 (the multi-column matrix-vector kernel) and path 5 (the
    few-column MFMA kernel golem's lock-step slots run, 2 to 16 columns), bit
    for bit against golem's accumulator, and every column of the product
    equal to that column's one-column product bit for bit (golem's batch ==
    one at a time, nn/dot_q4_0.go:143-146)."""
    if path == 4 and cols > 16384:
        pytest.skip("the multi-column matrix-vector kernel covers a row with at most 16 wavefronts of 4 stretches")
    log(f"multi-column dots rows={rows} cols={cols} M={M} span={span} path={path}")
    w, b, wd, act = setup(dev, orc, rows, cols, M, 900 + rows + M)
    start, end = span
    got = dev.q4_0_block_dots(wd, act, M, start, end, path)
    acc = orc.q4_0_block_acc(w, b, rows)[:, start:end, :]
    np.testing.assert_array_equal(got, acc - 8 * b.qsum_rows()[:, None, :])
    y = dev.get(dev.matmul_q4_0(wd, act, M, start, end))
    q, sc, qs = act[:3]
    for m in range(M):
        y1 = dev.full((1, rows), float("nan"))
        capi.call("gx_matmul_q4_0", dev.ctx.ptr, wd.ptr, capi.vp(q[m:m + 1]), capi.vp(sc[m:m + 1]),
                  capi.vp(qs[m:m + 1]), None, 1, start, end, None, capi.vp(y1), rows)
        y1 = dev.get(y1)[0]
        np.testing.assert_array_equal(y[m, start:end].view(np.uint32), y1[start:end].view(np.uint32))
    assert np.isnan(y[:, :start]).all() and np.isnan(y[:, end:]).all()


@pytest.mark.parametrize("rows,cols,span", [
    (2560, 9728, (0, 2560)),      # Down: 10 wavefronts a workgroup
    (2560, 4096, (17, 2500)),     # O, a range that cuts quarter tiles
    (9728, 2560, (0, 9728)),      # config 0's matrix (the product runs whole tiles there)
    (16448, 2560, (3, 16441)),    # 257 tiles
    (100, 16640, (0, 100)),       # 65 stretches: two stretches a lane
])
def test_one_column_integers_every_shape(dev, orc, rows, cols, span):
    """Path 3 -- the quarter-tile one-column kernel the decode's O and Down
    products run -- bit for bit against golem's accumulator, and its outputs
    equal the SGPR kernel's (path 0's) bit for bit."""
    log(f"one-column dots rows={rows} cols={cols} span={span}")
    w, b, wd, act = setup(dev, orc, rows, cols, 1, 700 + rows)
    start, end = span
    got = dev.q4_0_block_dots(wd, act, 1, start, end, 3)
    acc = orc.q4_0_block_acc(w, b, rows)[:, start:end, :]
    np.testing.assert_array_equal(got, acc - 8 * b.qsum_rows()[:, None, :])
    y = dev.get(dev.matmul_q4_0(wd, act, 1, start, end))[0]
    q, sc, qs = act[:3]
    y2 = dev.full((2, rows), float("nan"))
    # two columns, the second a copy of the first: the multi-column kernel computes both
    q2, sc2, qs2 = (torch_cat2(dev, t) for t in (q, sc, qs))
    capi.call("gx_matmul_q4_0", dev.ctx.ptr, wd.ptr, capi.vp(q2), capi.vp(sc2), capi.vp(qs2), None, 2, start, end,
              None, capi.vp(y2), rows)
    y2 = dev.get(y2)
    np.testing.assert_array_equal(y[start:end].view(np.uint32), y2[0, start:end].view(np.uint32))
    np.testing.assert_array_equal(y[start:end].view(np.uint32), y2[1, start:end].view(np.uint32))


def torch_cat2(dev, t):
    """Two rows of the same activation (a [1][n] device tensor)."""
    return dev.torch.cat([t, t], 0).contiguous()


def _fused_case(orc, g, rows, cols, with_add):
    w = synth.q4_0_weights(g, rows, cols)
    x = g.standard_normal(cols).astype(np.float32)
    add = g.standard_normal(cols).astype(np.float32) if with_add else None
    gain = (1.0 + 0.02 * g.standard_normal(cols)).astype(np.float32)
    xa = x + add if with_add else x.copy()
    normed = orc.rms_norm_plain(xa, gain, 1e-6)
    b = orc.Batch(normed[None, :]).quantize()
    return w, x, add, gain, b


@pytest.mark.parametrize("rows,cols,swiglu,span", [
    (6144, 2560, 0, (0, 6144)),    # config 3's Q|K|V
    (19456, 2560, 1, (0, 19456)),  # config 3's Gate|Up with the SwiGLU epilogue
    (1536, 512, 0, (5, 1500)),     # a small model's Q|K|V, a cut range
    (128, 8192, 1, (0, 128)),      # a long row: two stretch slots a wavefront
])
def test_fused_norm_integers(dev, orc, rows, cols, swiglu, span):
    """The fused one-position products (pre-norm + Q8_0 inside the kernel)
    export the integers of the Q8_0 form they made: golem's accumulator over
    Q8_0(RMSNormPlain(x + add, gain)) minus 8*sum(q), bit for bit."""
    g = synth.rng(800 + rows + swiglu)
    for with_add in (True, False):
        log(f"fused dots rows={rows} cols={cols} swiglu={swiglu} add={with_add}")
        w, x, add, gain, b = _fused_case(orc, g, rows, cols, with_add)
        wd = dev.weight(w, capi.Q4_0, rows, cols)
        xd, gd = dev.put(x), dev.put(gain)
        ad = dev.put(add) if with_add else None
        start, end = span
        out = dev.empty((end - start, cols // 32), np.int32)
        q8 = dev.empty((rows // 2,), np.int8) if swiglu else None
        s8 = dev.empty((rows // 64,), np.float32) if swiglu else None
        qs8 = dev.empty((rows // 64,), np.int32) if swiglu else None
        capi.call("gx_q4_0_fused_block_dots", dev.ctx.ptr, wd.ptr, swiglu, capi.vp(xd), capi.vp(ad), capi.vp(gd),
                  np.float32(1e-6), start, end, capi.vp(q8), capi.vp(s8), capi.vp(qs8), capi.vp(out))
        got = dev.get(out)
        acc = orc.q4_0_block_acc(w, b, rows)[0, start:end, :]
        np.testing.assert_array_equal(got, acc - 8 * b.qsum_rows()[0][None, :])
        wd.free()


def test_block_acc_oracle_agrees_with_c_loop(orc):
    """The numpy per-block accumulator used above equals the oracle's C loop."""
    g = synth.rng(5)
    rows, cols = 3, 256
    w = synth.q4_0_weights(g, rows, cols)
    b = orc.Batch(synth.activations(g, 2, cols)).quantize()
    acc = orc.q4_0_block_acc(w, b, rows)
    q = b.q_rows()
    wb = w.reshape(rows, cols // 32, 18)
    import ctypes
    lib = orc.load()
    for c in range(2):
        for r in range(rows):
            for blk in range(cols // 32):
                nib = np.ascontiguousarray(wb[r, blk, 2:])
                qq = np.ascontiguousarray(q[c, blk * 32:(blk + 1) * 32])
                v = lib.orc_q4_0_acc(nib.ctypes.data_as(ctypes.c_void_p), qq.ctypes.data_as(ctypes.c_void_p))
                assert v == acc[c, r, blk]


@pytest.mark.parametrize("rows,cols,M", [(9728, 2560, 1), (1024, 2560, 2), (2560, 9728, 1), (1408, 2816, 4),
                                         (2816, 704, 8), (136, 4096, 5), (77, 256, 3)])
def test_matvec_against_golem(dev, orc, rows, cols, M):
    log(f"q4_0 matvec rows={rows} cols={cols} M={M}")
    w, b, wd, act = setup(dev, orc, rows, cols, M, 200 + rows + M)
    got = dev.get(dev.matmul_q4_0(wd, act, M))
    row_form = orc.mat_vec_q4_0_rows(w, b, rows)
    packed = orc.pack_q4_0(w, rows, cols)
    packed_form = orc.matrix_rows(orc.Q4_0, w, rows, cols, b, packed=packed)
    for c in range(M):
        rel, at = orc.compare_floats(got[c], row_form[c])
        assert rel <= TOL, f"column {c}: {rel:.3g} of RMS at row {at} (row layout)"
        rel, at = orc.compare_floats(got[c], packed_form[c])
        assert rel <= TOL, f"column {c}: {rel:.3g} of RMS at row {at} (packed)"


@pytest.mark.parametrize("span", [(0, 130), (1, 129), (3, 11), (127, 130), (64, 128)])
def test_row_ranges_and_bias(dev, orc, span):
    """Only rows in [start, end) are written (pack_matvec_test.go:14 checks the
    same with NaN sentinels), and the bias is added to those rows
    (nn/matrix.go:126-130)."""
    rows, cols, M = 130, 2080, 12
    w, b, wd, act = setup(dev, orc, rows, cols, M, 300)
    bias = synth.activations(synth.rng(301), 1, rows)[0]
    start, end = span
    for m in (1, 6, M):
        log(f"range {span} M={m}")
        bm = orc.Batch(b.F[:m]).quantize()
        actm = dev.quantize_q8_0(b.F[:m], with_corr=False)
        got = dev.get(dev.matmul_q4_0(wd, actm, m, start, end, bias=bias))
        want = orc.matrix_rows(orc.Q4_0, w, rows, cols, bm, start, end, bias=bias)
        assert np.all(np.isnan(got[:, :start])) and np.all(np.isnan(got[:, end:]))
        assert not np.any(np.isnan(got[:, start:end]))
        for c in range(m):
            rel, at = orc.compare_floats(got[c, start:end], want[c, start:end])
            assert rel <= TOL, f"column {c}: {rel:.3g} at {at}"


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("rows,cols", [(9728, 2560), (2560, 9728), (2816, 704), (200, 2816)])
def test_batch_equals_one_at_a_time(dev, orc, rows, cols, f16):
    """Every column of a batch -- one column on the matrix-vector kernel, 2..16
    on the few-column MFMA kernel, larger M on the int8-MFMA kernel, with the
    fp16 copy given (f16) or withheld: the product reads only the int8 form
    either way -- is bit-identical to the same column computed alone."""
    M = 70
    g = synth.rng(400 + rows)
    w = synth.q4_0_weights(g, rows, cols)
    x = synth.activations(g, M, cols)
    # Scales that are fp16 subnormals, on both sides of the product: every
    # 7th weight block and two tokens whose Q8_0 scales fall below 2^-14.
    wb = w.reshape(-1, 18)
    sub = g.integers(1, 0x400, size=len(wb[::7]), dtype=np.uint16)
    wb[::7, 0:2] = sub.view(np.uint8).reshape(-1, 2)
    x[5] *= np.float32(3e-6)
    x[40] *= np.float32(1e-7)
    wd = dev.weight(w, capi.Q4_0, rows, cols)
    act = dev.quantize_q8_0(x, with_corr=False)
    log(f"batch==alone rows={rows} cols={cols} f16={f16}")
    whole = dev.get(dev.matmul_q4_0(wd, act, M, f16=f16))
    # Each sub-batch is quantised on its own (the fp16 copy is panel-ordered,
    # so a prefix of tokens is not a prefix of the buffer; the quantiser is
    # exact per token, which test_gpu_quant pins).
    for m in (1, 2, 3, 5, 8, 9, 16, 17, 33):
        part = dev.get(dev.matmul_q4_0(wd, dev.quantize_q8_0(x[:m], with_corr=False), m, f16=f16))
        np.testing.assert_array_equal(part.view(np.uint32), whole[:m].view(np.uint32))
    for c in (0, 17, 69):
        one = dev.quantize_q8_0(x[c:c + 1], with_corr=False)
        alone = dev.get(dev.matmul_q4_0(wd, one, 1))
        np.testing.assert_array_equal(alone[0].view(np.uint32), whole[c].view(np.uint32))


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("M", [64, 512, 2048])
def test_gemm_against_golem(dev, orc, M, f16):
    rows, cols = 9728, 2560
    log(f"q4_0 gemm M={M} f16={f16}")
    w, b, wd, act = setup(dev, orc, rows, cols, M, 500 + M)
    got = dev.get(dev.matmul_q4_0(wd, act, M, f16=f16))
    # The oracle on a sample of rows and columns (the whole product would take
    # the scalar oracle minutes).
    sel_rows = np.r_[0:64, 4000:4064, rows - 64:rows]
    cols_sel = [0, 1, M // 2, M - 1]
    sub = orc.Batch(b.F[cols_sel]).quantize()
    wsub = w.reshape(rows, -1)[sel_rows].reshape(-1)
    want = orc.mat_vec_q4_0_rows(wsub, sub, len(sel_rows))
    for i, c in enumerate(cols_sel):
        rel, at = orc.compare_floats(got[c, sel_rows], want[i])
        assert rel <= TOL, f"column {c}: {rel:.3g} at {at}"


def test_gemm_integers_config_2(dev, orc):
    """Config 2 at M = 2048: the int8-MFMA product's own per-block integers
    (direct-to-LDS kernel, biased chain) for 64 rows of every token, bit for
    bit against golem's accumulator; and its outputs for those rows against
    one token at a time through the matrix-vector kernel, bit for bit."""
    rows, cols, M = 9728, 2560, 2048
    w, b, wd, act = setup(dev, orc, rows, cols, M, 2)
    start, end = 4032, 4096
    log("config 2 M=2048 block dots, int8 MFMA")
    got = dev.q4_0_block_dots(wd, act, M, start, end, 1)
    wsub = w.reshape(rows, -1)[start:end].reshape(-1)
    acc = orc.q4_0_block_acc(wsub, b, end - start)
    np.testing.assert_array_equal(got, acc - 8 * b.qsum_rows()[:, None, :])
    y = dev.get(dev.matmul_q4_0(wd, act, M, f16=False))
    for c in (0, 1023, 2047):
        one = dev.quantize_q8_0(b.F[c:c + 1], with_corr=False)
        alone = dev.get(dev.matmul_q4_0(wd, one, 1))
        np.testing.assert_array_equal(alone[0].view(np.uint32), y[c].view(np.uint32))


def test_errors_are_golem_panics(dev):
    g = synth.rng(9)
    with pytest.raises(capi.GxError, match="multiple of the block size"):
        dev.weight(synth.q4_0_weights(g, 4, 64), capi.Q4_0, 4, 48)
    wd = dev.weight(synth.q4_0_weights(g, 4, 64), capi.Q4_0, 4, 64)
    act = dev.quantize_q8_0(synth.activations(g, 1, 64), with_corr=False)
    with pytest.raises(capi.GxError, match="out of"):
        dev.matmul_q4_0(wd, act, 1, 0, 5)


@pytest.mark.parametrize("rows,cols", [(2560, 9728), (2560, 4096), (200, 8192), (64, 4352), (100, 16640)])
def test_quarter_tile_matvec_equals_one_workgroup(dev, rows, cols):
    """One column of a matrix with few tiles runs on quarter tiles (a
    workgroup per 16 rows, a lane per (row, stretch)); more than 64 stretches
    (16640 inputs) fall back to whole tiles.  Every result equals, bit for
    bit, column 0 of a two-column product, which one workgroup per tile
    computes; so do row ranges that cut the quarters, with and without a
    bias, and rows outside the range keep their sentinels."""
    g = synth.rng(300 + rows)
    w = synth.q4_0_weights(g, rows, cols)
    wd = dev.weight(w, capi.Q4_0, rows, cols)
    bias = g.standard_normal(rows).astype(np.float32)
    log(f"quarter-tile matvec rows={rows} cols={cols}")
    for it in range(8):
        x = synth.activations(g, 2, cols)
        act = dev.quantize_q8_0(x, with_corr=False)
        one = dev.get(dev.matmul_q4_0(wd, [a[:1] for a in act[:3]] + [None], 1))
        two = dev.get(dev.matmul_q4_0(wd, act, 2))
        np.testing.assert_array_equal(one[0].view(np.uint32), two[0].view(np.uint32), err_msg=f"launch {it}")
    start, end = 7, rows - 5
    y = dev.put(np.full((1, rows), np.nan, np.float32))
    dev.matmul_q4_0(wd, [a[:1] for a in act[:3]] + [None], 1, start, end, bias=bias, y=y)
    got = dev.get(y)[0]
    want = two[0] + bias
    np.testing.assert_array_equal(got[start:end].view(np.uint32), want[start:end].view(np.uint32))
    assert np.isnan(got[:start]).all() and np.isnan(got[end:]).all()
    wd.free()
