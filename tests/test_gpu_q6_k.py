"""The Q6_K product against the oracle: bit for bit.

golem's dotQ6_KGo (nn/dot_q6_k.go:19-54) sums exact per-superblock integers
and applies (float(isum) * d) * kscale serially; the device kernel does the
same, so the per-superblock integers and the float outputs are compared bit
for bit (the benchmark's bar is 2e-5 of RMS; this is stricter).  Several
columns through one weight read give each column exactly its one-column
result, as golem's dotQ6_Kx2 does (dot_q6_k_x2_test.go:12).
"""
import numpy as np
import pytest

from golem_amd import capi, synth
from tests.gpu_util import log

pytestmark = pytest.mark.gpu


def setup(dev, orc, rows, cols, M, seed):
    g = synth.rng(seed)
    w = synth.q6_k_weights(g, rows, cols)
    x = synth.activations(g, M, cols)
    b = orc.Batch(x).quantize_k()
    wd = dev.weight(w, capi.Q6_K, rows, cols)
    act = dev.quantize_q8_k(x)
    return w, b, wd, act


def test_dequantized_rows(dev, orc):
    """DequantizeQ6_K (nn/dequant_q6_k.go:18-51) bit for bit."""
    rows, cols = 70, 512
    g = synth.rng(2)
    w = synth.q6_k_weights(g, rows, cols)
    wd = dev.weight(w, capi.Q6_K, rows, cols)
    ids = np.array([0, 5, 63, 64, 69, 5], dtype=np.int32)
    got = dev.rows(wd, ids)
    rb = cols // 256 * 210
    want = np.stack([orc.dequantize_q6_k(w[r * rb:(r + 1) * rb], cols) for r in ids])
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,cols,M", [(64, 256, 1), (130, 2560, 3)])
def test_block_integers_bit_exact(dev, orc, rows, cols, M):
    log(f"q6_k block dots rows={rows} cols={cols} M={M}")
    w, b, wd, act = setup(dev, orc, rows, cols, M, 600 + rows)
    got = dev.q6_k_block_dots(wd, act, M, 1, rows)
    want = orc.q6_k_block_isum(w, b, rows)[:, 1:rows, :]
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("rows,cols,M", [(151936, 2560, 1), (4096, 2560, 2), (1000, 2560, 8), (77, 512, 5)])
def test_matvec_bit_exact(dev, orc, rows, cols, M):
    log(f"q6_k matvec rows={rows} cols={cols} M={M}")
    w, b, wd, act = setup(dev, orc, rows, cols, M, 700 + M)
    got = dev.get(dev.matmul_q6_k(wd, act, M))
    want = orc.mat_vec_q6_k_rows(w, b, rows)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_columns_share_one_read(dev, orc):
    rows, cols, M = 300, 2560, 8
    w, b, wd, act = setup(dev, orc, rows, cols, M, 800)
    whole = dev.get(dev.matmul_q6_k(wd, act, M))
    for c in range(M):
        one = tuple(a[c:c + 1] for a in act)
        alone = dev.get(dev.matmul_q6_k(wd, one, 1))
        np.testing.assert_array_equal(alone[0].view(np.uint32), whole[c].view(np.uint32))


def test_row_range_and_bias(dev, orc):
    rows, cols, M = 200, 512, 2
    w, b, wd, act = setup(dev, orc, rows, cols, M, 900)
    bias = synth.activations(synth.rng(901), 1, rows)[0]
    got = dev.get(dev.matmul_q6_k(wd, act, M, 7, 150, bias=bias))
    want = orc.matrix_rows(orc.Q6_K, w, rows, cols, b, 7, 150, bias=bias)
    assert np.all(np.isnan(got[:, :7])) and np.all(np.isnan(got[:, 150:]))
    np.testing.assert_array_equal(got[:, 7:150].view(np.uint32), want[:, 7:150].view(np.uint32))
