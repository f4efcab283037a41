"""MatVecRows for golem's fine-grained callers, coalesced behind the C ABI.

golem's engines call Matrix.MatVecRows (nn/matrix.go:84-92) on 32-row slices
from pool workers (qwen/block.go:82-90, qwen/attention.go:57-84).
gx_matvec_rows_q4_0 / _q6_k compute the whole product once per (matrix,
activation, generation, M) and serve every slice from it.  Checked here: each
slice, requested in shuffled order from eight threads at once, equals the
rows of the whole product bit for bit (gx_matmul_q4_0 / _q6_k, themselves
pinned against the oracle in test_gpu_q4_0 / test_gpu_q6_k); one product
runs per generation however many slices are asked; a new generation
recomputes; freeing the matrix forgets its products.
"""
import ctypes
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from golem_amd import capi, synth
from tests.gpu_util import log

pytestmark = pytest.mark.gpu


def stats(dev):
    products, served = ctypes.c_uint64(), ctypes.c_uint64()
    capi.call("gx_matvec_rows_stats", dev.ctx.ptr, ctypes.byref(products), ctypes.byref(served))
    return products.value, served.value


def serve_slices(dev, name, w, act, M, generation, ys, rows, step=32, workers=8, seed=0):
    """Every 32-row slice of the product, in shuffled order, from a pool of
    threads (ctypes releases the GIL during each call)."""
    slices = [(s, min(s + step, rows)) for s in range(0, rows, step)]
    synth.rng(seed).shuffle(slices)

    def one(se):
        s, e = se
        capi.call(name, dev.ctx.ptr, w.ptr, capi.vp(act[0]), capi.vp(act[1]), capi.vp(act[2]), M,
                  ctypes.c_uint64(generation), s, e, ctypes.c_void_p(ys.ctypes.data), ys.shape[1])

    with ThreadPoolExecutor(workers) as pool:
        list(pool.map(one, slices))
    return len(slices)


@pytest.mark.parametrize("rows,cols,M", [(1000, 2560, 1), (520, 1024, 3), (300, 704, 12)])
def test_q4_0_slices_share_one_product(dev, rows, cols, M):
    g = synth.rng(311 + rows + M)
    wd = dev.weight(synth.q4_0_weights(g, rows, cols), capi.Q4_0, rows, cols)
    act = dev.quantize_q8_0(synth.activations(g, M, cols), with_corr=False, with_q16=False)
    full = dev.get(dev.matmul_q4_0(wd, act, M, f16=False))
    p0, s0 = stats(dev)
    ys = np.full((M, rows + 5), np.nan, np.float32)  # ldys beyond the rows: nothing past them is written
    n = serve_slices(dev, "gx_matvec_rows_q4_0", wd, act, M, 7, ys, rows)
    p1, s1 = stats(dev)
    np.testing.assert_array_equal(ys[:, :rows].view(np.uint32), full.view(np.uint32))
    assert np.isnan(ys[:, rows:]).all()
    assert (p1 - p0, s1 - s0) == (1, n), f"{p1 - p0} products, {s1 - s0} slices for {n} calls"
    # the same generation again: served from the kept product
    ys2 = np.full((M, rows), np.nan, np.float32)
    serve_slices(dev, "gx_matvec_rows_q4_0", wd, act, M, 7, ys2, rows, seed=1)
    assert stats(dev)[0] == p1
    np.testing.assert_array_equal(ys2.view(np.uint32), full.view(np.uint32))
    # new contents under a new generation (same buffers, as a Batch refills
    # itself): recomputed once
    x2 = synth.activations(g, M, cols)
    b = dev.quantize_q8_0(x2, with_corr=False, with_q16=False)
    for dst, src in zip(act[:3], b[:3]):
        dst.copy_(src)
    full2 = dev.get(dev.matmul_q4_0(wd, act, M, f16=False))
    ys3 = np.full((M, rows), np.nan, np.float32)
    serve_slices(dev, "gx_matvec_rows_q4_0", wd, act, M, 8, ys3, rows, seed=2)
    assert stats(dev)[0] == p1 + 1
    np.testing.assert_array_equal(ys3.view(np.uint32), full2.view(np.uint32))
    log(f"  rows q4_0 {rows}x{cols} M={M}: {n} slices from one product a generation")


def test_q6_k_slices_share_one_product(dev):
    rows, cols, M = 700, 2560, 2
    g = synth.rng(977)
    wd = dev.weight(synth.q6_k_weights(g, rows, cols), capi.Q6_K, rows, cols)
    act = dev.quantize_q8_k(synth.activations(g, M, cols))
    full = dev.get(dev.matmul_q6_k(wd, act, M))
    p0, s0 = stats(dev)
    ys = np.full((M, rows), np.nan, np.float32)
    n = serve_slices(dev, "gx_matvec_rows_q6_k", wd, act, M, 1, ys, rows)
    p1, s1 = stats(dev)
    np.testing.assert_array_equal(ys.view(np.uint32), full.view(np.uint32))
    assert (p1 - p0, s1 - s0) == (1, n)


def test_freeing_a_matrix_forgets_its_products(dev):
    rows, cols, M = 128, 512, 1
    g = synth.rng(5)
    act = dev.quantize_q8_0(synth.activations(g, M, cols), with_corr=False, with_q16=False)
    for k in range(2):  # a second matrix may reuse the first one's address
        wd = dev.weight(synth.q4_0_weights(g, rows, cols), capi.Q4_0, rows, cols)
        full = dev.get(dev.matmul_q4_0(wd, act, M, f16=False))
        ys = np.full((M, rows), np.nan, np.float32)
        capi.call("gx_matvec_rows_q4_0", dev.ctx.ptr, wd.ptr, capi.vp(act[0]), capi.vp(act[1]), capi.vp(act[2]), M,
                  ctypes.c_uint64(3), 0, rows, ctypes.c_void_p(ys.ctypes.data), rows)
        np.testing.assert_array_equal(ys.view(np.uint32), full.view(np.uint32))
        wd.free()


def test_rows_refuse_bad_ranges(dev):
    rows, cols = 64, 256
    g = synth.rng(9)
    wd = dev.weight(synth.q4_0_weights(g, rows, cols), capi.Q4_0, rows, cols)
    act = dev.quantize_q8_0(synth.activations(g, 1, cols), with_corr=False, with_q16=False)
    ys = np.zeros((1, rows), np.float32)
    for s, e, ld in [(0, rows + 1, rows + 1), (10, 5, rows), (0, rows, rows - 1)]:
        with pytest.raises(capi.GxError):
            capi.call("gx_matvec_rows_q4_0", dev.ctx.ptr, wd.ptr, capi.vp(act[0]), capi.vp(act[1]),
                      capi.vp(act[2]), 1, ctypes.c_uint64(1), s, e, ctypes.c_void_p(ys.ctypes.data), ld)
