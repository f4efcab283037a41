"""The committed vectors of tests/golden/hot_path_slices.npz (slices of
configs 0, 1 and 4 with the oracle's outputs, written by
tests/golden/make_golden.py): the oracle must still produce them bit for
bit (CPU), and the device path must match them -- the Q8_0 / Q8_K forms,
Q6_K integers, outputs, router logits and chosen experts bit for bit, the
Q4_0 per-block integers through golem's identity acc = sum (n - 8) q +
8 sum q, the Q4_0 outputs within golem's 1e-5 of RMS (compareFloats), the
expert weights within 1e-6 relative."""
import os

import numpy as np
import pytest

import oracle
from golem_amd import capi

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "hot_path_slices.npz")
ROWS = 64


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN) as z:
        return {k: z[k] for k in z.files}


def same_bits(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and a.dtype == b.dtype and a.tobytes() == b.tobytes()


def test_oracle_reproduces_golden(gold):
    b0 = oracle.Batch(gold["c0_x"]).quantize()
    assert same_bits(b0.q_rows(), gold["c0_q"]) and same_bits(b0.scales_rows(), gold["c0_scales"])
    assert same_bits(b0.corr_rows(), gold["c0_corr"])
    assert same_bits(oracle.q4_0_block_acc(gold["c0_w"], b0, ROWS), gold["c0_acc"])
    assert same_bits(oracle.mat_vec_q4_0_rows(gold["c0_w"], b0, ROWS), gold["c0_y"])
    b1 = oracle.Batch(gold["c1_x"]).quantize_k()
    assert same_bits(b1.QK, gold["c1_qk"]) and same_bits(b1.KScales, gold["c1_kscales"])
    assert same_bits(b1.BSums, gold["c1_bsums"])
    assert same_bits(oracle.q6_k_block_isum(gold["c1_w"], b1, ROWS), gold["c1_isum"])
    assert same_bits(oracle.mat_vec_q6_k_rows(gold["c1_w"], b1, ROWS), gold["c1_y"])
    logits, ids, weights = oracle.route_one(gold["c4_x"], gold["c4_router"], 8)
    assert same_bits(logits, gold["c4_logits"]) and same_bits(ids, gold["c4_ids"])
    assert same_bits(weights, gold["c4_weights"])


@pytest.mark.gpu
def test_device_matches_golden(dev, gold):
    # Q8_0 and the Q4_0 product, config 0's first 64 rows
    act = dev.quantize_q8_0(gold["c0_x"], with_corr=True, with_q16=False)
    q, sc, qs, _, co = (None if a is None else dev.get(a) for a in act)
    assert same_bits(q, gold["c0_q"]) and same_bits(sc, gold["c0_scales"]) and same_bits(co, gold["c0_corr"])
    w0 = dev.weight(gold["c0_w"], capi.Q4_0, ROWS, 2560)
    qsum = gold["c0_q"].reshape(1, 1, 80, 32).astype(np.int64).sum(axis=3)
    # sum (n - 8) q as the shipped kernels compute it: path 3 is the
    # one-column kernel this M = 1 product runs, path 0 the SGPR kernel of
    # small batches, path 1 the int8-MFMA product
    for path in (3, 0, 1):
        isum = dev.q4_0_block_dots(w0, act, 1, 0, ROWS, path)
        np.testing.assert_array_equal(isum.astype(np.int64) + 8 * qsum, gold["c0_acc"].astype(np.int64),
                                      err_msg=f"path {path}")
    y0 = dev.get(dev.matmul_q4_0(w0, act, 1))
    rel, at = oracle.compare_floats(y0[0], gold["c0_y"][0])
    assert rel <= 1e-5, f"Q4_0 rows: {rel:.3g} of RMS at {at}"
    w0.free()
    # Q8_K and the Q6_K head, config 1's first 64 rows: bit for bit
    act1 = dev.quantize_q8_k(gold["c1_x"])
    qk, ks, bs = (dev.get(a) for a in act1)
    assert same_bits(qk.reshape(-1), gold["c1_qk"]) and same_bits(ks.reshape(-1), gold["c1_kscales"])
    assert same_bits(bs.reshape(-1), gold["c1_bsums"])
    w1 = dev.weight(gold["c1_w"], capi.Q6_K, ROWS, 2560)
    assert same_bits(dev.q6_k_block_dots(w1, act1, 1, 0, ROWS), gold["c1_isum"])
    assert same_bits(dev.get(dev.matmul_q6_k(w1, act1, 1)), gold["c1_y"])
    w1.free()
    # the router: logits and chosen experts bit for bit
    E, D, k = 128, 256, 8
    wr = dev.weight(gold["c4_router"], capi.F32, E, D)
    xd = dev.put(gold["c4_x"].reshape(1, D))
    logits, ids, wts = dev.empty((1, E), np.float32), dev.empty((1, k), np.int32), dev.empty((1, k), np.float32)
    capi.call("gx_moe_route", dev.ctx.ptr, wr.ptr, None, capi.vp(xd), D, 1, k, np.float32(1e-6), capi.vp(logits),
              capi.vp(ids), capi.vp(wts))
    assert same_bits(dev.get(logits)[0], gold["c4_logits"]) and same_bits(dev.get(ids)[0], gold["c4_ids"])
    np.testing.assert_allclose(dev.get(wts)[0], gold["c4_weights"], rtol=1e-6, atol=0)
    wr.free()
