"""The device activation quantisers against the oracle, bit for bit.

Q8_0: Batch.quantizeBlock (nn/batch.go:109-143).  Q8_K: Batch.QuantizeK
(nn/batch.go:159-213).  Inputs include the cases the quantisers branch on:
an all-zero block, a block whose scale is an fp16 subnormal, exact ties of
nearestInt, equal magnitudes of opposite sign (the Q8_K extreme is the
first), and values large enough to clamp.
"""
import numpy as np
import pytest

from golem_amd import synth
from tests.gpu_util import log, q16_rows

pytestmark = pytest.mark.gpu


def edge_rows(K, seed):
    g = synth.rng(seed)
    x = synth.activations(g, 6, K)
    x[1, :64] = 0.0                                     # zero blocks / zero start of a superblock
    x[1, 256:512] = 0.0                                 # a zero superblock
    x[2, :32] = np.float32(3e-6) * g.standard_normal(32).astype(np.float32)  # subnormal fp16 scale
    x[3, :32] = np.arange(-16, 16, dtype=np.float32) + 0.5       # halves after scaling
    x[3, 32:64] = 127.0 * np.sign(g.standard_normal(32)).astype(np.float32)
    x[4, :256] = g.standard_normal(256).astype(np.float32)
    x[4, 10], x[4, 200] = -7.0, 7.0                      # equal magnitude, opposite sign: the first wins
    x[5] *= np.float32(1e4)
    return x


@pytest.mark.parametrize("M,K", [(1, 2560), (3, 704), (6, 2816), (64, 2560)])
def test_q8_0_bit_exact(dev, orc, M, K):
    log(f"q8_0 M={M} K={K}")
    x = synth.activations(synth.rng(10 + M), M, K)
    if M >= 6:
        x[:6] = edge_rows(K, 11)[:6, :K]
    b = orc.Batch(x).quantize()
    q, sc, qs, q16, co = dev.quantize_q8_0(x)
    np.testing.assert_array_equal(dev.get(q), b.q_rows())
    rows16 = q16_rows(dev.get(q16), M, K)
    np.testing.assert_array_equal(rows16[:M], b.q_rows().astype(np.float32))
    assert not np.any(rows16[M:]), "the fp16 copy's padding tokens are not zero"
    np.testing.assert_array_equal(dev.get(sc).view(np.uint32), b.scales_rows().view(np.uint32))
    np.testing.assert_array_equal(dev.get(qs), b.qsum_rows())
    np.testing.assert_array_equal(dev.get(co).view(np.uint32), b.corr_rows().view(np.uint32))


@pytest.mark.parametrize("M,K", [(1, 2560), (6, 2560), (5, 9728)])
def test_q8_k_bit_exact(dev, orc, M, K):
    log(f"q8_k M={M} K={K}")
    x = synth.activations(synth.rng(20 + M), M, K)
    if M >= 6:
        x[:6] = edge_rows(K, 21)[:6, :K]
    b = orc.Batch(x).quantize_k()
    q, ks, bs = dev.quantize_q8_k(x)
    np.testing.assert_array_equal(dev.get(q).reshape(-1), b.QK)
    np.testing.assert_array_equal(dev.get(ks).reshape(-1).view(np.uint32), b.KScales.view(np.uint32))
    np.testing.assert_array_equal(dev.get(bs).reshape(-1), b.BSums)
