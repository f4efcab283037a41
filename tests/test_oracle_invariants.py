"""The oracle's products and quantisers pinned by what the mathematics fixes.

golem's quant fixtures (testdata/gemma/quants, nn/quants_reference_test.go)
are gitignored in the reference and absent, so nothing recorded from ggml
can pin these functions here.  Instead:
  - quantisers: closed-form invariants (range, error bound, zero blocks, the
    Q8_K extreme landing on -128, group sums) and hand-built examples;
  - Q4_0 integers: brute force in Python integers, and the identity
    acc = sum (n-8) q + 8 sum q;
  - Q4_0 floats: agreement with a float64 dequantise-then-dot built from
    numpy alone (golem's own bar for its ggml parity is 1e-5 of RMS);
  - Q6_K: the integer identity and golem's dequantisation bar
    (nn/dot_q6_k_test.go:13-48), with the dequantisation itself checked
    against an independent numpy unpacking of the bits;
  - the packed layout agrees with the row layout (nn/pack_q4_0_test.go:11);
  - Matrix.rows writes only [start, end) and adds the bias there
    (nn/pack_matvec_test.go:14).
Each independent check is also shown to fail on a planted mistake (a
swapped nibble order, a dropped recentring term, a transposed operand), so
that it is known to have teeth.
"""
import numpy as np
import pytest

from golem_amd import synth


# ---- independent numpy restatements used as checkers ------------------------

def np_dequant_q4_0(w, rows, cols, swap_nibbles=False):
    wb = w.reshape(rows, cols // 32, 18)
    d = wb[:, :, 0:2].copy().view(np.float16)[:, :, 0].astype(np.float64)
    nib = wb[:, :, 2:]
    lo = (nib & 0x0F).astype(np.float64) - 8
    hi = (nib >> 4).astype(np.float64) - 8
    if swap_nibbles:  # a plausible mistake: weights 2j, 2j+1 in one byte
        vals = np.stack([lo, hi], axis=3).reshape(rows, cols // 32, 32)
    else:
        vals = np.concatenate([lo, hi], axis=2)
    return (vals * d[:, :, None]).reshape(rows, cols)


def np_dequant_q6_k(w, rows, cols):
    wb = w.reshape(rows, cols // 256, 210)
    out = np.zeros((rows, cols // 256, 256), dtype=np.float64)
    d = wb[:, :, 208:210].copy().view(np.float16)[:, :, 0].astype(np.float64)
    sc = wb[:, :, 192:208].view(np.int8).astype(np.float64)
    for half in range(2):
        l = wb[:, :, half * 64:half * 64 + 64].astype(np.int64)
        h = wb[:, :, 128 + half * 32:128 + half * 32 + 32].astype(np.int64)
        for sub in range(4):
            src = l[:, :, 0:32] if sub in (0, 2) else l[:, :, 32:64]
            nib = (src & 0x0F) if sub < 2 else (src >> 4)
            q = nib | (((h >> (2 * sub)) & 3) << 4)
            pos = half * 128 + sub * 32 + np.arange(32)
            grp = pos // 16
            out[:, :, pos] = (q - 32) * sc[:, :, grp] * d[:, :, None]
    return out.reshape(rows, cols)


# ---- quantisers ----------------------------------------------------------

@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q8_0_invariants(orc, seed):
    g = synth.rng(seed)
    x = synth.activations(g, 5, 512)
    x[1, :32] = 0
    x[2] *= 1e-3
    b = orc.Batch(x).quantize()
    q = b.q_rows().reshape(5, -1, 32).astype(np.int64)
    S = b.scales_rows()
    assert q.min() >= -127 and q.max() <= 127
    # the scale is max|x|/127 rounded through fp16
    peak = np.abs(x.reshape(5, -1, 32)).max(axis=2)
    want_scale = (peak / np.float32(127)).astype(np.float32).astype(np.float16).astype(np.float32)
    assert np.array_equal(S, want_scale)
    # each q is x/scale rounded: |q*scale - x| <= scale/2 + the fp16 slack
    inv = np.where(peak > 0, np.float32(127) / np.where(peak > 0, peak, 1), 0).astype(np.float32)
    want_q = np.rint((x.reshape(5, -1, 32) * inv[:, :, None]).astype(np.float32))
    assert np.array_equal(q, np.clip(want_q, -128, 127).astype(np.int64))
    # a zero block stays zero, with zero scale and correction
    assert np.all(q[1, 0] == 0) and S[1, 0] == 0 and b.corr_rows()[1, 0] == 0
    # Corr = (8*scale)*float(sum q)
    corr = (np.float32(8) * S).astype(np.float32) * q.sum(axis=2).astype(np.float32)
    assert np.array_equal(b.corr_rows(), corr.astype(np.float32))


def test_q8_0_hand_example(orc):
    x = np.zeros((1, 32), dtype=np.float32)
    x[0, 0], x[0, 1], x[0, 2], x[0, 3] = 127, -63.5, 0.5, 1.5
    b = orc.Batch(x).quantize()
    # peak 127: scale 1, inverse 1; halves round to even
    assert list(b.q_rows()[0, :4]) == [127, -64, 0, 2]
    assert b.Scales[0] == 1.0 and b.Corr[0] == 8 * (127 - 64 + 0 + 2)


def test_q8_k_invariants(orc):
    g = synth.rng(4)
    x = synth.activations(g, 3, 512)
    x[1, :256] = 0
    x[2, 10], x[2, 20] = -9.0, 9.0  # equal magnitudes: the first (negative) is the extreme
    b = orc.Batch(x).quantize_k()
    q = b.QK.reshape(3, 2, 256).astype(np.int64)
    assert q.max() <= 127 and q.min() >= -128
    assert np.all(q[1, 0] == 0) and b.KScales[2] == 0 and np.all(b.BSums.reshape(3, -1)[1, :16] == 0)
    assert q[2, 0, 10] == -128 and q[2, 0, 20] == 127  # -128/extreme * 9 = 128 -> clamped
    # the scale is 1/inverse = -extreme/128
    assert np.isclose(b.KScales.reshape(3, 2)[2, 0], 9.0 / 128, rtol=0, atol=1e-7)
    bs = q.reshape(3, -1, 16).sum(axis=2)
    assert np.array_equal(b.BSums.reshape(3, -1).astype(np.int64), bs)
    # every extreme lands on -128 exactly
    for c in (0, 2):
        for s in range(2):
            blk = x[c, s * 256:(s + 1) * 256]
            at = int(np.argmax(np.abs(blk)))
            assert q[c, s, at] == -128


# ---- Q4_0 ----------------------------------------------------------------

def test_q4_0_integers_brute_force(orc):
    g = synth.rng(8)
    rows, cols = 5, 128
    w = synth.q4_0_weights(g, rows, cols)
    b = orc.Batch(synth.activations(g, 3, cols)).quantize()
    acc = orc.q4_0_block_acc(w, b, rows)
    q = b.q_rows()
    wb = w.reshape(rows, cols // 32, 18)
    for c in range(3):
        for r in range(rows):
            for blk in range(cols // 32):
                total = 0
                for j in range(16):
                    byte = int(wb[r, blk, 2 + j])
                    total += (byte & 15) * int(q[c, blk * 32 + j]) + (byte >> 4) * int(q[c, blk * 32 + 16 + j])
                assert total == acc[c, r, blk]
                signed = sum((int(v) - 8) * int(a) for v, a in zip(
                    [int(wb[r, blk, 2 + j]) & 15 for j in range(16)] + [int(wb[r, blk, 2 + j]) >> 4 for j in range(16)],
                    q[c, blk * 32:(blk + 1) * 32]))
                assert total == signed + 8 * int(q[c, blk * 32:(blk + 1) * 32].astype(np.int64).sum())


def _q4_float64(w, b, rows, cols, **kw):
    deq = np_dequant_q4_0(w, rows, cols, **kw)
    qa = (b.q_rows().astype(np.float64).reshape(b.size, -1, 32) * b.scales_rows()[:, :, None]).reshape(b.size, cols)
    return (qa @ deq.T).astype(np.float32)


@pytest.mark.parametrize("rows,cols,size", [(40, 2560, 3), (17, 4096, 2), (9, 704, 1)])
def test_q4_0_row_layout_against_float64(orc, rows, cols, size):
    g = synth.rng(rows)
    w = synth.q4_0_weights(g, rows, cols)
    b = orc.Batch(synth.activations(g, size, cols)).quantize()
    got = orc.mat_vec_q4_0_rows(w, b, rows)
    want = _q4_float64(w, b, rows, cols)
    for c in range(size):
        rel, _ = orc.compare_floats(got[c], want[c])
        assert rel <= 1e-5
    # the check has teeth: a swapped nibble order is far outside the bar
    wrong = _q4_float64(w, b, rows, cols, swap_nibbles=True)
    assert orc.compare_floats(got[0], wrong[0])[0] > 1e-2


def test_dequantize_q4_0_matches_numpy(orc):
    g = synth.rng(9)
    w = synth.q4_0_weights(g, 3, 256)
    want = np_dequant_q4_0(w, 3, 256).astype(np.float32)
    for r in range(3):
        got = orc.dequantize_q4_0_row(w[r * 8 * 18:(r + 1) * 8 * 18], 256)
        assert np.array_equal(got, want[r])


@pytest.mark.parametrize("cols", [32, 64, 256, 1536, 2080])
def test_packed_matches_row_layout(orc, cols):
    """TestPackQ4_0MatchesTheRowLayout (nn/pack_q4_0_test.go:11-50) and
    TestPackedMatrixAgreesWithTheRowLayout (nn/pack_matvec_test.go:14-74):
    rel 1e-3 + 1e-4, rows outside [start, end) untouched."""
    g = synth.rng(cols)
    for rows in (8, 24, 30, 65):
        w = synth.q4_0_weights(g, rows, cols)
        b = orc.Batch(synth.activations(g, 6, cols)).quantize()
        plain = orc.matrix_rows(orc.Q4_0, w, rows, cols, b)
        packed = orc.pack_q4_0(w, rows, cols)
        for start, end in ((0, rows), (1, rows - 1), (3, 11), (rows - 3, rows)):
            if not (0 <= start < end <= rows):
                continue
            got = orc.matrix_rows(orc.Q4_0, w, rows, cols, b, start, end, packed=packed)
            assert np.all(np.isnan(got[:, :start])) and np.all(np.isnan(got[:, end:]))
            gap = np.abs(got[:, start:end] - plain[:, start:end])
            assert np.all(gap <= 1e-3 * np.abs(plain[:, start:end]) + 1e-4)


def test_pack_layout_is_a_permutation(orc):
    """PackQ4_0 moves every nibble of eight rows and nothing else: unpacking
    the group per the layout (nn/pack_q4_0.go:27-35, lowRows/highRows) gives
    back the row-layout weights."""
    g = synth.rng(12)
    rows, cols = 16, 96
    w = synth.q4_0_weights(g, rows, cols)
    p = orc.pack_q4_0(w, rows, cols).reshape(rows // 8, cols // 32, 144)
    wb = w.reshape(rows, cols // 32, 18)
    low, high = [0, 1, 4, 5], [2, 3, 6, 7]
    for grp in range(rows // 8):
        for blk in range(cols // 32):
            chunk = p[grp, blk]
            for r in range(8):
                assert bytes(chunk[2 * r:2 * r + 2]) == bytes(wb[grp * 8 + r, blk, 0:2])
            vals = np.zeros((8, 32), dtype=np.int64)
            for gg in range(4):
                for s in range(4):
                    for j in range(8):
                        byte = int(chunk[16 + gg * 32 + s * 8 + j])
                        vals[low[s], gg * 8 + j] = byte & 15
                        vals[high[s], gg * 8 + j] = byte >> 4
            for r in range(8):
                nib = wb[grp * 8 + r, blk, 2:].astype(np.int64)
                assert np.array_equal(vals[r], np.concatenate([nib & 15, nib >> 4]))


def test_bias_only_on_range(orc):
    g = synth.rng(13)
    rows, cols = 20, 64
    w = synth.q4_0_weights(g, rows, cols)
    b = orc.Batch(synth.activations(g, 2, cols)).quantize()
    bias = np.arange(rows, dtype=np.float32)
    base = orc.matrix_rows(orc.Q4_0, w, rows, cols, b)
    got = orc.matrix_rows(orc.Q4_0, w, rows, cols, b, 4, 9, bias=bias)
    assert np.all(np.isnan(got[:, :4])) and np.all(np.isnan(got[:, 9:]))
    assert np.array_equal(got[:, 4:9], (base[:, 4:9] + bias[4:9]).astype(np.float32))


# ---- Q6_K ----------------------------------------------------------------

def test_dequantize_q6_k_matches_numpy(orc):
    g = synth.rng(14)
    rows, cols = 4, 512
    w = synth.q6_k_weights(g, rows, cols)
    want = np_dequant_q6_k(w, rows, cols)
    for r in range(rows):
        got = orc.dequantize_q6_k(w[r * 420:(r + 1) * 420], cols)
        # golem rounds (d*sc) then *(q-32): two float32 roundings of an exact product
        assert np.allclose(got, want[r], rtol=2 ** -22, atol=0)


def test_q6_k_integer_identity(orc):
    """isum = sum_g sc_g sum (q6 - 32) a over the group, exactly."""
    g = synth.rng(15)
    rows, cols = 3, 512
    w = synth.q6_k_weights(g, rows, cols)
    b = orc.Batch(synth.activations(g, 2, cols)).quantize_k()
    isum = orc.q6_k_block_isum(w, b, rows)
    wb = w.reshape(rows, 2, 210)
    for c in range(2):
        a = b.QK[c * cols:(c + 1) * cols].astype(np.int64).reshape(2, 256)
        for r in range(rows):
            for s in range(2):
                deq_int = np.zeros(256, dtype=np.int64)
                blk = wb[r, s]
                for half in range(2):
                    l = blk[half * 64:half * 64 + 64].astype(np.int64)
                    h = blk[128 + half * 32:160 + half * 32].astype(np.int64)
                    for sub in range(4):
                        src = l[0:32] if sub in (0, 2) else l[32:64]
                        nib = (src & 15) if sub < 2 else (src >> 4)
                        qv = nib | (((h >> (2 * sub)) & 3) << 4)
                        pos = half * 128 + sub * 32 + np.arange(32)
                        deq_int[pos] = (qv - 32) * blk[192:208].view(np.int8).astype(np.int64)[pos // 16]
                assert int((deq_int * a[s]).sum()) == isum[c, r, s]


def test_q6_k_against_dequantisation(orc):
    """TestMatVecQ6_KAgreesWithDequantization's bar (nn/dot_q6_k_test.go:13-48):
    within 5e-3 of the row's sum of |terms|, with x = sin(0.37 i)."""
    g = synth.rng(16)
    rows, cols = 6, 1536
    w = synth.q6_k_weights(g, rows, cols)
    x = np.sin(np.arange(cols) * 0.37).astype(np.float32)[None, :]
    b = orc.Batch(x).quantize_k()
    got = orc.mat_vec_q6_k_rows(w, b, rows)[0]
    deq = np.stack([orc.dequantize_q6_k(w[r * 6 * 210:(r + 1) * 6 * 210], cols) for r in range(rows)])
    terms = deq.astype(np.float64) * x[0].astype(np.float64)
    want = terms.sum(axis=1)
    energy = np.abs(terms).sum(axis=1)
    assert np.all(np.abs(got - want) <= 5e-3 * energy)
    # teeth: the transposed operand (sub-scale groups misassigned) fails the bar
    wrong = np_dequant_q6_k(w, rows, cols).reshape(rows, -1, 16)[:, ::-1].reshape(rows, cols)
    assert np.any(np.abs(got - (wrong * x[0]).sum(axis=1)) > 5e-3 * energy)


def test_q6_k_columns_independent(orc):
    """Two columns give each its one-column result (dot_q6_k_x2_test.go:12)."""
    g = synth.rng(17)
    rows, cols = 10, 512
    w = synth.q6_k_weights(g, rows, cols)
    x = synth.activations(g, 2, cols)
    both = orc.mat_vec_q6_k_rows(w, orc.Batch(x).quantize_k(), rows)
    for c in range(2):
        one = orc.mat_vec_q6_k_rows(w, orc.Batch(x[c:c + 1]).quantize_k(), rows)
        assert np.array_equal(one[0].view(np.uint32), both[c].view(np.uint32))
