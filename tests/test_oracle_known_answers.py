"""The oracle pinned by the known answers golem's own tests hold, and by
library routines and closed forms that fix the same functions independently.

Each test names the golem test or the mathematics it follows.  A check that
only retyped the oracle's formula would pin nothing, so every one compares
against something computed another way.
"""
import math

import numpy as np
import pytest


# ---- fp16 (nn/half_test.go) ------------------------------------------------

def test_half_round_trip_exhaustive(orc):
    """TestHalfRoundTrip (nn/half_test.go:9-21): every binary16 except NaN
    payloads survives halfToFloat then floatToHalf."""
    lib = orc.load()
    for h in range(1 << 16):
        e, m = (h >> 10) & 0x1F, h & 0x3FF
        if e == 0x1F and m != 0:
            continue
        assert lib.orc_float_to_half(lib.orc_half_to_float(h)) == h, hex(h)


def test_half_to_float_matches_numpy_exhaustive(orc):
    """halfToFloat against numpy's own binary16 widening, all 65536 patterns
    (NaNs compared as NaN)."""
    lib = orc.load()
    bits = np.arange(1 << 16, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_half_to_float(int(h)) for h in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("f,want", [
    (0.0, 0x0000), (1.0, 0x3C00), (-2.0, 0xC000), (65504.0, 0x7BFF), (131008.0, 0x7C00),
    (6.0e-8, 0x0001), (1.0e-9, 0x0000), (1.00048828125, 0x3C00), (1.00146484375, 0x3C02),
])
def test_float_to_half_known_answers(orc, f, want):
    """TestFloatToHalfRounds (nn/half_test.go:24-44)."""
    assert orc.float_to_half(np.float32(f)) == want


def test_float_to_half_matches_numpy_rne(orc):
    """floatToHalf against numpy's round-to-nearest-even float32 -> float16 on
    two million random finite float32 patterns plus every exact halfway
    case of the normal range."""
    lib = orc.load()
    g = np.random.Generator(np.random.PCG64(123))
    bits = g.integers(0, 1 << 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    # halfway points: a half's value plus half an ulp, for a spread of exponents
    h = np.arange(0x0400, 0x7BFF, 7, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float32)
    hi = (h + 1).view(np.float16).astype(np.float32)
    mid = ((lo.astype(np.float64) + hi.astype(np.float64)) / 2).astype(np.float32)
    f = np.concatenate([f[:200_000], mid, -mid])
    want = f.astype(np.float16).view(np.uint16)
    got = np.fromiter((lib.orc_float_to_half(float(v)) for v in f), dtype=np.uint16, count=len(f))
    # numpy keeps NaN payload bits; golem writes 0x7E00 -- inputs here are finite
    assert np.array_equal(got, want)


def test_nearest_int_is_rint(orc):
    """nearestInt (nn/batch.go:221-224) is round-half-even for |x| < 2^22: it
    equals numpy's rint, including every .5 case."""
    lib = orc.load()
    g = np.random.Generator(np.random.PCG64(7))
    xs = np.concatenate([g.uniform(-300, 300, 20000), np.arange(-260, 260) + 0.5,
                         g.uniform(-4e6, 4e6, 2000)]).astype(np.float32)
    got = np.array([lib.orc_nearest_int(float(x)) for x in xs])
    assert np.array_equal(got, np.rint(xs).astype(np.int64))


# ---- GELU table (nn/gelu_table_test.go) ------------------------------------

def test_gelu_table_matches_ggml(orc):
    """TestGELUTableMatchesGGML (nn/gelu_table_test.go:11-23): exact values."""
    got = orc.gelu_table([1, -1, 0.5, 3, -0.125, 0.0625])
    want = np.array([0.8413086, -0.15881348, 0.34570312, 2.9960938, -0.056274414, 0.032806396],
                    dtype=np.float32)
    assert np.array_equal(got, want)


def test_gelu_table_cutoffs(orc):
    """TestGELUTableCutoffs (nn/gelu_table_test.go:25-34)."""
    assert np.array_equal(orc.gelu_table([-10, -12.5, 10, 42]), np.array([0, 0, 10, 42], dtype=np.float32))


def test_gelu_table_tracks_formula(orc):
    """TestGELUTableTracksTheFormula (nn/gelu_table_test.go:38-52)."""
    xs = np.arange(-9.0, 9.0, 0.045).astype(np.float32)
    got = orc.gelu_table(xs)
    for x, v in zip(xs, got):
        exact = 0.5 * x * (1 + math.tanh(0.79788456080286535587989211986876 * x * (1 + 0.044715 * x * x)))
        assert abs(v - exact) <= 5e-3


# ---- expf (nn/swiglu_test.go) ------------------------------------------------

def _ulp_gap(a, b):
    ia = np.float32(a).view(np.int32).astype(np.int64)
    ib = np.float32(b).view(np.int32).astype(np.int64)
    return abs(ia - ib)


def test_expf_within_two_ulp(orc):
    """TestExpfMatchesTheExactExponential (nn/swiglu_test.go:18-38): within 2
    ulp of the correctly rounded exponential over [-87, 88]."""
    for x in np.linspace(-87, 88, 20001).astype(np.float32):
        exact = np.float32(math.exp(float(x)))
        assert _ulp_gap(orc.expf(x), exact) <= 2, x


def test_expf_at_extremes(orc):
    """TestExpfAtTheExtremes (nn/swiglu_test.go:40-66): 0 -> 1 exactly; far
    outside the range the exact routine answers (0 and inf)."""
    assert orc.expf(0.0) == 1.0
    assert orc.expf(-200.0) == 0.0
    assert math.isinf(orc.expf(200.0))


# ---- RMSNormPlain (nn/gemma_ops_test.go) -------------------------------------

def test_rms_norm_plain_closed_forms(orc):
    """TestRMSNormPlain / WithoutGain / DoesNotCentre (nn/gemma_ops_test.go:8-52)."""
    x = orc.rms_norm_plain([1, -2, 3, -4], [2, 2, 2, 2], 1e-6)
    inv = 1 / math.sqrt(7.5 + 1e-6)
    for v, w in zip(x, [1 * inv * 2, -2 * inv * 2, 3 * inv * 2, -4 * inv * 2]):
        assert abs(v - w) <= 1e-6
    x = orc.rms_norm_plain([3, 4], None, 0.0)
    inv = 1 / math.sqrt(12.5)
    assert abs(x[0] - 3 * inv) <= 1e-6 and abs(x[1] - 4 * inv) <= 1e-6
    x = orc.rms_norm_plain([5, 5, 5, 5], None, 0.0)
    assert np.all(np.abs(x - 1) <= 1e-6)


# ---- chooseExperts (gemma/moe_test.go) ---------------------------------------

def test_choose_experts_renormalizes(orc):
    """TestChooseExpertsRenormalizes (gemma/moe_test.go:207-232)."""
    ids, weights = orc.choose_experts([1, 4, 0, 3, 2], 3)
    assert list(ids) == [1, 3, 4]
    assert abs(float(weights.sum()) - 1) <= 1e-6
    want = math.exp(4) / (math.exp(4) + math.exp(3) + math.exp(2))
    assert abs(weights[0] - want) <= 1e-6


def test_choose_experts_ties_to_lower_index(orc):
    """TestChooseExpertsIsStableInTies (gemma/moe_test.go:234-244)."""
    for _ in range(8):
        ids, _w = orc.choose_experts([2, 2, 2, 1], 2)
        assert list(ids) == [0, 1]


# ---- DotF32 ------------------------------------------------------------------

def test_dot_f32_generic_order(orc):
    """DotF32's generic order (nn/dot_f32.go:20-32), checked against a float64
    sum within the float32 error bound, and against an explicit simulation of
    four float32 accumulators (numpy float32 arithmetic, one rounding per
    operation) bit for bit."""
    g = np.random.Generator(np.random.PCG64(3))
    for n in (1, 3, 4, 7, 2816, 2819):
        a = g.standard_normal(n).astype(np.float32)
        b = g.standard_normal(n).astype(np.float32)
        got = orc.dot_f32(a, b)
        s = [np.float32(0)] * 4
        whole = n - n % 4
        for i in range(whole):
            s[i % 4] = np.float32(s[i % 4] + np.float32(a[i] * b[i]))
        for i in range(whole, n):
            s[0] = np.float32(s[0] + np.float32(a[i] * b[i]))
        want = np.float32(np.float32(s[0] + s[1]) + np.float32(s[2] + s[3]))
        assert np.float32(got).view(np.uint32) == want.view(np.uint32)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        bound = n * 2 ** -23 * float(np.sum(np.abs(a.astype(np.float64) * b)))
        assert abs(got - exact) <= bound + 1e-30


def test_dot_f32_avx2_order_bounds(orc):
    """dotF32AVX2's order (the router's DotF32) against float64: within the
    standard bound n * eps * sum|a b| of a float32 sum; exact on small
    integers; and it is not the generic order's chain (a mistake that summed
    in the generic order would pass the bound but not the instructions' bits,
    test_cpu_baseline.py)."""
    g = np.random.default_rng(5)
    for n in (5, 64, 2816, 3000):
        a = (g.standard_normal(n) * 3).astype(np.float32)
        b = (g.standard_normal(n) * 0.02).astype(np.float32)
        exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        bound = n * 2.0 ** -24 * float(np.sum(np.abs(a.astype(np.float64) * b)))
        assert abs(orc.dot_f32_avx2(a, b) - exact) <= bound
    a = np.arange(1, 97, dtype=np.float32)
    b = np.ones(96, dtype=np.float32)
    assert orc.dot_f32_avx2(a, b) == float(96 * 97 // 2)


# ---- the softmax exponential --------------------------------------------------

def test_exp_neg_is_the_float64_exp_rounded_to_float():
    """orc_exp_neg (the device's exp_neg: straight-line float64 steps) against
    the C library's exp in float64 rounded to float, which is what
    SoftmaxInPlace takes (nn/ops.go:59-73): bit for bit on every float of
    [-110, 0] in a stride of 97 through the bit patterns (11.6 million
    values; every one of the 1.12 billion was checked once on the host),
    on dense runs around the points where the range reduction's n steps
    (k ln2 / 2), and at the edges: 0, -0, the least values above -110, -inf
    (+0) and NaN."""
    import oracle
    lib = oracle.load()
    lo, hi = np.uint32(0x80000000), np.float32(-110.0).view(np.uint32)
    pats = np.arange(int(lo), int(hi) + 1, 97, dtype=np.uint64).astype(np.uint32)
    xs = [pats.view(np.float32)]
    for k in range(1, 318):  # n changes near -(k - 1/2) ln2
        c = np.float32(-(k - 0.5) * np.log(2.0))
        xs.append((c.view(np.uint32) + np.arange(-2000, 2000, dtype=np.int64)).astype(np.uint32).view(np.float32))
    xs.append(np.array([0.0, -0.0, -110.0, np.nextafter(np.float32(-110), np.float32(0))], np.float32))
    x = np.ascontiguousarray(np.concatenate(xs).astype(np.float32))
    x = x[(x <= 0) & (x >= -110)]
    bad = lib.orc_exp_neg_check(oracle._p(x), len(x), None)
    assert bad == 0, f"{bad} of {len(x)} differ from the C library's"
    assert lib.orc_exp_neg(np.float32(-np.inf)) == 0.0
    assert np.isnan(lib.orc_exp_neg(np.float32(np.nan)))
    assert lib.orc_exp_neg(np.float32(-200.0)) == 0.0
    assert lib.orc_exp_neg(np.float32(0.0)) == 1.0
