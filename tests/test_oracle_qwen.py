"""The oracle's Qwen3 pieces against what the mathematics fixes, and golem's
batch property in the oracle itself.

- RoPETable.Prepare (nn/rope.go:33-59): position 0 gives cos 1, sin 0 (the
  rotation is the identity); theta_i = pos * base^(-2i/dims) against a direct
  float64 evaluation; Apply pairs element i with i + dims/2 (NeoX), checked
  against a complex multiplication in float64 to float32 rounding.
- the attention of one position is its value exactly (a softmax over one score
  is 1, and 1 * v + 0 is v); two equal keys split the probability evenly.
- a prompt read in one batch is bit-identical to it read a token at a time
  (qwen/model_test.go:79), through the oracle's model.
"""
import math

import numpy as np

import oracle
from golem_amd import synth


def test_rope_position_zero_is_identity():
    lib = oracle.load()
    c = np.zeros(64, np.float32)
    s = np.zeros(64, np.float32)
    lib.orc_rope_prepare(128, 0, 1e6, oracle._p(c), oracle._p(s))
    assert np.all(c == 1.0) and np.all(s == 0.0)
    v = synth.rng(1).standard_normal(128).astype(np.float32)
    w = v.copy()
    lib.orc_rope_apply(oracle._p(w), 128, oracle._p(c), oracle._p(s))
    np.testing.assert_array_equal(w, v)


def test_rope_angles_and_pairs():
    lib = oracle.load()
    dims, pos, base = 128, 513, 1e6
    c = np.zeros(dims // 2, np.float32)
    s = np.zeros(dims // 2, np.float32)
    lib.orc_rope_prepare(dims, pos, base, oracle._p(c), oracle._p(s))
    for i in (0, 1, 17, 63):
        theta = pos * base ** (-2 * i / dims)
        assert c[i] == np.float32(math.cos(theta)) and s[i] == np.float32(math.sin(theta))
    v = synth.rng(2).standard_normal(dims).astype(np.float32)
    w = v.copy()
    lib.orc_rope_apply(oracle._p(w), dims, oracle._p(c), oracle._p(s))
    z = (v[:dims // 2].astype(np.float64) + 1j * v[dims // 2:]) * (c.astype(np.float64) + 1j * s)
    np.testing.assert_allclose(w[:dims // 2], z.real, rtol=0, atol=1e-6)
    np.testing.assert_allclose(w[dims // 2:], z.imag, rtol=0, atol=1e-6)


def test_attention_of_one_position_is_its_value():
    lib = oracle.load()
    hd, kv = 64, 2
    g = synth.rng(3)
    K = g.standard_normal((4, kv, hd)).astype(np.float16).astype(np.float32)
    V = g.standard_normal((4, kv, hd)).astype(np.float16).astype(np.float32)
    q = g.standard_normal(hd).astype(np.float32)
    scores = np.zeros(4, np.float32)
    dst = np.zeros(hd, np.float32)
    lib.orc_attend(oracle._p(q), oracle._p(K), oracle._p(V), kv, hd, 1, 1, np.float32(0.125), oracle._p(scores),
                   oracle._p(dst))
    np.testing.assert_array_equal(dst, V[0, 1])
    # two identical keys: probabilities 1/2 each (exact in fp16), values averaged
    K[1] = K[0]
    lib.orc_attend(oracle._p(q), oracle._p(K), oracle._p(V), kv, hd, 0, 2, np.float32(0.125), oracle._p(scores),
                   oracle._p(dst))
    assert scores[0] == scores[1] == np.float32(0.5)
    np.testing.assert_array_equal(dst, np.float32(0.5) * V[0, 0] + np.float32(0.5) * V[1, 0])


def test_oracle_batch_equals_one_at_a_time():
    from oracle.qwen import QwenOracle
    cfg = synth.QwenConfig(256, 512, 2, 4, 2, 64, 1024, 32)
    o = QwenOracle(cfg, synth.qwen_weights(cfg, 5, symmetric=True))
    prompt = [int(t) for t in synth.rng(6).integers(0, cfg.vocab, 9)]
    o.reset()
    batch = o.forward(prompt, 0)
    k_batch = [k.copy() for k in o.K]
    o.reset()
    alone = np.stack([o.forward([t], i)[0] for i, t in enumerate(prompt)])
    np.testing.assert_array_equal(batch.view(np.uint32), alone.view(np.uint32))
    for a, b in zip(k_batch, o.K):
        np.testing.assert_array_equal(a, b)


def test_oracle_moe_half_adds_both_branches():
    """golem's TestMoEHalfAddsBothBranches (gemma/moe_test.go:273-322) on the
    oracle's moeHalf: both branches contribute, they differ, and the output
    is the residual plus post_ffw_norm of their sum."""
    from golem_amd.gemma import MoEConfig, moe_weights
    from oracle.gemma import moe_half
    cfg = MoEConfig(64, 64, 6, 2, 64)
    g = synth.rng(70)
    w = moe_weights(cfg, g)
    resid = synth.activations(g, 2, cfg.dim)
    out, shared, experts, ids, _ = moe_half(cfg, w, resid)
    for t in range(2):
        assert np.any(shared[t] != 0) and np.any(experts[t] != 0)
        assert not np.array_equal(shared[t], experts[t])
        assert len(set(ids[t].tolist())) == cfg.used
        want = resid[t] + oracle.rms_norm_plain(shared[t] + experts[t], w["post_ffw_norm"], cfg.eps)
        np.testing.assert_array_equal(out[t].view(np.uint32), want.astype(np.float32).view(np.uint32))


def _parallel(lib, q, K, V, kv, hd, n, scale):
    scores = np.zeros(max(n, 1), np.float32)
    dst = np.zeros(hd, np.float32)
    lib.orc_attend_parallel(oracle._p(q), oracle._p(K), oracle._p(V), K.shape[1], hd, kv, n, scale,
                         oracle._p(scores), oracle._p(dst))
    return dst, scores


def test_parallel_order_attention_closed_forms():
    """orc_attend_parallel (the decode attention's parallel order, this build's,
    not golem's): one position gives its value exactly; n identical keys give
    every position probability fp16(1/n) and the values' average; a total of
    exactly representable exponentials (all scores equal) is n whatever the
    order."""
    lib = oracle.load()
    hd, kv = 64, 2
    g = synth.rng(30)
    n = 200
    K = g.standard_normal((n, kv, hd)).astype(np.float16).astype(np.float32)
    V = g.standard_normal((n, kv, hd)).astype(np.float16).astype(np.float32)
    q = g.standard_normal(hd).astype(np.float16).astype(np.float32)
    dst, _ = _parallel(lib, q, K, V, 1, hd, 1, np.float32(0.125))
    np.testing.assert_array_equal(dst, V[0, 1])
    K[:, 0] = K[0, 0]  # every key of head 0 equal: probabilities fp16(1/n)
    dst, probs = _parallel(lib, q, K, V, 0, hd, n, np.float32(0.125))
    p = np.float32(np.float16(np.float32(1) / np.float32(n)))
    assert np.all(probs[:n] == p)
    want = np.float64(p) * V[:n, 0].astype(np.float64).sum(axis=0)
    np.testing.assert_allclose(dst, want, rtol=0, atol=1e-5)


def test_parallel_order_attention_near_golem():
    """The parallel order against golem's serial order (orc_attend) and a
    float64 evaluation: its head values within 1e-4 of RMS of golem's and of
    the exact softmax-weighted sum of the fp16-rounded probabilities -- a
    dropped run, a block summed twice, a probability of the wrong position or
    a value of the wrong element fails by far more."""
    lib = oracle.load()
    g = synth.rng(31)
    for hd, kv, n in ((128, 8, 640), (64, 2, 97), (32, 1, 33), (128, 4, 513)):
        K = g.standard_normal((n, kv, hd)).astype(np.float16).astype(np.float32)
        V = (g.standard_normal((n, kv, hd)) * 2).astype(np.float16).astype(np.float32)
        q = (g.standard_normal(hd) * 1.5).astype(np.float16).astype(np.float32)
        scale = np.float32(1 / math.sqrt(hd))
        h = kv - 1
        got, probs = _parallel(lib, q, K, V, h, hd, n, scale)
        scores = np.zeros(n, np.float32)
        serial = np.zeros(hd, np.float32)
        lib.orc_attend(oracle._p(q), oracle._p(K), oracle._p(V), kv, hd, h, n, scale, oracle._p(scores),
                       oracle._p(serial))
        rel, _ = oracle.compare_floats(got, serial)
        assert rel <= 1e-4, (hd, n, rel)
        s = (K[:, h].astype(np.float64) @ q.astype(np.float64)) * float(scale)
        e = np.exp(s - s.max())
        np.testing.assert_allclose(probs[:n], np.float16(e / e.sum()).astype(np.float32), rtol=2e-3, atol=1e-7)
        exact = probs[:n].astype(np.float64) @ V[:, h].astype(np.float64)
        rel, _ = oracle.compare_floats(got, exact.astype(np.float32))
        assert rel <= 1e-5, (hd, n, rel)
