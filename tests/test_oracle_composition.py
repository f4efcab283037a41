"""The oracle's compositions -- ExpertFFN (gemma/moe.go:112-180), moeHalf
(gemma/block.go:161-206) and the Qwen3 decoder (qwen/) -- against dense
float64 references written here in numpy, independently of oracle.c, and
the same checks with a mistake planted in the oracle's composition, which
must fail them.

- ExpertFFN: golem's own dense oracle (denseOracle, gemma/moe_test.go:66-118)
  restated, on golem's test shape (Dim 32, 6 experts, top 2, ExpertFFN 64,
  F32 stacks ~ N(0, 0.1), `wave` inputs) and golem's bar, 1e-4 absolute
  (TestExpertFFNMatchesTheOracle, :137-158).  F32 stacks are multiplied in
  float (Matrix.rows' F32 case), so the Q8_0 forms play no part.
- The Q4_0 expert units and moeHalf: the same dense arithmetic over the
  dequantised weights; the oracle quantises its activations to Q8_0, so the
  bar is 0.1 of RMS (worst element; the Q8_0 step is 1/254 of a block's
  largest value) and a planted mistake must exceed three times it.
- The Qwen3 decoder: a dense float64 block (norms, NeoX RoPE over the whole
  head, causal GQA attention, SwiGLU) over the dequantised weights, against
  QwenOracle's hidden states and logits.

Planted mistakes (each must move the result far past the bar): gate and up
swapped, DownScale dropped, the router fed the branch input, the post-norm
gains exchanged, a branch left out, the residual not added, RoPE pairing
adjacent elements, the query and key norms exchanged, key-value heads
assigned round-robin.
"""
import math

import numpy as np
import pytest

import oracle
from golem_amd import synth


# ---- independent float64 pieces -------------------------------------------

def rms64(x, gain=None, eps=1e-6):
    x = np.asarray(x, np.float64)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return y if gain is None else y * np.asarray(gain, np.float64)


def gelu_table64(x):
    """GELUTable (nn/gelu_table.go:19-52) in numpy: the tanh GELU of the
    input rounded to fp16, rounded to float32 and then fp16; inputs at or
    beyond +-10 pass through (or give 0)."""
    x = np.asarray(x, np.float32)
    h = x.astype(np.float16).astype(np.float64)
    g = 0.5 * h * (1.0 + np.tanh(0.7978845608028654 * h * (1.0 + 0.044715 * h * h)))
    t = g.astype(np.float32).astype(np.float16).astype(np.float64)
    return np.where(x <= -10, 0.0, np.where(x >= 10, x.astype(np.float64), t))


def choose64(logits, used):
    """chooseExperts (gemma/moe.go:62-88): repeated argmax (ties to the lower
    index), softmax over the chosen in float64."""
    lg = np.asarray(logits, np.float64).copy()
    ids = []
    for _ in range(used):
        i = int(np.argmax(lg))
        ids.append(i)
        lg[i] = -np.inf
    top = np.asarray(logits, np.float64)[ids]
    e = np.exp(top - top[0])
    return np.array(ids, np.int32), e / e.sum()


def dequant_q4_0(w, rows, cols):
    """Q4_0 rows (nn/dot_q4_0.go:3-13: byte j's low nibble is weight j, its
    high nibble weight j+16, stored +8; fp16 scale first) as float64."""
    b = np.asarray(w, np.uint8).reshape(rows, cols // 32, 18)
    d = b[:, :, :2].copy().view(np.float16).astype(np.float64)  # [rows][blocks][1]
    q = b[:, :, 2:]
    vals = np.concatenate([(q & 0x0F), (q >> 4)], axis=2).astype(np.float64) - 8.0
    return (vals * d).reshape(rows, cols)


def wave(n, phase):
    return np.sin(np.arange(n, dtype=np.float64) * 0.7 + phase).astype(np.float32)


# ---- ExpertFFN --------------------------------------------------------------

class Moe:
    """golem's randomMoEBlock shapes (gemma/moe_test.go:21-64) with numpy's
    generator: F32 router and stacks ~ N(0, 0.1), gains 1 + N(0, 0.05)."""

    def __init__(self, seed, D=32, E=6, used=2, FE=64, quant="f32"):
        g = synth.rng(seed)
        self.D, self.E, self.used, self.FE, self.quant = D, E, used, FE, quant
        self.router = (g.standard_normal((E, D)) * 0.1).astype(np.float32)
        self.router_scale = (1 + 0.05 * g.standard_normal(D)).astype(np.float32)
        self.down_scale = (1 + 0.05 * g.standard_normal(E)).astype(np.float32)
        if quant == "f32":
            self.gu = (g.standard_normal((E, 2 * FE, D)) * 0.1).astype(np.float32)
            self.dn = (g.standard_normal((E, D, FE)) * 0.1).astype(np.float32)
            self.gu64, self.dn64 = self.gu.astype(np.float64), self.dn.astype(np.float64)
        else:
            # per-expert scales far from one, so that dropping them shows
            self.down_scale = (1 + 0.5 * g.standard_normal(E)).astype(np.float32)
            self.gu_b = synth.q4_0_weights(g, E * 2 * FE, D).reshape(E, -1)
            self.dn_b = synth.q4_0_weights(g, E * D, FE).reshape(E, -1)
            self.gu64 = np.stack([dequant_q4_0(self.gu_b[e], 2 * FE, D) for e in range(E)])
            self.dn64 = np.stack([dequant_q4_0(self.dn_b[e], D, FE) for e in range(E)])

    def dense(self, resid, inp):
        """denseOracle (gemma/moe_test.go:66-118), float64."""
        x = rms64(resid) * (1 / math.sqrt(self.D)) * self.router_scale.astype(np.float64)
        logits = self.router.astype(np.float64) @ x
        ids, wts = choose64(logits, self.used)
        out = np.zeros(self.D)
        for k, e in enumerate(ids):
            gate = self.gu64[e, :self.FE] @ np.asarray(inp, np.float64)
            up = self.gu64[e, self.FE:] @ np.asarray(inp, np.float64)
            mid = gelu_table64(gate) * up
            out += wts[k] * self.down_scale[e] * (self.dn64[e] @ mid)
        return out, ids

    def oracle(self, resid, inp, plant=None):
        """ExpertFFN through the oracle: Route, the units, the Axpy sum; `plant`
        names a mistake to make in that composition."""
        router_in = inp if plant == "router reads the branch" else resid
        _, ids, wts = oracle.route_one(router_in, self.router, self.used, 1e-6, self.router_scale)
        parts = []
        for e in ids:
            if self.quant == "f32":
                gu, dn, q = self.gu[e], self.dn[e], oracle.F32
                if plant == "gate and up swapped":
                    gu = np.concatenate([gu[self.FE:], gu[:self.FE]])
            else:
                gu, dn, q = self.gu_b[e], self.dn_b[e], oracle.Q4_0
                if plant == "gate and up swapped":
                    half = len(gu) // 2
                    gu = np.concatenate([gu[half:], gu[:half]])
            parts.append(oracle.expert_unit(gu, dn, inp, self.D, self.FE, quant=q))
        ds = None if plant == "DownScale dropped" else self.down_scale
        return oracle.expert_reduce(np.stack(parts), ids, wts, self.D, ds), ids


PLANTS = ["gate and up swapped", "DownScale dropped", "router reads the branch"]


@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5])
def test_expert_ffn_matches_golems_dense_oracle(orc, seed):
    """TestExpertFFNMatchesTheOracle (gemma/moe_test.go:137-158): the branch
    input wave(Dim, 0), the router's input wave(Dim, 1.3), 1e-4 absolute."""
    m = Moe(seed)
    inp, resid = wave(m.D, 0), wave(m.D, 1.3)
    want, want_ids = m.dense(resid, inp)
    got, ids = m.oracle(resid, inp)
    assert ids.tolist() == want_ids.tolist()
    assert np.max(np.abs(got - want)) <= 1e-4


@pytest.mark.parametrize("plant", PLANTS)
def test_expert_ffn_planted_mistakes_fail(orc, plant):
    worst = 0.0
    for seed in (1, 2, 3):
        m = Moe(seed)
        inp, resid = wave(m.D, 0), wave(m.D, 1.3)
        want, _ = m.dense(resid, inp)
        got, _ = m.oracle(resid, inp, plant=plant)
        worst = max(worst, float(np.max(np.abs(got - want))))
    assert worst > 10 * 1e-4, f"{plant}: only {worst:.3g} from the dense oracle (the bar is 1e-4)"


def test_expert_ffn_batch_matches_one_position(orc):
    """TestExpertFFNBatchMatchesOnePosition (gemma/moe_test.go:164-205): five
    positions (inputs wave(Dim, 0.31 t), residuals wave(Dim, 0.91 t + 2))
    through the oracle's composition in one pass equal the same positions
    alone -- here both follow the dense oracle within golem's 1e-4."""
    m = Moe(2)
    for t in range(5):
        inp, resid = wave(m.D, 0.31 * t), wave(m.D, 0.91 * t + 2)
        want, _ = m.dense(resid, inp)
        got, _ = m.oracle(resid, inp)
        assert np.max(np.abs(got - want)) <= 1e-4, f"position {t}"


def _rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / np.sqrt(np.mean(want * want)))


# Q8_0 activations move each product by about 1% of its RMS (a step of 1/254
# of a block's largest value, in every product), and the largest of a few
# thousand such errors reaches ~5%; every planted mistake moves the result by
# several tens of percent.
Q8_BAR = 0.1


@pytest.mark.parametrize("plant", [None] + PLANTS)
def test_q4_0_expert_units_against_dense(orc, plant):
    """The Q4_0 units the configs run, at config 4's widths (2816 wide,
    experts of 704, top 8 of 16 here), against the dense float64 arithmetic
    over the dequantised weights; the planted mistakes fail."""
    m = Moe(40, D=2816, E=16, used=8, FE=704, quant="q4_0")
    g = synth.rng(41)
    worst = 0.0
    for t in range(2):
        inp = g.standard_normal(m.D).astype(np.float32)
        resid = g.standard_normal(m.D).astype(np.float32)
        want, want_ids = m.dense(resid, inp)
        got, ids = m.oracle(resid, inp, plant=plant)
        if plant is None:
            assert ids.tolist() == want_ids.tolist()
        worst = max(worst, _rel(got, want))
    print(f"q4_0 units plant={plant}: {worst:.3g} of RMS")
    if plant is None:
        assert worst <= Q8_BAR, f"{worst:.3g} of RMS"
    else:
        assert worst > 3 * Q8_BAR, f"{plant}: only {worst:.3g} of RMS"


# ---- moeHalf ----------------------------------------------------------------

def dense_moe_half(cfg, w, resid):
    """moeHalf (gemma/block.go:161-206) in float64 over dequantised weights."""
    D, F, E, FE, k = cfg.dim, cfg.ffn, cfg.experts, cfg.expert_ffn, cfg.used
    gate = dequant_q4_0(w["gate"], F, D)
    up = dequant_q4_0(w["up"], F, D)
    down = dequant_q4_0(w["down"], D, F)
    gu = dequant_q4_0(w["gate_up_exps"], E * 2 * FE, D).reshape(E, 2 * FE, D)
    dn = dequant_q4_0(w["down_exps"], E * D, FE).reshape(E, D, FE)
    out = []
    for r in np.asarray(resid, np.float64):
        normed = rms64(r, w["ffn_norm"])
        shared = down @ (gelu_table64(gate @ normed) * (up @ normed))
        exp_in = rms64(r, w["pre_ffw_norm_2"])
        x = rms64(r) * (1 / math.sqrt(D)) * w["router_scale"].astype(np.float64)
        ids, wts = choose64(w["router"].astype(np.float64) @ x, k)
        experts = np.zeros(D)
        for j, e in enumerate(ids):
            mid = gelu_table64(gu[e, :FE] @ exp_in) * (gu[e, FE:] @ exp_in)
            experts += wts[j] * w["down_scale"][e] * (dn[e] @ mid)
        shared = rms64(shared, w["post_ffw_norm_1"])
        experts = rms64(experts, w["post_ffw_norm_2"])
        out.append(r + rms64(shared + experts, w["post_ffw_norm"]))
    return np.stack(out)


@pytest.mark.parametrize("plant", [None, "post-norm gains exchanged", "shared branch left out", "residual not added"])
def test_moe_half_against_dense(orc, plant):
    from golem_amd.gemma import MoEConfig, moe_weights
    from oracle.gemma import moe_half
    cfg = MoEConfig(256, 512, 8, 2, 128)
    g = synth.rng(71)
    w = moe_weights(cfg, g)
    for name in ("post_ffw_norm", "post_ffw_norm_1", "post_ffw_norm_2"):  # gains far from one, so that a swap shows
        w[name] = (1 + 0.6 * g.standard_normal(cfg.dim)).astype(np.float32)
    resid = (3 * g.standard_normal((3, cfg.dim))).astype(np.float32)
    want = dense_moe_half(cfg, w, resid)
    wo = dict(w)
    if plant == "post-norm gains exchanged":
        wo["post_ffw_norm_1"], wo["post_ffw_norm_2"] = w["post_ffw_norm_2"], w["post_ffw_norm_1"]
    out, shared, experts, _, _ = moe_half(cfg, wo, resid)
    if plant == "shared branch left out":
        out = np.stack([resid[t] + oracle.rms_norm_plain(experts[t], w["post_ffw_norm"], cfg.eps)
                        for t in range(len(resid))])
    if plant == "residual not added":
        out = out - resid
    rel = max(_rel(out[t] - resid[t], want[t] - resid[t]) for t in range(len(resid)))
    print(f"moe half plant={plant}: {rel:.3g} of RMS")
    if plant is None:
        assert rel <= Q8_BAR, f"{rel:.3g} of RMS"
    else:
        assert rel > 3 * Q8_BAR, f"{plant}: only {rel:.3g} of RMS"


# ---- the Qwen3 decoder -------------------------------------------------------

def dense_qwen(cfg, w, tokens, plant=None):
    """ForwardBatch (qwen/model.go:127-175) for one prompt in float64 over the
    dequantised weights: the final-normed hidden states of every position.
    `plant` makes one mistake in this reference (to show the comparison
    catches it; the oracle is never changed)."""
    hd, H, KV = cfg.head_dim, cfg.heads, cfg.kv_heads
    qd, kvd = H * hd, KV * hd
    emb = np.stack([oracle.dequantize_q6_k(w["token_embd"][t * (cfg.dim // 256) * 210:(t + 1) * (cfg.dim // 256) * 210],
                                           cfg.dim) for t in tokens]).astype(np.float64)
    M = len(tokens)
    half = hd // 2
    freqs = np.array([cfg.rope_base ** (-2.0 * i / hd) for i in range(half)])

    def rope(v, p):
        th = p * freqs
        c, s = np.cos(th), np.sin(th)
        if plant == "RoPE pairs adjacent elements":
            a, b = v[0::2].copy(), v[1::2].copy()
            out = v.copy()
            out[0::2], out[1::2] = a * c - b * s, a * s + b * c
            return out
        a, b = v[:half], v[half:]
        return np.concatenate([a * c - b * s, a * s + b * c])

    xs = emb.copy()
    for b in w["blocks"]:
        Wq, Wk, Wv = dequant_q4_0(b["q"], qd, cfg.dim), dequant_q4_0(b["k"], kvd, cfg.dim), dequant_q4_0(b["v"], kvd, cfg.dim)
        Wo = dequant_q4_0(b["o"], cfg.dim, qd)
        Wg, Wu = dequant_q4_0(b["gate"], cfg.ffn, cfg.dim), dequant_q4_0(b["up"], cfg.ffn, cfg.dim)
        Wd = dequant_q4_0(b["down"], cfg.dim, cfg.ffn)
        qn, kn = (b["k_norm"], b["q_norm"]) if plant == "query and key norms exchanged" else (b["q_norm"], b["k_norm"])
        normed = rms64(xs, b["attn_norm"])
        q, k, v = normed @ Wq.T, normed @ Wk.T, normed @ Wv.T
        Q = np.stack([np.concatenate([rope(rms64(q[t, h * hd:(h + 1) * hd], qn), t) for h in range(H)]) for t in range(M)])
        K = np.stack([np.stack([rope(rms64(k[t, h * hd:(h + 1) * hd], kn), t) for h in range(KV)]) for t in range(M)])
        V = v.reshape(M, KV, hd)
        att = np.zeros((M, qd))
        for t in range(M):
            for h in range(H):
                kvh = h % KV if plant == "key-value heads round-robin" else h // (H // KV)
                sc = K[:t + 1, kvh] @ Q[t, h * hd:(h + 1) * hd] / math.sqrt(hd)
                p = np.exp(sc - sc.max())
                att[t, h * hd:(h + 1) * hd] = (p / p.sum()) @ V[:t + 1, kvh]
        xs = xs + att @ Wo.T
        normed = rms64(xs, b["ffn_norm"])
        gt, up = normed @ Wg.T, normed @ Wu.T
        xs = xs + (gt / (1 + np.exp(-gt)) * up) @ Wd.T
    return rms64(xs, w["output_norm"], cfg.eps)


QWEN_PLANTS = ["RoPE pairs adjacent elements", "query and key norms exchanged", "key-value heads round-robin"]


@pytest.mark.parametrize("plant", [None] + QWEN_PLANTS)
def test_qwen_oracle_against_dense(orc, plant):
    """QwenOracle's hidden states (two blocks, a 10-token prompt, head 64 with
    two query heads per key-value head, zero-mean weights) against the dense
    float64 decoder; each planted mistake in the dense decoder is caught."""
    from oracle.qwen import QwenOracle
    cfg = synth.QwenConfig(256, 512, 2, 4, 2, 64, 1024, 32)
    w = synth.qwen_weights(cfg, 81, symmetric=True)
    for b in w["blocks"]:  # head-norm gains far from one, so that exchanging them shows
        b["q_norm"] = (1 + 0.6 * synth.rng(82).standard_normal(cfg.head_dim)).astype(np.float32)
        b["k_norm"] = (1 + 0.6 * synth.rng(83).standard_normal(cfg.head_dim)).astype(np.float32)
    prompt = [int(t) for t in synth.rng(84).integers(0, cfg.vocab, 10)]
    got = QwenOracle(cfg, w).forward(prompt, 0)
    want = dense_qwen(cfg, w, prompt, plant)
    rel = max(_rel(got[t], want[t]) for t in range(len(prompt)))
    print(f"qwen plant={plant}: {rel:.3g} of RMS")
    if plant is None:
        assert rel <= Q8_BAR, f"{rel:.3g} of RMS"
    else:
        assert rel > 3 * Q8_BAR, f"{plant}: only {rel:.3g} of RMS"
