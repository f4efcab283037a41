"""Config 3's prompt path at its configured length: a 512-token prefill at the
full width (2560, FFN 9728, 32/8 heads of 128) on the device against the
oracle's restatement of golem's engine (oracle/qwen.py).

A prompt of more than 16 positions runs kernels a short prompt never
reaches: the 64-token int8 MFMA product (Q|K|V, O, Down), the same product
with the SwiGLU + Q8_0 epilogue (Gate|Up), the head-norm/RoPE pass at
M = 512, and the prompt attention's three passes (scores, softmax, values in
16-token workgroups).  golem reads such a prompt through ForwardBatch
(qwen/model.go:127-175) and Attention (qwen/attention.go:86-124).

- the attention alone at config 3's heads over a 512-position prompt: the
  Q8_0 of every head of one or more tokens of each 16-token group, bit for
  bit against golem's orc_attend;
- two full-width blocks over a 512-token prompt, stage by stage on sampled
  positions of every token group (each stage fed the device's own inputs,
  as in test_gpu_qwen_full.py), plus every key and value cache entry of
  all 512 positions bit for bit;
- a 48-token prompt read in one batch equal, bit for bit, to the same
  tokens one at a time at full width (TestBatchAgreesWithOneAtATime,
  qwen/model_test.go:78).
"""
import math

import numpy as np
import pytest
import torch

from golem_amd import capi, synth
from golem_amd.qwen import QwenModel
from tests.gpu_util import log

pytestmark = pytest.mark.gpu

TOL = 1e-5
PROMPT = 512
# one token of every 16-token group of the values pass (at a different
# offset in each), and the groups' edges at both ends and the middle
SAMPLE = sorted(set([16 * g + (7 * g) % 16 for g in range(PROMPT // 16)]
                    + [0, 1, 15, 16, 17, 255, 256, 510, 511]))


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _config3(layers, context):
    return synth.QwenConfig(2560, 9728, layers, 32, 8, 128, 151936, context)


def test_prompt_attention_config3_heads_512(dev, orc):
    """gx_qwen_attention over a 512-position prompt (every position a query
    at its own position, the last seeing all 512) at config 3's heads."""
    hd, heads, kv = 128, 32, 8
    g = synth.rng(512)
    M = PROMPT
    pos = np.arange(M, dtype=np.int32)
    context = M
    kcf = g.standard_normal((M, kv, hd)).astype(np.float16)
    vcf = (g.standard_normal((M, kv, hd)) * 2).astype(np.float16)
    qf = (g.standard_normal((M, heads * hd)) * 1.5).astype(np.float16)
    vt = np.ascontiguousarray(vcf.transpose(1, 2, 0))  # [kv][hd][context]
    kt = np.ascontiguousarray(kcf.reshape(M, kv, hd // 8, 8).transpose(1, 2, 0, 3))  # [kv][hd/8][context][8]
    q8 = dev.empty((M, heads * hd), np.int8)
    sc = dev.empty((M, heads * hd // 32), np.float32)
    qs = dev.empty((M, heads * hd // 32), np.int32)
    n = capi.size_out("gx_qwen_attention_workspace_bytes", M, heads, M - 1)
    ws = dev.empty((n,), np.uint8)
    ins = [dev.put(a) for a in (qf.view(np.int16), pos, kt.view(np.int16), vt.view(np.int16))]
    log(f"prompt attention {heads}/{kv} heads x {hd}, {M} positions")
    capi.call("gx_qwen_attention", dev.ctx.ptr, capi.vp(ins[0]), M, heads, kv, hd, M - 1, capi.vp(ins[1]),
              capi.vp(ins[2]), capi.vp(ins[3]), context, capi.vp(q8), capi.vp(sc), capi.vp(qs), capi.vp(ws), n,
              None, 0)
    lib = orc.load()
    K32, V32 = np.ascontiguousarray(kcf.astype(np.float32)), np.ascontiguousarray(vcf.astype(np.float32))
    scale = np.float32(1 / math.sqrt(float(hd)))
    out = np.zeros((len(SAMPLE), heads * hd), np.float32)
    scores = np.zeros(M, np.float32)
    for i, t in enumerate(SAMPLE):
        for h in range(heads):
            query = np.ascontiguousarray(qf[t, h * hd:(h + 1) * hd].astype(np.float32))
            dst = np.zeros(hd, np.float32)
            lib.orc_attend(orc._p(query), orc._p(K32), orc._p(V32), kv, hd, h // (heads // kv), t + 1, scale,
                           orc._p(scores), orc._p(dst))
            out[i, h * hd:(h + 1) * hd] = dst
    b = orc.Batch(out).quantize()
    got_q, got_s, got_qs = dev.get(q8)[SAMPLE], dev.get(sc)[SAMPLE], dev.get(qs)[SAMPLE]
    for i, t in enumerate(SAMPLE):
        assert np.array_equal(got_q[i], b.q_rows()[i]), f"token {t} (group {t // 16}): head Q8_0"
        assert np.array_equal(_bits(got_s[i]), _bits(b.scales_rows()[i])), f"token {t}: head scales"
        assert np.array_equal(got_qs[i], b.qsum_rows()[i]), f"token {t}: head sums"
    log(f"  {len(SAMPLE)} tokens from {len(set(t // 16 for t in SAMPLE))} token groups bit for bit")


def check_block_sampled(model, om, orc, prompt, layer):
    """One block of a long prompt, stage by stage, on the SAMPLE positions;
    every stage fed the device's own inputs so nothing accumulates."""
    from oracle import Batch
    cfg, M, S = model.cfg, len(prompt), SAMPLE
    pos = list(range(M))
    xin = model.residual(prompt, 0, layer)
    xout = model.residual(prompt, 0, layer + 1)

    def dev(t):
        return t[:M].cpu().numpy().copy()

    set_q, set_s, attn = dev(model.set8.q), dev(model.set8.s), dev(model.attn)
    mid_q, mid_s, ffn = dev(model.mid8.q), dev(model.mid8.s), dev(model.ffn)
    kc, vc = model.kc[layer].cpu().numpy(), model.vc[layer].cpu().numpy()
    # the Gate|Up floats of the device's own pre-norm (the block hands SwiGLU's
    # Q8_0 on from the product's epilogue without them)
    model._mm(model.blocks[layer]["gu"], model.x8, M, model.gu, 2 * cfg.ffn)
    x8_q, x8_s, gu = dev(model.x8.q), dev(model.x8.s), dev(model.gu)
    # likewise the Q|K|V floats (the heads' norms, RoPE and cache stores run
    # in the product's epilogue): the block input's attention pre-norm and
    # Q8_0 again, then the product alone
    b = model.blocks[layer]
    xd = torch.from_numpy(np.ascontiguousarray(xin)).cuda()
    aq = torch.empty((M, cfg.dim), dtype=torch.int8, device="cuda")
    asc = torch.empty((M, cfg.dim // 32), dtype=torch.float32, device="cuda")
    aqs = torch.empty((M, cfg.dim // 32), dtype=torch.int32, device="cuda")
    capi.call("gx_norm_quant", model.ctx.ptr, capi.vp(xd), cfg.dim, None, cfg.dim, capi.vp(b["attn_norm"]), M,
              cfg.dim, np.float32(cfg.eps), None, 0, capi.vp(aq), capi.vp(asc), capi.vp(aqs))
    qkv_d = torch.empty((M, model.qd + 2 * model.kvd), dtype=torch.float32, device="cuda")
    capi.call("gx_matmul_q4_0", model.ctx.ptr, b["qkv"].ptr, capi.vp(aq), capi.vp(asc), capi.vp(aqs), None, M, 0,
              model.qd + 2 * model.kvd, None, capi.vp(qkv_d), model.qd + 2 * model.kvd)
    qkv = qkv_d.cpu().numpy()

    def rel(got, want):
        return max(orc.compare_floats(got[i], want[i])[0] for i in range(len(want)))

    qd, kvd, hd = model.qd, model.kvd, cfg.head_dim
    worst = {}
    nA = om.norm(layer, xin[S], "attn_norm")
    q, k, v = (om._mat(layer, n, nA) for n in ("q", "k", "v"))
    worst["qkv"] = rel(qkv[S], np.concatenate([q, k, v], axis=1))
    # head norms + RoPE + cache entries of every position, then the attention
    # of the sampled tokens over the device's Q|K|V rows
    out = om.attend(layer, qkv[:, :qd], qkv[:, qd:qd + kvd], qkv[:, qd + kvd:], pos, only=S)
    got_k = kc[0].view(np.float16).astype(np.float32)  # [kv][hd/8][context][8]
    got_k = got_k[:, :, :M, :].transpose(2, 0, 1, 3).reshape(M, cfg.kv_heads, hd)
    got_v = vc[0].view(np.float16).astype(np.float32)[:, :, :M].transpose(2, 0, 1)  # [kv][hd][context]
    assert np.array_equal(_bits(got_k), _bits(om.K[layer][:M])), f"block {layer}: key cache"
    assert np.array_equal(_bits(got_v), _bits(om.V[layer][:M])), f"block {layer}: value cache"
    heads = Batch(out).quantize()
    for i, t in enumerate(S):
        assert np.array_equal(set_q[t], heads.q_rows()[i]), f"block {layer} token {t}: attention Q8_0"
        assert np.array_equal(_bits(set_s[t]), _bits(heads.scales_rows()[i])), f"block {layer} token {t}: scales"
    worst["o"] = rel(attn[S], om._mat(layer, "o", heads))
    xs = xin[S] + attn[S]
    nF = om.norm(layer, xs, "ffn_norm")
    assert np.array_equal(x8_q[S], nF.q_rows()), f"block {layer}: FFN pre-norm Q8_0"
    assert np.array_equal(_bits(x8_s[S]), _bits(nF.scales_rows())), f"block {layer}: FFN pre-norm scales"
    g4 = gu[S].reshape(len(S), -1, 64)  # gate and up rows interleaved by 32
    gate, up = g4[:, :, :32].reshape(len(S), -1), g4[:, :, 32:].reshape(len(S), -1)
    worst["gate"] = rel(gate, om._mat(layer, "gate", nF))
    worst["up"] = rel(up, om._mat(layer, "up", nF))
    mid = Batch(om.swiglu(gate, up)).quantize()
    assert np.array_equal(mid_q[S], mid.q_rows()), f"block {layer}: SwiGLU Q8_0"
    assert np.array_equal(_bits(mid_s[S]), _bits(mid.scales_rows())), f"block {layer}: SwiGLU scales"
    worst["down"] = rel(ffn[S], om._mat(layer, "down", mid))
    assert np.array_equal(_bits(xout[S]), _bits(xs + ffn[S])), f"block {layer}: residual adds"
    for stage, r in worst.items():
        assert r <= TOL, f"block {layer} {stage}: {r:.3g} of RMS"
    log(f"  block {layer}: " + ", ".join(f"{k} {v:.2g}" for k, v in worst.items()) + " of RMS")
    return max(worst.values())


@pytest.mark.parametrize("symmetric", [False, True])
def test_prompt_512_two_blocks_stage_by_stage(dev, orc, symmetric):
    from oracle.qwen import QwenOracle
    cfg = _config3(2, PROMPT)
    log(f"config 3 width, 2 blocks, {PROMPT}-token prompt, symmetric={symmetric}: drawing weights")
    w = synth.qwen_weights(cfg, 3 + symmetric, symmetric=symmetric)
    model = QwenModel(dev.ctx, cfg, w, max_batch=PROMPT, attention="golem")
    om = QwenOracle(cfg, w)
    prompt = [int(t) for t in synth.rng(3).integers(0, cfg.vocab, PROMPT)]
    for layer in range(cfg.layers):
        check_block_sampled(model, om, orc, prompt, layer)
    log(f"  {len(SAMPLE)} sampled positions from {len(set(t // 16 for t in SAMPLE))} token groups")
    model.free()


def test_prompt_48_batch_equals_one_at_a_time_full_width(dev):
    """golem's TestBatchAgreesWithOneAtATime (qwen/model_test.go:78) at
    config 3's width: 48 tokens in one batch (the 64-token int8 product,
    the prompt attention's three passes over three token groups) against the
    same tokens one position at a time (the decode kernels), hidden states
    and caches bit for bit, in golem's attention order."""
    cfg = _config3(2, 64)
    w = synth.qwen_weights(cfg, 35, symmetric=True)
    model = QwenModel(dev.ctx, cfg, w, max_batch=48, attention="golem")
    prompt = [int(t) for t in synth.rng(35).integers(0, cfg.vocab, 48)]
    log(f"config 3 width, 2 blocks: {len(prompt)} tokens in one batch against one at a time")
    model.reset()
    batch = dev.get(model.forward(prompt, 0)).copy()
    kb = [k.cpu().numpy().copy() for k in model.kc]
    vb = [v.cpu().numpy().copy() for v in model.vc]
    model.reset()
    alone = np.stack([dev.get(model.forward([t], i))[0].copy() for i, t in enumerate(prompt)])
    np.testing.assert_array_equal(_bits(batch), _bits(alone))
    for layer in range(cfg.layers):
        np.testing.assert_array_equal(kb[layer], model.kc[layer].cpu().numpy())
        np.testing.assert_array_equal(vb[layer], model.vc[layer].cpu().numpy())
    torch.cuda.synchronize()
    model.free()


# (head width, heads, key-value heads, prompt length M, first position, context)
PROMPT_PARALLEL = [(128, 32, 8, PROMPT, 0, 640), (64, 4, 2, 70, 0, 80), (128, 8, 2, 37, 100, 200),
                   (32, 8, 1, 5, 0, 8), (96, 4, 4, 33, 31, 72), (128, 4, 1, 64, 960, 1024)]
# One fp16 step of a probability near 1 (2^-11), times a value element of
# ~3 RMS: what one probability that rounds the other way moves a head by.
FP16_STEP = 2e-3


def _prompt_case(dev, orc, hd, heads, kv, M, start, context, exact):
    """A prompt's caches and queries (cache entries past the prompt hold NaN
    bits), the MFMA form's head floats and Q8_0, and the rows compared.
    exact: queries and keys on a grid of 1/4 (|q|, |k| <= 1/2), so that every
    dot product is exact in any order and the scores are golem's bits."""
    g = synth.rng(700 + M + hd + start + exact)
    n = start + M
    pos = np.arange(start, n, dtype=np.int32)
    if exact:
        kcf = (g.integers(-2, 3, (n, kv, hd)) * 0.25).astype(np.float16)
        qf = (g.integers(-2, 3, (M, heads * hd)) * 0.25).astype(np.float16)
    else:
        kcf = g.standard_normal((n, kv, hd)).astype(np.float16)
        qf = (g.standard_normal((M, heads * hd)) * 1.5).astype(np.float16)
    vcf = (g.standard_normal((n, kv, hd)) * 2).astype(np.float16)
    nan = np.array([0x7E00], np.uint16).view(np.float16)[0]
    vt = np.full((kv, hd, context), nan, np.float16)
    vt[:, :, :n] = vcf.transpose(1, 2, 0)
    kt = np.full((kv, hd // 8, context, 8), nan, np.float16)
    kt[:, :, :n, :] = kcf.reshape(n, kv, hd // 8, 8).transpose(1, 2, 0, 3)
    ins = [dev.put(a) for a in (qf.view(np.int16), pos, kt.view(np.int16), vt.view(np.int16))]
    log(f"prompt attention (MFMA) hd={hd} heads={heads}/{kv} M={M} from {start}, context {context}, exact={exact}")
    heads_f = dev.empty((M, heads * hd), np.float32)
    capi.call("gx_qwen_attention_heads", dev.ctx.ptr, capi.vp(ins[0]), M, heads, kv, hd, n - 1, capi.vp(ins[1]),
              capi.vp(ins[2]), capi.vp(ins[3]), context, capi.vp(heads_f))
    q8 = dev.empty((M, heads * hd), np.int8)
    sc = dev.empty((M, heads * hd // 32), np.float32)
    qs = dev.empty((M, heads * hd // 32), np.int32)
    nw = capi.size_out("gx_qwen_attention_workspace_bytes", M, heads, n - 1)
    ws = dev.empty((nw,), np.uint8)
    capi.call("gx_qwen_attention_parallel", dev.ctx.ptr, capi.vp(ins[0]), M, heads, kv, hd, n - 1, capi.vp(ins[1]),
              capi.vp(ins[2]), capi.vp(ins[3]), context, capi.vp(q8), capi.vp(sc), capi.vp(qs), capi.vp(ws), nw,
              None, 0)
    rows = list(range(M)) if M <= 80 else SAMPLE
    got = dev.get(heads_f)[rows]
    # the Q8_0 output is the head floats' own, bit for bit
    mine = orc.Batch(np.ascontiguousarray(got)).quantize()
    gq = dev.get(q8)[rows]
    np.testing.assert_array_equal(gq, mine.q_rows())
    np.testing.assert_array_equal(_bits(dev.get(sc)[rows]), _bits(mine.scales_rows()))
    np.testing.assert_array_equal(dev.get(qs)[rows], mine.qsum_rows())
    return qf, kcf, vcf, pos, rows, got, gq


def _oracle_heads(orc, fn, qf, kcf, vcf, pos, rows, hd, heads, kv):
    lib = orc.load()
    K32, V32 = np.ascontiguousarray(kcf.astype(np.float32)), np.ascontiguousarray(vcf.astype(np.float32))
    scale = np.float32(1 / math.sqrt(float(hd)))
    want = np.zeros((len(rows), heads * hd), np.float32)
    scores = np.zeros(len(kcf), np.float32)
    for i, t in enumerate(rows):
        for h in range(heads):
            query = np.ascontiguousarray(qf[t, h * hd:(h + 1) * hd].astype(np.float32))
            dst = np.zeros(hd, np.float32)
            getattr(lib, fn)(orc._p(query), orc._p(K32), orc._p(V32), kv, hd, h // (heads // kv), int(pos[t]) + 1,
                             scale, orc._p(scores), orc._p(dst))
            want[i, h * hd:(h + 1) * hd] = dst
    return want


def _compare(orc, got, want, gq, rows, pos, heads, hd, bar):
    worst, over = 0.0, 0
    for i, t in enumerate(rows):
        for h in range(heads):
            rel, at = orc.compare_floats(got[i, h * hd:(h + 1) * hd], want[i, h * hd:(h + 1) * hd])
            worst = max(worst, rel)
            over += rel > 1e-4
            assert rel <= bar, f"token {t} (position {pos[t]}) head {h}: {rel:.3g} of RMS at {at}"
    dq = gq.astype(np.int32) - orc.Batch(want).quantize().q_rows().astype(np.int32)
    moved = int(np.count_nonzero(dq))
    log(f"  {len(rows)} tokens: worst {worst:.2g} of RMS ({over} of {len(rows) * heads} heads above 1e-4), "
        f"{moved} of {dq.size} Q8_0 values one step off")
    assert np.abs(dq).max() <= 1 and moved <= max(2, dq.size // 100)


@pytest.mark.parametrize("hd,heads,kv,M,start,context", PROMPT_PARALLEL)
def test_prompt_attention_mfma_exact_scores(dev, orc, hd, heads, kv, M, start, context):
    """The MFMA prompt form on scores that are exact in any order (queries and
    keys on a grid of 1/4): everything up to the probabilities is then the
    decode's parallel order bit for bit -- the same maximum, float64
    exponentials, pairwise block totals and fp16 probabilities -- so against
    its restatement (orc_attend_parallel) the heads differ only by the value
    sums' order (the matrix core's against runs of 32 fma chains): within
    1e-5 of RMS (about 1e-6 seen).  A wrong token, head, position bound or value element moves
    a head by O(1).  Ragged token tiles, prompts that continue a cache, head
    widths 32 to 128, prefixes up to the form's 1024; cache entries past the
    prompt hold NaN bits, so a position no token attends never reaches a
    sum."""
    qf, kcf, vcf, pos, rows, got, gq = _prompt_case(dev, orc, hd, heads, kv, M, start, context, True)
    want = _oracle_heads(orc, "orc_attend_parallel", qf, kcf, vcf, pos, rows, hd, heads, kv)
    _compare(orc, got, want, gq, rows, pos, heads, hd, 1e-5)


@pytest.mark.parametrize("hd,heads,kv,M,start,context", PROMPT_PARALLEL)
def test_prompt_attention_mfma_against_golem(dev, orc, hd, heads, kv, M, start, context):
    """The MFMA prompt form on random fp16 queries and keys against golem's
    attention (orc_attend, qwen/attention.go:86-124).  The scores are now
    golem's within an ulp or two, not bit for bit, and golem rounds every
    probability to fp16 (attention.go:112-114): a probability that sits on a
    rounding boundary goes the other way, and a short prefix's probabilities
    are large, so a head can move by one fp16 step of its largest probability
    times a value element -- up to FP16_STEP of RMS (4e-4 seen at a token of
    18 positions).  The bar is that step; the heads above the decode form's
    1e-4 are counted and logged, and the Q8_0 of the heads is golem's but for
    values on a rounding boundary (one step, at most 1 % of them)."""
    qf, kcf, vcf, pos, rows, got, gq = _prompt_case(dev, orc, hd, heads, kv, M, start, context, False)
    want = _oracle_heads(orc, "orc_attend", qf, kcf, vcf, pos, rows, hd, heads, kv)
    _compare(orc, got, want, gq, rows, pos, heads, hd, FP16_STEP)
