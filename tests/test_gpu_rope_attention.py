"""gx_qwen_rope_attention, the decode step's head norms + RoPE + cache store
+ attention in one kernel, against the two calls it replaces
(gx_qwen_qk_rope then gx_qwen_attention, qwen/attention.go:57-124 at batch
1), bit for bit: the Q8_0 of the heads (values, scales, sums) and both caches
after the call.

The caches are filled with random entries first, so that the position's own
key and value -- which the fused kernel takes from its computed copies, not
from the entries it is writing -- meet a full prefix.  Cases: golem's head of
128 with four query heads per key-value head (config 3), the other head widths
and group sizes, the first position, a middle one and the last, max_pos at the
position and at the end of the cache (the captured decode graph's launch), and
the slots form: a conversation's own caches, and a position in no
conversation (its output NaN-derived, nothing stored)."""
import numpy as np
import pytest
import torch

from golem_amd import capi, synth

CASES = [(128, 32, 8, 640), (128, 16, 8, 200), (64, 4, 2, 304), (32, 8, 1, 96), (96, 4, 4, 136),
         (64, 8, 1, 768)]


def run_case(dev, hd, heads, kv, context, pos, max_pos, slots=None, nslots=1, seed=0, parallel=False):
    g = synth.rng(seed + 7 * pos + hd)
    width = (heads + 2 * kv) * hd
    qkv = (g.standard_normal((1, width)) * 3).astype(np.float32)
    qn = (1 + 0.02 * g.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.02 * g.standard_normal(hd)).astype(np.float32)
    cos = g.uniform(-1, 1, (context, hd // 2)).astype(np.float32)
    sin = g.uniform(-1, 1, (context, hd // 2)).astype(np.float32)
    kc0 = (g.standard_normal((nslots, kv, hd // 8, context, 8))).astype(np.float16)
    vc0 = (g.standard_normal((nslots, kv, hd, context)) * 2).astype(np.float16)
    ins = [dev.put(a) for a in (qkv, np.array([pos], np.int32), qn, kn, cos, sin)]
    sl = dev.put(np.array([slots], np.int32)) if slots is not None else None
    eps = np.float32(1e-6)
    outs = []
    for fused in (False, True):
        kc = dev.put(kc0.view(np.int16))
        vc = dev.put(vc0.view(np.int16))
        q8 = dev.empty((1, heads * hd), np.int8)
        sc = dev.empty((1, heads * hd // 32), np.float32)
        qs = dev.empty((1, heads * hd // 32), np.int32)
        sfx = "_parallel" if parallel else ""
        if fused:
            capi.call("gx_qwen_rope_attention" + sfx, dev.ctx.ptr, capi.vp(ins[0]), width, heads, kv, hd, max_pos,
                      capi.vp(ins[1]), capi.vp(ins[2]), capi.vp(ins[3]), capi.vp(ins[4]), capi.vp(ins[5]), eps,
                      capi.vp(kc), capi.vp(vc), context, capi.vp(q8), capi.vp(sc), capi.vp(qs),
                      capi.vp(sl) if sl is not None else None, nslots)
        else:
            qh = dev.empty((1, heads * hd), np.int16)
            capi.call("gx_qwen_qk_rope", dev.ctx.ptr, capi.vp(ins[0]), width, 1, heads, kv, hd, capi.vp(ins[1]),
                      capi.vp(ins[2]), capi.vp(ins[3]), capi.vp(ins[4]), capi.vp(ins[5]), eps, capi.vp(qh),
                      capi.vp(kc), capi.vp(vc), context, capi.vp(sl) if sl is not None else None, nslots)
            n = capi.size_out("gx_qwen_attention_workspace_bytes", 1, heads, max_pos)
            ws = dev.empty((n,), np.uint8)
            capi.call("gx_qwen_attention" + sfx, dev.ctx.ptr, capi.vp(qh), 1, heads, kv, hd, max_pos, capi.vp(ins[1]),
                      capi.vp(kc), capi.vp(vc), context, capi.vp(q8), capi.vp(sc), capi.vp(qs), capi.vp(ws), n,
                      capi.vp(sl) if sl is not None else None, nslots)
        dev.ctx.sync()
        outs.append([dev.get(a) for a in (q8, sc, qs, kc, vc)])
    for name, a, b in zip(("q", "scales", "sums", "key cache", "value cache"), *outs):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), \
            f"{name} differs (hd {hd}, heads {heads}/{kv}, pos {pos}, max_pos {max_pos}, slot {slots}, " \
            f"parallel {parallel})"
    return outs[1] + [kc0.view(np.int16), vc0.view(np.int16)]


@pytest.mark.gpu
@pytest.mark.parametrize("parallel", [False, True])
@pytest.mark.parametrize("hd,heads,kv,context", CASES)
def test_rope_attention_matches_two_calls(dev, hd, heads, kv, context, parallel):
    for pos in (0, 7, 8, context // 2 + 3, context - 1):
        run_case(dev, hd, heads, kv, context, pos, pos, parallel=parallel)
    run_case(dev, hd, heads, kv, context, context // 3, context - 1, parallel=parallel)


@pytest.mark.gpu
@pytest.mark.parametrize("parallel", [False, True])
def test_rope_attention_slots(dev, parallel):
    hd, heads, kv, context = 128, 32, 8, 256
    run_case(dev, hd, heads, kv, context, 100, context - 1, slots=2, nslots=3, parallel=parallel)
    run_case(dev, hd, heads, kv, context, 50, context - 1, slots=5, nslots=3, parallel=parallel)


@pytest.mark.gpu
@pytest.mark.parametrize("parallel", [False, True])
def test_rope_attention_outside_the_prefix(dev, parallel):
    """A position past max_pos but inside the cache is stored and attends
    positions 0 .. max_pos; one at the cache's end (a replayed step whose
    counter reached the end of the context) stores nothing -- both caches
    come out as they went in -- and its query is NaN; in both cases the
    fused kernel agrees with the two calls bit for bit."""
    hd, heads, kv, context = 64, 4, 2, 64
    run_case(dev, hd, heads, kv, context, 40, 30, parallel=parallel)
    q8, sc, qs, kc, vc, kc0, vc0 = run_case(dev, hd, heads, kv, context, context, context - 1, parallel=parallel)
    assert np.array_equal(kc, kc0) and np.array_equal(vc, vc0)


@pytest.mark.gpu
def test_rope_attention_refuses_long_prefix(dev):
    hd, heads, kv, context = 64, 4, 2, 1024
    z = dev.empty((1 << 16,), np.float32)
    with pytest.raises(capi.GxError, match="at most 768"):
        capi.call("gx_qwen_rope_attention", dev.ctx.ptr, capi.vp(z), (heads + 2 * kv) * hd, heads, kv, hd, 800,
                  capi.vp(z), capi.vp(z), capi.vp(z), capi.vp(z), capi.vp(z), np.float32(1e-6), capi.vp(z),
                  capi.vp(z), context, capi.vp(z), capi.vp(z), capi.vp(z), None, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("parallel", [False, True])
@pytest.mark.parametrize("hd,heads,kv,context,M", [(128, 32, 8, 80, 8), (64, 4, 2, 304, 3), (128, 16, 8, 520, 5)])
def test_rope_attention_slots_equal_one_at_a_time(dev, hd, heads, kv, context, M, parallel):
    """gx_qwen_rope_attention_slots: M tokens of M conversations in one call
    (the lock-step step) give, token by token, what the one-token call gives
    for that token alone -- Q8_0 heads and both caches bit for bit."""
    g = synth.rng(400 + M + hd)
    nslots = M + 1
    width = (heads + 2 * kv) * hd
    qkv = (g.standard_normal((M, width)) * 3).astype(np.float32)
    qn = (1 + 0.02 * g.standard_normal(hd)).astype(np.float32)
    kn = (1 + 0.02 * g.standard_normal(hd)).astype(np.float32)
    cos = g.uniform(-1, 1, (context, hd // 2)).astype(np.float32)
    sin = g.uniform(-1, 1, (context, hd // 2)).astype(np.float32)
    kc0 = g.standard_normal((nslots, kv, hd // 8, context, 8)).astype(np.float16)
    vc0 = (g.standard_normal((nslots, kv, hd, context)) * 2).astype(np.float16)
    pos = g.integers(0, context, M).astype(np.int32)
    slots = g.permutation(nslots)[:M].astype(np.int32)  # M different conversations
    max_pos = context - 1
    eps = np.float32(1e-6)
    ins = [dev.put(a) for a in (qkv, pos, qn, kn, cos, sin, slots)]
    kc, vc = dev.put(kc0.view(np.int16)), dev.put(vc0.view(np.int16))
    q8 = dev.empty((M, heads * hd), np.int8)
    sc = dev.empty((M, heads * hd // 32), np.float32)
    qs = dev.empty((M, heads * hd // 32), np.int32)
    capi.call("gx_qwen_rope_attention_slots", dev.ctx.ptr, capi.vp(ins[0]), width, M, heads, kv, hd, max_pos,
              capi.vp(ins[1]), capi.vp(ins[2]), capi.vp(ins[3]), capi.vp(ins[4]), capi.vp(ins[5]), eps, capi.vp(kc),
              capi.vp(vc), context, capi.vp(q8), capi.vp(sc), capi.vp(qs), capi.vp(ins[6]), nslots,
              1 if parallel else 0)
    got = [dev.get(a) for a in (q8, sc, qs, kc, vc)]
    kc1, vc1 = dev.put(kc0.view(np.int16)), dev.put(vc0.view(np.int16))
    name = "gx_qwen_rope_attention_parallel" if parallel else "gx_qwen_rope_attention"
    for t in range(M):
        q1 = dev.empty((1, heads * hd), np.int8)
        s1 = dev.empty((1, heads * hd // 32), np.float32)
        u1 = dev.empty((1, heads * hd // 32), np.int32)
        capi.call(name, dev.ctx.ptr, capi.vp(ins[0][t:t + 1]), width, heads, kv, hd, max_pos, capi.vp(ins[1][t:t + 1]),
                  capi.vp(ins[2]), capi.vp(ins[3]), capi.vp(ins[4]), capi.vp(ins[5]), eps, capi.vp(kc1), capi.vp(vc1),
                  context, capi.vp(q1), capi.vp(s1), capi.vp(u1), capi.vp(ins[6][t:t + 1]), nslots)
        for nm, a, b in (("q", got[0][t], dev.get(q1)[0]), ("scales", got[1][t], dev.get(s1)[0]),
                         ("sums", got[2][t], dev.get(u1)[0])):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"token {t}: {nm}"
    assert np.array_equal(got[3].view(np.uint8), dev.get(kc1).view(np.uint8)), "key cache"
    assert np.array_equal(got[4].view(np.uint8), dev.get(vc1).view(np.uint8)), "value cache"
    with pytest.raises(capi.GxError):
        capi.call("gx_qwen_rope_attention_slots", dev.ctx.ptr, capi.vp(ins[0]), width, M, heads, kv, hd, max_pos,
                  capi.vp(ins[1]), capi.vp(ins[2]), capi.vp(ins[3]), capi.vp(ins[4]), capi.vp(ins[5]), eps,
                  capi.vp(kc), capi.vp(vc), context, capi.vp(q8), capi.vp(sc), capi.vp(qs), None, nslots, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("hd,heads,kv", [(128, 32, 8), (64, 8, 2), (96, 4, 4), (32, 8, 1)])
def test_parallel_extent_independent(dev, hd, heads, kv):
    """The parallel order does not depend on the launch's extent: a token
    launched for its own prefix (max_pos = its position) and for longer
    extents (as a captured decode step, launched for the whole cache, runs
    it) gives the same bits -- the 64-position blocks of the softmax total
    and the 32-position runs of the value sums are fixed, whichever form
    (one key row a thread or two; a 32-element value slice or the whole head
    a workgroup, below 129 positions) the launch takes."""
    context = 640
    for pos in (0, 31, 32, 63, 64, 111, 300, 511):
        own = run_case(dev, hd, heads, kv, context, pos, pos, parallel=True)
        for max_pos in sorted({min(pos + 33, context - 1), 400, context - 1} - {pos}):
            if max_pos < pos:
                continue
            other = run_case(dev, hd, heads, kv, context, pos, max_pos, parallel=True)
            for name, a, b in zip(("q", "scales", "sums", "key cache", "value cache"), own[:5], other[:5]):
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{name}: pos {pos} max_pos {max_pos}"
