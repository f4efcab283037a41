"""Several conversations over one set of weights (golem's qwen/slots.go and
qwen/place.go): SetSlots / UseSlot / ForwardSlots and LogitsBatch on the
device, against the same conversations run alone.

golem's tests, restated on a small model of Qwen3's structure:
- TestMixedBatchAgreesWithOneAtATime (qwen/place_test.go:8-50): the last
  tokens of two conversations drawn together out of two slots are, bit for
  bit, what each gives alone;
- TestSlotsAreIndependent (qwen/slots_test.go:8-44): a slot continuing its
  conversation after another slot wrote a different one gives what one cache
  alone gives;
- TestSetSlotsRefusesAContextItCannotCut (qwen/slots_test.go:46-54);
- TestLogitsBatchAgreesWithOneAtATime (qwen/place_test.go:52-68).
And the server's use of them (cmd/golem-server/runner.go:233-297): several
conversations decoded in lock step, one product per weight matrix per step,
draw each conversation's own greedy tokens.
"""
import numpy as np
import pytest
import torch

from golem_amd import capi, synth
from golem_amd.qwen import QwenModel
from tests.gpu_util import log

pytestmark = pytest.mark.gpu

CFG = synth.QwenConfig(256, 512, 2, 4, 2, 64, 1024, 48)


def _model(dev, seed=81):
    w = synth.qwen_weights(CFG, seed, symmetric=True)
    return w, QwenModel(dev.ctx, CFG, w, max_batch=16)


def _prompts():
    mine = [int(t) for t in synth.rng(82).integers(0, CFG.vocab, 9)]
    return mine, mine[::-1]


def _bits(x):
    return x.cpu().numpy().view(np.uint32)


def test_mixed_batch_agrees_with_one_at_a_time(dev):
    w, solo = _model(dev)
    mine, theirs = _prompts()
    last = len(mine) - 1
    solo.reset()
    solo.forward(mine[:last], 0)
    want_mine = _bits(solo.forward(mine[last:], last)[0])
    solo.reset()
    solo.forward(theirs[:last], 0)
    want_theirs = _bits(solo.forward(theirs[last:], last)[0])

    m = QwenModel(dev.ctx, CFG, w, max_batch=16)
    m.set_slots(2)
    assert (m.nslots, m.slot_context) == (2, 24)
    m.use_slot(0)
    m.forward(mine[:last], 0)
    m.use_slot(1)
    m.forward(theirs[:last], 0)
    got = m.forward_slots([mine[last], theirs[last]], [0, 1], [last, last])
    np.testing.assert_array_equal(_bits(got[0]), want_mine)
    np.testing.assert_array_equal(_bits(got[1]), want_theirs)
    solo.free()
    m.free()


def test_slots_are_independent(dev):
    w, solo = _model(dev)
    mine, theirs = _prompts()
    nxt = mine[0]
    solo.reset()
    solo.forward(mine, 0)
    want = _bits(solo.forward([nxt], len(mine))[0])
    m = QwenModel(dev.ctx, CFG, w, max_batch=16)
    m.set_slots(2)
    m.use_slot(0)
    m.forward(mine, 0)
    m.use_slot(1)
    m.forward(theirs, 0)
    m.use_slot(0)
    np.testing.assert_array_equal(_bits(m.forward([nxt], len(mine))[0]), want)
    solo.free()
    m.free()


def test_set_slots_refuses_a_context_it_cannot_cut(dev):
    _, m = _model(dev)
    with pytest.raises(ValueError, match="0 slots"):
        m.set_slots(0)
    with pytest.raises(ValueError, match="leaves no position each"):
        m.set_slots(CFG.max_context + 1)
    m.set_slots(3)
    with pytest.raises(IndexError):
        m.use_slot(3)
    with pytest.raises(ValueError, match="past a slot"):
        m.forward_slots([1], [0], [m.slot_context])
    m.free()


def test_logits_batch_agrees_with_one_at_a_time(dev):
    _, m = _model(dev)
    mine, _ = _prompts()
    m.reset()
    m.forward(mine, 0)
    first = _bits(m.logits(0).clone())
    second = _bits(m.logits(len(mine) - 1).clone())
    together = m.logits_batch([0, len(mine) - 1])
    np.testing.assert_array_equal(_bits(together[0]), first)
    np.testing.assert_array_equal(_bits(together[1]), second)
    m.free()


@pytest.mark.parametrize("nconv", [3, 6])
def test_lock_step_decode_draws_each_conversations_tokens(dev, nconv):
    """nconv conversations (prompts of different lengths) decoded together,
    one forward_slots + one head read per step: each draws the greedy tokens
    it draws alone (6 conversations: the attention's per-token path at M > 4
    and the products' 4- and 2-column forms)."""
    cfg = synth.QwenConfig(256, 512, 2, 4, 2, 64, 1024, 16 * nconv)  # 16 positions a conversation
    w = synth.qwen_weights(cfg, 81, symmetric=True)
    solo = QwenModel(dev.ctx, cfg, w, max_batch=16)
    g = synth.rng(90 + nconv)
    prompts = [[int(t) for t in g.integers(0, cfg.vocab, 3 + i)] for i in range(nconv)]
    steps = 5
    want = [solo.greedy(p, steps) for p in prompts]
    m = QwenModel(dev.ctx, cfg, w, max_batch=16)
    m.set_slots(nconv)
    toks = []
    for i, p in enumerate(prompts):
        m.use_slot(i)
        m.forward(p, 0)
        toks.append(int(m.next_token(len(p) - 1).item()))
    got = [[t] for t in toks]
    pos = [len(p) for p in prompts]
    for _ in range(steps - 1):
        m.forward_slots(toks, list(range(nconv)), pos)
        toks = [int(t) for t in m.next_tokens(range(nconv)).cpu().tolist()]
        for i in range(nconv):
            got[i].append(toks[i])
        pos = [p + 1 for p in pos]
    log(f"  {nconv} conversations: {got}")
    assert got == want
    # the same steps from the device's own tokens and positions (slots_step)
    for i, p in enumerate(prompts):
        m.use_slot(i)
        m.forward(p, 0)
    m.start_slots([w_[0] for w_ in want], [len(p) for p in prompts])
    steps_dev = [m.slots_step(nconv).cpu().tolist() for _ in range(steps - 1)]
    assert [[w_[0]] + [s_[i] for s_ in steps_dev] for i, w_ in enumerate(want)] == want
    solo.free()
    m.free()


@pytest.mark.parametrize("nconv", [3, 6, 8])
def test_lock_step_hidden_states_equal_each_alone(dev, nconv):
    """Every step of a lock-step batch gives each conversation, bit for bit,
    the hidden state the same conversation gets run alone on the device with
    the same tokens (qwen/model_test.go:78's batch-equals-one-at-a-time, per
    slot): the products give each column its one-column result and the
    attention's order does not depend on the launch, so a token routed to
    another slot's cache or position, or a column crossed with another,
    shows as a difference in the bits."""
    cfg = synth.QwenConfig(256, 512, 2, 4, 2, 64, 1024, 16 * nconv)
    w = synth.qwen_weights(cfg, 85, symmetric=True)
    g = synth.rng(290 + nconv)
    prompts = [[int(t) for t in g.integers(0, cfg.vocab, 2 + (5 * i) % 9)] for i in range(nconv)]
    steps = 5
    m = QwenModel(dev.ctx, cfg, w, max_batch=16)
    m.set_slots(nconv)
    toks = []
    for i, p in enumerate(prompts):
        m.use_slot(i)
        m.forward(p, 0)
        toks.append(int(m.next_token(len(p) - 1).item()))
    fed = [[t] for t in toks]
    pos = [len(p) for p in prompts]
    hidden = []
    for _ in range(steps):
        hidden.append(_bits(m.forward_slots(toks, list(range(nconv)), pos)))
        toks = [int(t) for t in m.next_tokens(range(nconv)).cpu().tolist()]
        for i in range(nconv):
            fed[i].append(toks[i])
        pos = [p + 1 for p in pos]
    m.free()
    solo = QwenModel(dev.ctx, cfg, w, max_batch=16)
    for i, p in enumerate(prompts):
        solo.reset()
        solo.forward(p, 0)
        for s in range(steps):
            want = _bits(solo.forward([fed[i][s]], len(p) + s)[0])
            np.testing.assert_array_equal(hidden[s][i], want, err_msg=f"conversation {i}, step {s}")
    log(f"  {nconv} conversations: every step's hidden states bit for bit those run alone")
    solo.free()


@pytest.mark.parametrize("nconv", [3, 6])
def test_captured_slot_steps_match_eager(dev, nconv):
    """slots_step as replays of its captured form (capture_slots): the ids
    after every step, and at the end every cache and the hidden states, bit
    for bit those of the eager steps.  An eager step launches the attention
    for its own longest prefix, the captured one for the whole slot; each
    token stops at its own prefix and the parallel attention's value runs
    are fixed, so the two agree.  (A small random model repeats its ids; the
    caches, which hold every step's keys and values, and the hidden states
    carry the check.)  Each replay is followed by eager work (the check) and
    a synchronisation."""
    cfg = synth.QwenConfig(256, 512, 2, 4, 2, 64, 1024, 16 * nconv)
    w = synth.qwen_weights(cfg, 83, symmetric=False)
    m = QwenModel(dev.ctx, cfg, w, max_batch=16)
    m.set_slots(nconv)
    g = synth.rng(95 + nconv)
    prompts = [[int(t) for t in g.integers(0, cfg.vocab, 2 + i)] for i in range(nconv)]
    steps = 6

    def seed():
        m.reset()
        toks = []
        for i, p in enumerate(prompts):
            m.use_slot(i)
            m.forward(p, 0)
            toks.append(int(m.next_token(len(p) - 1).item()))
        m.start_slots(toks, [len(p) for p in prompts])

    seed()
    eager = [m.slots_step(nconv).cpu().tolist() for _ in range(steps)]
    kc = [k.clone() for k in m.kc]
    vc = [v.clone() for v in m.vc]
    hidden = m.hidden[:nconv].clone()
    seed()
    got = []
    for _ in range(steps):
        got.append(m.slots_step(nconv, graph=True).cpu().tolist())
        torch.cuda.synchronize()
    log(f"  {nconv} conversations, captured steps: {got}")
    assert got == eager
    for layer in range(cfg.layers):
        assert torch.equal(kc[layer], m.kc[layer]) and torch.equal(vc[layer], m.vc[layer]), f"layer {layer}"
    assert torch.equal(hidden.view(torch.int32), m.hidden[:nconv].view(torch.int32))
    m.free()


def test_a_slot_out_of_range_stores_nothing(dev):
    """gx_qwen_qk_rope with a token in no conversation: nothing lands in any
    cache, and its query heads are NaN."""
    heads, kv, hd, ctx_len, M = 4, 2, 64, 16, 2
    width = (heads + 2 * kv) * hd
    g = synth.rng(95)
    qkv = dev.put(g.standard_normal((M, width)).astype(np.float32))
    pos = dev.put(np.array([3, 5], np.int32))
    slots = dev.put(np.array([1, 7], np.int32))
    gains = dev.put(np.ones(hd, np.float32))
    cos = dev.put(np.ones((ctx_len, hd // 2), np.float32))
    sin = dev.put(np.zeros((ctx_len, hd // 2), np.float32))
    qh = torch.zeros((M, heads * hd), dtype=torch.int16, device="cuda")
    kc = torch.zeros((2, kv, hd // 8, ctx_len, 8), dtype=torch.int16, device="cuda")
    vc = torch.zeros((2, kv, hd, ctx_len), dtype=torch.int16, device="cuda")
    vp = capi.vp
    capi.call("gx_qwen_qk_rope", dev.ctx.ptr, vp(qkv), width, M, heads, kv, hd, vp(pos), vp(gains), vp(gains),
              vp(cos), vp(sin), np.float32(1e-6), vp(qh), vp(kc), vp(vc), ctx_len, vp(slots), 2)
    q = qh.cpu().numpy()
    assert np.all(q[1] == 0x7E00) and not np.any(q[0] == 0x7E00)
    kcn, vcn = kc.cpu().numpy(), vc.cpu().numpy()
    assert not np.any(kcn[0]) and not np.any(vcn[0]), "slot 0 was written"
    assert np.any(kcn[1][:, :, 3, :]) and np.any(vcn[1][:, :, 3]), "token 0's key and value are missing"
    assert not np.any(kcn[1][:, :, 5, :]) and not np.any(vcn[1][:, :, 5]), "the stray token was stored"


@pytest.mark.parametrize("nconv", [3, 6])
def test_slots_against_golem(dev, orc, nconv):
    """Each conversation of a lock-step batch against golem's engine run alone
    on that conversation (oracle/qwen.py): at every step its hidden state
    within 5e-2 of RMS (the bar of the one-conversation tests, test_gpu_qwen)
    and its greedy ids identical -- qwen/place_test.go:8-50 checked against
    golem rather than against this build's own single-conversation path."""
    from oracle.qwen import QwenOracle
    loose = 5e-2
    cfg = synth.QwenConfig(256, 512, 2, 4, 2, 64, 1024, 16 * nconv)  # 16 positions a conversation
    w = synth.qwen_weights(cfg, 83, symmetric=True)
    om = QwenOracle(cfg, w)
    g = synth.rng(190 + nconv)
    prompts = [[int(t) for t in g.integers(0, cfg.vocab, 3 + i)] for i in range(nconv)]
    steps = 5
    want = [om.greedy(p, steps)[0] for p in prompts]
    m = QwenModel(dev.ctx, cfg, w, max_batch=16)
    m.set_slots(nconv)
    seqs, toks, worst = [], [], 0.0
    for i, p in enumerate(prompts):
        m.use_slot(i)
        got = dev.get(m.forward(p, 0))[-1].copy()
        om.reset()
        rel = orc.compare_floats(got, om.forward(p, 0)[-1])[0]
        assert rel <= loose, f"conversation {i} prompt: {rel:.3g} of RMS"
        worst = max(worst, rel)
        toks.append(int(m.next_token(len(p) - 1).item()))
        seqs.append(list(p) + [toks[-1]])
    pos = [len(p) for p in prompts]
    for _ in range(steps - 1):
        hidden = dev.get(m.forward_slots(toks, list(range(nconv)), pos)).copy()
        for i in range(nconv):
            om.reset()
            rel = orc.compare_floats(hidden[i], om.forward(seqs[i], 0)[-1])[0]
            assert rel <= loose, f"conversation {i} at position {pos[i]}: {rel:.3g} of RMS"
            worst = max(worst, rel)
        toks = [int(t) for t in m.next_tokens(range(nconv)).cpu().tolist()]
        for i in range(nconv):
            seqs[i].append(toks[i])
        pos = [p + 1 for p in pos]
    got_ids = [s[len(p):] for s, p in zip(seqs, prompts)]
    log(f"  {nconv} conversations against golem: hidden within {worst:.2g} of RMS; ids {got_ids}")
    assert got_ids == want
    m.free()
