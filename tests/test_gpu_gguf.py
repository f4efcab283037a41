"""A Qwen3 checkpoint read from a GGUF file (golem_amd.gguf.load_qwen, golem's
qwen.LoadConfig + LoadWeights over tensors.OpenGGUF) drives the device model
exactly as the same weights handed over in memory do, and a pure Q4_0 file's
tied Q4_0 head (Logits over the Q8_0 form, qwen/model.go:181-194) decodes
golem's greedy tokens.

No real checkpoint exists on the box (golem's own file tests skip without
GOLEM_MODEL, tensors/gguf_test.go:9-21); the files are written by
tests/gguf_writer.py from the synthetic weights.
"""
import numpy as np
import pytest

from golem_amd import capi, gguf, synth
from golem_amd.qwen import QwenModel
from tests import gguf_writer as gw
from tests.gpu_util import log

pytestmark = pytest.mark.gpu

CFG = synth.QwenConfig(256, 512, 2, 4, 2, 64, 1024, 48)


def test_model_from_gguf_equals_model_from_memory(dev, tmp_path):
    w = synth.qwen_weights(CFG, 31, symmetric=True)
    path = gw.qwen_file(tmp_path / "q.gguf", CFG, w)
    g, cfg, fw = gguf.load_qwen(path, CFG.max_context)
    try:
        from_file = QwenModel(dev.ctx, cfg, fw, max_batch=16)
    finally:
        g.close()  # the model holds device copies; the mapping can go
    from_memory = QwenModel(dev.ctx, CFG, w, max_batch=16)
    prompt = [int(t) for t in synth.rng(32).integers(0, CFG.vocab, 10)]
    log(f"gguf model: prefill {len(prompt)}, greedy 6")
    for m in (from_file, from_memory):
        m.reset()
    a = dev.get(from_file.forward(prompt, 0))
    b = dev.get(from_memory.forward(prompt, 0))
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    assert from_file.greedy(prompt, 6) == from_memory.greedy(prompt, 6)
    from_file.free()
    from_memory.free()


@pytest.mark.parametrize("symmetric", [False, True])
def test_q4_0_tied_head_against_golem(dev, orc, tmp_path, symmetric):
    from oracle.qwen import QwenOracle
    w = synth.qwen_weights(CFG, 33, symmetric=symmetric)
    w["token_embd"] = synth.q4_0_weights(synth.rng(34), CFG.vocab, CFG.dim, symmetric=symmetric)
    w["token_embd_quant"] = capi.Q4_0
    path = gw.qwen_file(tmp_path / "pure.gguf", CFG, w)
    g, cfg, fw = gguf.load_qwen(path, CFG.max_context)
    try:
        assert fw["token_embd_quant"] == capi.Q4_0
        model = QwenModel(dev.ctx, cfg, fw, max_batch=16)
    finally:
        g.close()
    oracle_model = QwenOracle(CFG, w)  # the same bytes, held in memory
    prompt = [int(t) for t in synth.rng(35).integers(0, CFG.vocab, 12)]
    log(f"pure Q4_0 gguf symmetric={symmetric}: prefill {len(prompt)}")
    oracle_model.reset()
    want = oracle_model.forward(prompt, 0)
    model.reset()
    got = dev.get(model.forward(prompt, 0))
    rels = [orc.compare_floats(got[t], want[t])[0] for t in range(len(prompt))]
    log(f"  hidden, of RMS per position: {[float('%.2g' % r) for r in rels]}")
    assert max(rels) <= 5e-2
    lg = dev.get(model.logits(len(prompt) - 1))
    rel, at = orc.compare_floats(lg, oracle_model.logits(want[-1]))
    log(f"  last logits {rel:.3g} of RMS")
    assert rel <= 0.25, f"logits: {rel:.3g} of RMS at {at}"
    ids, margins = oracle_model.greedy(prompt, 6)
    got_ids = model.greedy(prompt, 6)
    log(f"  greedy {got_ids} (golem {ids}); margins {np.round(margins, 3).tolist()}")
    assert got_ids == ids
    # the captured decode step reads the Q4_0 head the same way
    assert model.greedy(prompt, 6, graph=True) == ids
    model.free()
