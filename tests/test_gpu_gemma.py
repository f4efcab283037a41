"""Gemma's mixture feed-forward half (moeHalf, gemma/block.go:146-206) on the
device (golem_amd.gemma.MoEHalf) against the oracle's restatement of it
(oracle/gemma.py), on a small block of the same structure.

- the routing (ids) is identical and the branches and the block output are
  within 1e-4 of RMS of golem's: the products differ from golem's by float
  rounding, and Q8_0 / the GELU table's fp16 index can move one step;
- golem's TestMoEHalfAddsBothBranches (gemma/moe_test.go:273-322): both
  branches contribute, they differ, and the output is exactly resid +
  RMSNormPlain(shared + experts, post_ffw_norm) of the device's own branch
  buffers;
- a batch equals its positions one at a time, bit for bit (products, experts
  and join all per position in one order, whatever the batch).
"""
import numpy as np
import pytest
import torch

from golem_amd import capi, synth
from golem_amd.gemma import MoEConfig, MoEHalf, moe_weights
from tests.gpu_util import log

pytestmark = pytest.mark.gpu

CFG = MoEConfig(256, 512, 16, 4, 64)


def _setup(dev, seed, M):
    g = synth.rng(seed)
    w = moe_weights(CFG, g)
    resid = synth.activations(g, M, CFG.dim)
    return w, resid, MoEHalf(dev.ctx, CFG, w, max_batch=16)


@pytest.mark.parametrize("M", [1, 3, 9])
def test_moe_half_against_golem(dev, orc, M):
    from oracle.gemma import moe_half
    w, resid, blk = _setup(dev, 40 + M, M)
    log(f"moe half M={M}")
    r = torch.from_numpy(resid).cuda()
    out = torch.empty_like(r)
    blk.forward(r, out)
    want, shared, experts, ids, wts = moe_half(CFG, w, resid)
    np.testing.assert_array_equal(dev.get(blk.ids[:M]), ids)
    rel_w = float(np.max(np.abs(dev.get(blk.weights[:M]) - wts)))
    log(f"  routing weights max diff {rel_w:.3g}")
    assert rel_w <= 1e-6
    for name, got, exp in (("shared", blk.shared[:M], shared), ("experts", blk.experts_out[:M], experts),
                           ("out", out, want)):
        got = dev.get(got)
        rels = [orc.compare_floats(got[t], exp[t])[0] for t in range(M)]
        log(f"  {name}: {[float('%.2g' % x) for x in rels]} of RMS")
        assert max(rels) <= 1e-4, f"{name}: {max(rels):.3g} of RMS"
    blk.free()


def test_moe_half_adds_both_branches(dev, orc):
    w, resid, blk = _setup(dev, 50, 1)
    r = torch.from_numpy(resid).cuda()
    out = torch.empty_like(r)
    blk.forward(r, out)
    shared, experts, got = dev.get(blk.shared[:1])[0], dev.get(blk.experts_out[:1])[0], dev.get(out)[0]
    assert np.any(shared != 0), "the shared expert contributed nothing"
    assert np.any(experts != 0), "the expert branch contributed nothing"
    assert not np.array_equal(shared, experts), "one branch is reading the other's buffer"
    combined = orc.rms_norm_plain(shared + experts, w["post_ffw_norm"], np.float32(CFG.eps))
    np.testing.assert_array_equal(got.view(np.uint32), (resid[0] + combined).astype(np.float32).view(np.uint32))
    blk.free()


def test_moe_half_batch_equals_one_at_a_time(dev):
    M = 9
    w, resid, blk = _setup(dev, 60, M)
    r = torch.from_numpy(resid).cuda()
    out = torch.empty_like(r)
    blk.forward(r, out)
    batch = dev.get(out)
    for t in range(M):
        one = torch.empty_like(r[t:t + 1])
        blk.forward(r[t:t + 1].clone(), one)
        np.testing.assert_array_equal(dev.get(one)[0].view(np.uint32), batch[t].view(np.uint32))
    # out may be the residual itself
    blk.forward(r, r)
    np.testing.assert_array_equal(dev.get(r).view(np.uint32), batch.view(np.uint32))
    blk.free()


def test_join_refuses_one_buffer_for_both_branches(dev):
    x = torch.zeros((1, 64), dtype=torch.float32, device="cuda")
    g = torch.ones(64, dtype=torch.float32, device="cuda")
    vp = capi.vp
    with pytest.raises(capi.GxError, match="separate buffers"):
        capi.call("gx_moe_join", dev.ctx.ptr, vp(x), 64, vp(x), 64, vp(x), 64, vp(g), vp(g), vp(g), 1, 64,
                  np.float32(1e-6), vp(x), 64)
