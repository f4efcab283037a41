"""gx_moe_experts_noalloc -- the mixture-of-experts entry point that
allocates nothing (its scratch is a static device array the library holds)
-- against gx_moe_experts with a caller's workspace, bit for bit, on two
calls in a row, the second with fewer positions: config 4's shape (hidden
2816, 128 experts of 704, top 8), 40 positions (the expert-grouped MFMA
path) then 3 (the per-unit matrix-vector path).  A call too large for the
scratch is refused with an error before any work is queued."""
import numpy as np
import pytest

from golem_amd import capi, synth
from tests.gpu_util import log
from tests.test_gpu_moe import Moe

pytestmark = pytest.mark.gpu


def noalloc(dev, moe, x, ids, w):
    M = x.shape[0]
    xd = dev.put(x)
    out = dev.full((M, moe.D), float("nan"))
    capi.call("gx_moe_experts_noalloc", dev.ctx.ptr, moe.wgu.ptr, moe.wdn.ptr, None, capi.vp(xd), moe.D, M, moe.k,
              capi.vp(ids), capi.vp(w), capi.vp(out), moe.D)
    return out


def test_noalloc_matches_the_workspace_form(dev):
    D, F, E, k = 2816, 704, 128, 8
    moe = Moe(dev, D, F, E, k, 44)
    for M in (40, 3):
        x = synth.activations(moe.g, M, D)
        logits, ids, w = moe.route(x)
        want = dev.get(moe.experts(x, ids, w))
        got = dev.get(noalloc(dev, moe, x, ids, w))
        log(f"no-alloc MoE, M={M}: {int(np.isnan(got).sum())} NaN")
        assert not np.isnan(got).any()
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_refuses_more_than_its_scratch(dev):
    D, F, E, k = 2816, 704, 128, 8
    moe = Moe(dev, D, F, E, k, 45)
    M = 256  # about 35 MB of workspace at this shape: more than the 16 MiB scratch
    x = dev.empty((M, D), np.float32)
    ids = dev.empty((M, k), np.int32)
    w = dev.empty((M, k), np.float32)
    out = dev.empty((M, D), np.float32)
    with pytest.raises(capi.GxError, match="bytes of scratch"):
        capi.call("gx_moe_experts_noalloc", dev.ctx.ptr, moe.wgu.ptr, moe.wdn.ptr, None, capi.vp(x), D, M, k,
                  capi.vp(ids), capi.vp(w), capi.vp(out), D)
