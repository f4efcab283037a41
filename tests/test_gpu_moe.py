"""The expert branch of golem's mixture of experts (gemma/moe.go:34-180)
against the oracle.

Selection: router logits bit for bit (golem's x86 DotF32 order, dotF32AVX2) and the
chosen experts identical; the 8th/9th logit margin is logged, as
gemma/moe_reference_test.go:117-136 does for its greedy ties.
Outputs: within 2e-5 of RMS (the benchmark's bar for config 4), for the
per-unit matrix-vector path (few positions) and the expert-grouped MFMA
path (more positions); a position's output is bit-identical in either, the
"batch == one at a time" of gemma/moe_test.go:164-201.
"""
import numpy as np
import pytest

from golem_amd import capi, synth
from tests.gpu_util import log

pytestmark = pytest.mark.gpu

TOL = 2e-5


class Moe:
    def __init__(self, dev, D, F, E, k, seed):
        g = synth.rng(seed)
        self.D, self.F, self.E, self.k = D, F, E, k
        self.gate_up = synth.q4_0_weights(g, E * 2 * F, D)
        self.down = synth.q4_0_weights(g, E * D, F)
        self.router = (g.standard_normal((E, D)) * 0.02).astype(np.float32)
        self.g = g
        self.dev = dev
        self.wgu = dev.weight(self.gate_up, capi.Q4_0, 2 * F, D, count=E)
        self.wdn = dev.weight(self.down, capi.Q4_0, D, F, count=E)
        self.wr = dev.weight(self.router, capi.F32, E, D)

    def expert_bytes(self, stack, rows, cols, e):
        n = rows * (cols // 32) * 18
        return stack[e * n:(e + 1) * n]

    def route(self, x):
        dev = self.dev
        M = x.shape[0]
        xd = dev.put(x)
        logits = dev.empty((M, self.E), np.float32)
        ids = dev.empty((M, self.k), np.int32)
        w = dev.empty((M, self.k), np.float32)
        capi.call("gx_moe_route", dev.ctx.ptr, self.wr.ptr, None, capi.vp(xd), self.D, M, self.k,
                  np.float32(1e-6), capi.vp(logits), capi.vp(ids), capi.vp(w))
        return logits, ids, w

    def experts(self, x, ids, w):
        dev = self.dev
        M = x.shape[0]
        import ctypes
        n = ctypes.c_size_t()
        capi.call("gx_moe_workspace_bytes", M, self.k, self.D, self.F, self.E, ctypes.byref(n))
        ws = dev.empty((n.value + 256,), np.uint8)
        xd = dev.put(x)
        out = dev.full((M, self.D), float("nan"))
        capi.call("gx_moe_experts", dev.ctx.ptr, self.wgu.ptr, self.wdn.ptr, None, capi.vp(xd), self.D, M, self.k,
                  capi.vp(ids), capi.vp(w), capi.vp(out), self.D, capi.vp(ws), n.value)
        return out

    def oracle(self, orc, x, ids, weights):
        """ExpertFFN through the oracle for the given choices."""
        out = np.zeros((x.shape[0], self.D), dtype=np.float32)
        for t in range(x.shape[0]):
            partials = np.stack([orc.expert_unit(self.expert_bytes(self.gate_up, 2 * self.F, self.D, e),
                                                 self.expert_bytes(self.down, self.D, self.F, e), x[t], self.D,
                                                 self.F) for e in ids[t]])
            out[t] = orc.expert_reduce(partials, ids[t], weights[t], self.D)
        return out


def test_gelu_table_matches_oracle_exhaustively(dev, orc):
    got = dev.empty((65536,), np.float32)
    capi.call("gx_gelu_table", dev.ctx.ptr, capi.vp(got))
    got = dev.get(got)
    want = orc.gelu_table_build()
    # every fp16 input that GELUTable can index: finite halves of magnitude < 10
    h = np.arange(65536, dtype=np.uint16)
    v = h.view(np.float16).astype(np.float32)
    used = np.isfinite(v) & (np.abs(v) < 10)
    assert np.array_equal(got[used].view(np.uint32), want[used].view(np.uint32))


@pytest.mark.parametrize("D,E,k,M", [(2816, 128, 8, 6), (512, 16, 4, 3)])
def test_route_bit_exact(dev, orc, D, E, k, M):
    m = Moe.__new__(Moe)
    g = synth.rng(40 + E)
    m.D, m.E, m.k, m.dev = D, E, k, dev
    m.router = (g.standard_normal((E, D)) * 0.02).astype(np.float32)
    m.wr = dev.weight(m.router, capi.F32, E, D)
    x = synth.activations(g, M, D)
    x[1] *= 1e-3
    logits, ids, w = m.route(x)
    logits, ids, w = dev.get(logits), dev.get(ids), dev.get(w)
    for t in range(M):
        ol, oi, ow = orc.route_one(x[t], m.router, k)
        np.testing.assert_array_equal(logits[t].view(np.uint32), ol.view(np.uint32))
        np.testing.assert_array_equal(ids[t], oi)
        np.testing.assert_allclose(w[t], ow, rtol=1e-6, atol=0)
        srt = np.sort(ol)[::-1]
        log(f"position {t}: experts {list(oi)}, k-th/next logit margin {srt[k - 1] - srt[k]:.3g}")


def test_route_ties_go_to_lower_index(dev, orc):
    """TestChooseExpertsIsStableInTies (gemma/moe_test.go:234-244) through the
    device router: two identical router rows give identical logits, and the
    lower index is chosen first."""
    g = synth.rng(5)
    D, E, k = 256, 8, 3
    router = (g.standard_normal((E, D)) * 0.02).astype(np.float32)
    router[5] = router[2]
    router[2] *= 10
    router[5] = router[2]
    m = Moe.__new__(Moe)
    m.D, m.E, m.k, m.dev = D, E, k, dev
    m.router = router
    m.wr = dev.weight(router, capi.F32, E, D)
    x = (router[2] * 100)[None, :].astype(np.float32)  # experts 2 and 5 (equal rows) score highest
    logits, ids, w = m.route(x)
    logits, ids = dev.get(logits)[0], dev.get(ids)[0]
    assert logits[2] == logits[5] and logits[2] > np.delete(logits, [2, 5]).max()
    assert ids[0] == 2 and ids[1] == 5


@pytest.mark.parametrize("D,E,k,M", [(4096, 10, 3, 33), (6144, 6, 2, 5), (6144, 6, 2, 3), (7168, 5, 2, 1),
                                     (8192, 4, 2, 2), (256, 130, 8, 17)])
def test_route_layouts_bit_exact(dev, orc, D, E, k, M):
    """The router's two logits kernels at their edges: one workgroup per
    (expert, position) for up to four positions while the row and input fit
    the LDS (D <= 7168), the streamed kernel otherwise (D = 8192 even at two
    positions); an expert count that is not a multiple of four; positions
    spanning several workgroups."""
    m = Moe.__new__(Moe)
    g = synth.rng(D + E)
    m.D, m.E, m.k, m.dev = D, E, k, dev
    m.router = (g.standard_normal((E, D)) * 0.02).astype(np.float32)
    m.wr = dev.weight(m.router, capi.F32, E, D)
    x = synth.activations(g, M, D)
    logits, ids, w = m.route(x)
    logits, ids, w = dev.get(logits), dev.get(ids), dev.get(w)
    for t in range(M):
        ol, oi, ow = orc.route_one(x[t], m.router, k)
        np.testing.assert_array_equal(logits[t].view(np.uint32), ol.view(np.uint32))
        np.testing.assert_array_equal(ids[t], oi)
        np.testing.assert_allclose(w[t], ow, rtol=1e-6, atol=0)


def test_route_nan_logit_follows_golem_scan(dev, orc):
    """chooseExperts scans in index order and replaces its best only on a
    strictly greater logit, so a NaN logit is chosen exactly when it is the
    first one not yet chosen: expert 0 (NaN) first, then the largest others."""
    D, E, k = 256, 8, 3
    g = synth.rng(8)
    router = (g.standard_normal((E, D)) * 0.02).astype(np.float32)
    router[0, 5] = np.nan
    router[4, 7] = np.nan
    m = Moe.__new__(Moe)
    m.D, m.E, m.k, m.dev = D, E, k, dev
    m.router = router
    m.wr = dev.weight(router, capi.F32, E, D)
    x = synth.activations(g, 2, D)
    logits, ids, w = m.route(x)
    logits, ids, w = dev.get(logits), dev.get(ids), dev.get(w)
    for t in range(2):
        ol, oi, ow = orc.route_one(x[t], router, k)
        assert np.isnan(logits[t, 0]) and np.isnan(logits[t, 4])
        assert oi[0] == 0 and 4 not in oi
        np.testing.assert_array_equal(ids[t], oi)
        assert np.all(np.isnan(w[t])) and np.all(np.isnan(ow))


@pytest.mark.parametrize("M", [1, 2, 20])
def test_experts_against_golem(dev, orc, M):
    """Small shape: the matrix-vector path (M <= 4) and the grouped path."""
    D, F, E, k = 512, 128, 16, 4
    moe = Moe(dev, D, F, E, k, 50)
    x = synth.activations(moe.g, M, D)
    logits, ids, w = moe.route(x)
    out = dev.get(moe.experts(x, ids, w))
    want = moe.oracle(orc, x, dev.get(ids), dev.get(w))
    for t in range(M):
        rel, at = orc.compare_floats(out[t], want[t])
        assert rel <= TOL, f"M={M} position {t}: {rel:.3g} of RMS at {at}"


def test_config4_decode_and_prefill(dev, orc):
    """Config 4's shape (hidden 2816, 128 experts of width 704, top 8): decode
    of one position, and a 40-position batch grouped by expert, each checked
    against golem through the oracle; the batch's positions are
    bit-identical to the same positions alone."""
    D, F, E, k = 2816, 704, 128, 8
    moe = Moe(dev, D, F, E, k, 4)
    M = 40
    x = synth.activations(moe.g, M, D)
    logits, ids, w = moe.route(x)
    log("config 4: routed")
    batch = dev.get(moe.experts(x, ids, w))
    idh, wh = dev.get(ids), dev.get(w)
    want = moe.oracle(orc, x[:3], idh[:3], wh[:3])
    for t in range(3):
        rel, at = orc.compare_floats(batch[t], want[t])
        assert rel <= TOL, f"position {t}: {rel:.3g} of RMS at {at}"
    for t in (0, 7, 39):
        one = dev.get(moe.experts(x[t:t + 1], ids[t:t + 1], w[t:t + 1]))
        np.testing.assert_array_equal(one[0].view(np.uint32), batch[t].view(np.uint32))
    log("config 4: decode and grouped prefill agree")


def test_config4_prefill_256(dev, orc):
    """Config 4's prefill at its configured size: 256 positions, 2048
    (position, slot) units grouped by expert.  Expert ids bit for bit against
    the oracle for every position (with the 8th/9th logit margin logged);
    outputs of sampled positions within 2e-5 of RMS of golem through the
    oracle; and sampled positions bit-identical to the same position run
    alone (moe_test.go:164-205)."""
    D, F, E, k = 2816, 704, 128, 8
    moe = Moe(dev, D, F, E, k, 4)
    M = 256
    x = synth.activations(moe.g, M, D)
    logits, ids, w = moe.route(x)
    idh, wh = dev.get(ids), dev.get(w)
    margins = []
    for t in range(M):
        ol, oi, ow = orc.route_one(x[t], moe.router, k)
        np.testing.assert_array_equal(idh[t], oi, err_msg=f"position {t}")
        srt = np.sort(ol)[::-1]
        margins.append(float(srt[k - 1] - srt[k]))
    log(f"config 4 prefill: ids identical at 256 positions; smallest 8th/9th margin {min(margins):.3g}")
    batch = dev.get(moe.experts(x, ids, w))
    sample = [0, 1, 100, 200, 255]
    want = moe.oracle(orc, x[sample], idh[sample], wh[sample])
    for i, t in enumerate(sample):
        rel, at = orc.compare_floats(batch[t], want[i])
        assert rel <= TOL, f"position {t}: {rel:.3g} of RMS at {at}"
    for t in (0, 128, 255):
        one = dev.get(moe.experts(x[t:t + 1], ids[t:t + 1], w[t:t + 1]))
        np.testing.assert_array_equal(one[0].view(np.uint32), batch[t].view(np.uint32))


def test_bad_expert_id_poisons_its_position(dev):
    D, F, E, k = 256, 64, 4, 2
    moe = Moe(dev, D, F, E, k, 60)
    for M in (1, 6):
        x = synth.activations(moe.g, M, D)
        ids = np.tile(np.array([0, 1], dtype=np.int32), (M, 1))
        ids[0, 1] = 9  # out of range
        w = np.full((M, k), 0.5, dtype=np.float32)
        out = dev.get(moe.experts(x, dev.put(ids), dev.put(w)))
        assert np.all(np.isnan(out[0]))
        assert not np.any(np.isnan(out[1:]))


def _moe_space(M, k, D, F, E):
    """Offsets of the sorted units and the work list in gx_moe_experts'
    workspace (its layout: each region rounded up to 256 bytes)."""
    U = M * k
    max_items = E + (U + 31) // 32
    sizes = [M * D, M * (D // 32) * 4, M * (D // 32) * 4, U * 2 * F * 4, U * F, U * (F // 32) * 4,
             U * (F // 32) * 4, U * D * 4, U * 4, max_items * 16]
    offs, at = [], 0
    for n in sizes:
        offs.append(at)
        at += (n + 255) & ~255
    return offs[8], offs[9], max_items, at


@pytest.mark.parametrize("M,k,E,bad,stride", [
    (256, 8, 128, 0, 0),     # 2,048 units: the one-pass sort, two chunks
    (512, 8, 128, 7, 0),     # 4,096 units, its largest; ids out of range
    (5, 2, 16, 1, 0),        # a ragged first chunk
    (300, 3, 100, 5, 0),     # experts not a power of two
    (40, 1, 1, 0, 0),        # one expert: no id bits to match
    (2000, 1, 8, 0, 0),      # almost every unit in one expert: many items
    (1100, 4, 16, 3, 0),     # 4,400 units: the chunked sort
    (50, 4, 200, 2, 0),      # 200 experts: the chunked sort
    (256, 8, 128, 0, 1),     # a row stride of D + 1: the chunked sort
])
def test_sort_places_units_stably(dev, M, k, E, bad, stride):
    """The units the experts' launch sorts (gemma/moe.go:120-141 runs a
    position's experts in slot order; the grouped product gathers each
    expert's units): sorted[] holds the valid units expert by expert, each
    expert's in unit order (numpy's stable argsort), and work[] each expert's
    items of up to 32 units {expert, first place, count, 0}, then zeros."""
    import ctypes
    D, F = 256, 64
    g = synth.rng(1000 + M + E)
    if k <= E:
        ids = np.stack([g.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
    else:
        ids = g.integers(0, E, (M, k)).astype(np.int32)
    if M == 2000:
        ids[:] = 3
        ids[g.choice(M, 40, replace=False), 0] = g.integers(0, E, 40)
    flat = ids.reshape(-1)
    if bad:
        at = g.choice(flat.size, bad, replace=False)
        flat[at] = np.where(np.arange(bad) % 2 == 0, -1, E)
    gu = synth.q4_0_weights(g, E * 2 * F, D)
    dn = synth.q4_0_weights(g, E * D, F)
    wgu, wdn = dev.weight(gu, capi.Q4_0, 2 * F, D, count=E), dev.weight(dn, capi.Q4_0, D, F, count=E)
    x = synth.activations(g, M, D)
    ld = D + stride
    xs = np.zeros((M, ld), np.float32)
    xs[:, :D] = x
    w = g.uniform(0.05, 0.5, (M, k)).astype(np.float32)
    n = ctypes.c_size_t()
    capi.call("gx_moe_workspace_bytes", M, k, D, F, E, ctypes.byref(n))
    s_off, w_off, max_items, total = _moe_space(M, k, D, F, E)
    assert total == n.value
    ws = dev.full((n.value // 4,), -7, np.int32)
    out = dev.empty((M, D), np.float32)
    xd, idd, wd = dev.put(xs), dev.put(ids), dev.put(w)  # held until the launch has run
    capi.call("gx_moe_experts", dev.ctx.ptr, wgu.ptr, wdn.ptr, None, capi.vp(xd), ld, M, k, capi.vp(idd),
              capi.vp(wd), capi.vp(out), D, capi.vp(ws), n.value)
    wsh = dev.get(ws).view(np.uint8)
    valid = (flat >= 0) & (flat < E)
    want = np.argsort(np.where(valid, flat, E), kind="stable")[:int(valid.sum())].astype(np.int32)
    got = wsh[s_off:s_off + 4 * flat.size].view(np.int32)[:want.size]
    np.testing.assert_array_equal(got, want)
    counts = np.bincount(flat[valid], minlength=E)
    items, place = [], 0
    for e in range(E):
        for f in range(0, counts[e], 32):
            items.append((e, place + f, min(32, counts[e] - f), 0))
        place += counts[e]
    want_w = np.zeros((max_items, 4), np.int32)
    want_w[:len(items)] = items
    np.testing.assert_array_equal(wsh[w_off:w_off + 16 * max_items].view(np.int32).reshape(max_items, 4), want_w)
    wgu.free()
    wdn.free()
    log(f"sort: M={M} k={k} E={E} ({flat.size} units, {bad} out of range, stride D+{stride}) stable, "
        f"{len(items)} items")


def test_sort_forms_agree(dev):
    """The grouped path sorts the units by expert in one of two forms: one
    pass inside the launch that quantises the input (at most 4,096 units over
    at most 128 experts, the input whole float4s), or the three-phase sort
    after a quantising launch (more units, more experts, or a row stride not
    a multiple of four).  A position's output does not depend on which ran:
    1,100 positions x 4 (4,400 units: three-phase) against the same positions
    in halves of 550 (2,200 units: one pass); the halves read through a row
    stride of D + 1 (three-phase); and with 200 experts (three-phase at any
    size) sampled positions against the same position alone."""
    D, F, k = 256, 64, 4

    def draw(moe, M):
        ids = np.stack([moe.g.choice(moe.E, k, replace=False) for _ in range(M)]).astype(np.int32)
        w = moe.g.uniform(0.05, 0.5, (M, k)).astype(np.float32)
        return ids, w

    moe = Moe(dev, D, F, 16, k, 70)
    M = 1100
    x = synth.activations(moe.g, M, D)
    ids, w = draw(moe, M)
    whole = dev.get(moe.experts(x, dev.put(ids), dev.put(w)))
    assert not np.any(np.isnan(whole))
    for h in (slice(0, 550), slice(550, 1100)):
        half = dev.get(moe.experts(x[h], dev.put(ids[h]), dev.put(w[h])))
        np.testing.assert_array_equal(half.view(np.uint32), whole[h].view(np.uint32), err_msg=f"half {h}")
        # the same half read with a row stride of D + 1
        import ctypes
        Mh = half.shape[0]
        xs = np.zeros((Mh, D + 1), np.float32)
        xs[:, :D] = x[h]
        n = ctypes.c_size_t()
        capi.call("gx_moe_workspace_bytes", Mh, k, D, F, moe.E, ctypes.byref(n))
        ws = dev.empty((n.value,), np.uint8)
        xd, idd, wd = dev.put(xs), dev.put(ids[h]), dev.put(w[h])
        out = dev.full((Mh, D), float("nan"))
        capi.call("gx_moe_experts", dev.ctx.ptr, moe.wgu.ptr, moe.wdn.ptr, None, capi.vp(xd), D + 1, Mh, k,
                  capi.vp(idd), capi.vp(wd), capi.vp(out), D, capi.vp(ws), n.value)
        np.testing.assert_array_equal(dev.get(out).view(np.uint32), whole[h].view(np.uint32),
                                      err_msg=f"half {h}, stride D + 1")
    log("sort forms: 4,400 units (three-phase) == two halves of 2,200 (one pass) == strided halves")

    moe = Moe(dev, D, F, 200, k, 71)
    M = 300
    x = synth.activations(moe.g, M, D)
    ids, w = draw(moe, M)
    batch = dev.get(moe.experts(x, dev.put(ids), dev.put(w)))
    for t in (0, 1, 150, 299):
        one = dev.get(moe.experts(x[t:t + 1], dev.put(ids[t:t + 1]), dev.put(w[t:t + 1])))
        np.testing.assert_array_equal(one[0].view(np.uint32), batch[t].view(np.uint32), err_msg=f"position {t}")


@pytest.mark.parametrize("M,spread", [(2, 128), (40, 128), (40, 8)])
def test_expert_integers_bit_exact(dev, orc, M, spread):
    """The expert products' per-block integers (gx_moe_block_dots) at config
    4's shape, from the kernels gx_moe_experts runs: the fused
    matrix-vector kernels for 2 positions, the grouped int8-MFMA product for
    40 (experts drawn from all 128, and from only 8 so that an expert's 40
    units span several 32-unit items).  gate|up against the Q8_0 of each
    position's input, down against a given Q8_0 input, each equal to golem's
    accumulator less 8 * sum(q) (nn/dot_q4_0.go:58-63), for every unit of 2
    positions and a sample of the 320 units."""
    import ctypes
    from oracle import Batch
    D, F, E, k = 2816, 704, 128, 8
    moe = Moe(dev, D, F, E, k, 4)
    x = synth.activations(moe.g, M, D)
    pool = moe.g.choice(E, spread, replace=False)
    ids = np.stack([moe.g.choice(pool, k, replace=False) for _ in range(M)]).astype(np.int32)
    mid = synth.activations(moe.g, M * k, F)
    mb = Batch(mid).quantize()
    dgu = dev.empty((M * k, 2 * F, D // 32), np.int32)
    ddn = dev.empty((M * k, D, F // 32), np.int32)
    mq, ms, mqs = dev.put(mb.q_rows()), dev.put(mb.scales_rows()), dev.put(mb.qsum_rows())
    xd, idd = dev.put(x), dev.put(ids)  # held until the kernels have read them
    n = ctypes.c_size_t()
    capi.call("gx_moe_workspace_bytes", M, k, D, F, E, ctypes.byref(n))
    ws = dev.empty((n.value,), np.uint8)
    capi.call("gx_moe_block_dots", dev.ctx.ptr, moe.wgu.ptr, moe.wdn.ptr, capi.vp(xd), D, M, k, capi.vp(idd),
              capi.vp(mq), capi.vp(ms), capi.vp(mqs), capi.vp(ws), n.value, capi.vp(dgu), capi.vp(ddn))
    dgu, ddn = dev.get(dgu), dev.get(ddn)
    units = range(M * k) if M * k <= 16 else sorted(set(synth.rng(M).choice(M * k, 20, replace=False)) | {0, M * k - 1})
    for u in units:
        t, e = u // k, int(ids[u // k, u % k])
        xb = Batch(x[t:t + 1]).quantize()
        acc = orc.q4_0_block_acc(moe.expert_bytes(moe.gate_up, 2 * F, D, e), xb, 2 * F)[0]
        np.testing.assert_array_equal(dgu[u], acc - 8 * xb.qsum_rows()[0][None, :], err_msg=f"gate_up unit {u}")
        ub = Batch(mid[u:u + 1]).quantize()
        acc = orc.q4_0_block_acc(moe.expert_bytes(moe.down, D, F, e), ub, D)[0]
        np.testing.assert_array_equal(ddn[u], acc - 8 * ub.qsum_rows()[0][None, :], err_msg=f"down unit {u}")


def test_route_few_positions_repeats(dev, orc):
    """The few-position router (at most four positions: a workgroup per
    logit, then the choice): consecutive calls of 1..4 positions, each bit
    for bit against the oracle."""
    D, E, k = 2816, 128, 8
    m = Moe.__new__(Moe)
    g = synth.rng(77)
    m.D, m.E, m.k, m.dev = D, E, k, dev
    m.router = (g.standard_normal((E, D)) * 0.02).astype(np.float32)
    m.wr = dev.weight(m.router, capi.F32, E, D)
    for M in (1, 4, 2, 3, 1, 1, 4):
        x = synth.activations(g, M, D)
        logits, ids, w = m.route(x)
        logits, ids, w = dev.get(logits), dev.get(ids), dev.get(w)
        for t in range(M):
            ol, oi, ow = orc.route_one(x[t], m.router, k)
            np.testing.assert_array_equal(logits[t].view(np.uint32), ol.view(np.uint32))
            np.testing.assert_array_equal(ids[t], oi)
            np.testing.assert_allclose(w[t], ow, rtol=1e-6, atol=0)


def test_decode_graph_replays_match_eager(dev, orc):
    """Config 4's decode (route + experts, four launches) captured once into
    a HIP graph and replayed on new inputs, with eager work and
    synchronisations between the replays: every replay's output bit-identical
    to the eager call's, which is within 2e-5 of RMS of golem."""
    import ctypes
    import torch
    D, F, E, k = 2816, 704, 128, 8
    moe = Moe(dev, D, F, E, k, 4)
    n = ctypes.c_size_t()
    capi.call("gx_moe_workspace_bytes", 1, k, D, F, E, ctypes.byref(n))
    ws = dev.empty((n.value,), np.uint8)
    xs = dev.empty((1, D), np.float32)
    logits = dev.empty((1, E), np.float32)
    ids = dev.empty((1, k), np.int32)
    w = dev.empty((1, k), np.float32)
    out = dev.empty((1, D), np.float32)

    def step():
        capi.call("gx_moe_route", dev.ctx.ptr, moe.wr.ptr, None, capi.vp(xs), D, 1, k, np.float32(1e-6),
                  capi.vp(logits), capi.vp(ids), capi.vp(w))
        capi.call("gx_moe_experts", dev.ctx.ptr, moe.wgu.ptr, moe.wdn.ptr, None, capi.vp(xs), D, 1, k,
                  capi.vp(ids), capi.vp(w), capi.vp(out), D, capi.vp(ws), n.value)

    inputs = [synth.activations(moe.g, 1, D) for _ in range(4)]
    eager = []
    for x in inputs:
        xs.copy_(dev.put(x))
        step()
        eager.append((dev.get(ids).copy(), dev.get(out).copy()))
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    capi.call("gx_set_stream", dev.ctx.ptr, ctypes.c_void_p(stream.cuda_stream))
    try:
        with torch.cuda.graph(graph, stream=stream):
            step()
    finally:
        capi.call("gx_set_stream", dev.ctx.ptr, None)
    torch.cuda.synchronize()
    for rep in range(2):
        for i, x in enumerate(inputs):
            xs.copy_(dev.put(x))
            graph.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(dev.get(ids), eager[i][0])
            np.testing.assert_array_equal(dev.get(out).view(np.uint32), eager[i][1].view(np.uint32))
            # eager work between replays
            step()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(dev.get(out).view(np.uint32), eager[i][1].view(np.uint32))
    ol, oi, ow = orc.route_one(inputs[0][0], moe.router, k)
    np.testing.assert_array_equal(eager[0][0][0], oi)
    want = moe.oracle(orc, inputs[0], oi[None, :], ow[None, :])
    rel, at = orc.compare_floats(eager[0][1][0], want[0])
    assert rel <= TOL, f"{rel:.3g} of RMS at {at}"
    del graph


@pytest.mark.parametrize("M", [1, 3, 9])
def test_f32_expert_stacks_bit_exact(dev, orc, M):
    """F32 expert stacks (golem's ExpertStack takes any nn.Quant,
    gemma/weights.go:59-72; its own MoE oracle test runs on F32 stacks,
    gemma/moe_test.go:36-42): the input and mid enter the DotF32 products
    unquantised (nn/matrix.go:113-120), GELUTable * up between them, the
    weighted sum with DownScale -- bit for bit against the oracle's unit and
    reduction (oracle.expert_unit with quant F32, pinned on golem's dense
    oracle in test_oracle_composition).  An out-of-range id makes only its
    position NaN; stacks of two formats are refused."""
    D, F, E, k = 512, 128, 16, 4
    g = synth.rng(70 + M)
    gu = (g.standard_normal((E, 2 * F, D)) * 0.05).astype(np.float32)
    dn = (g.standard_normal((E, D, F)) * 0.05).astype(np.float32)
    wgu = dev.weight(gu, capi.F32, 2 * F, D, count=E)
    wdn = dev.weight(dn, capi.F32, D, F, count=E)
    ds = (1 + 0.1 * g.standard_normal(E)).astype(np.float32)
    x = (g.standard_normal((M, D)) * 2).astype(np.float32)
    ids = np.stack([g.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
    if M > 1:
        ids[1, 2] = E + 5  # out of range: position 1 is NaN, the others are not touched
    w = g.random((M, k)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    import ctypes
    n = ctypes.c_size_t()
    capi.call("gx_moe_workspace_bytes", M, k, D, F, E, ctypes.byref(n))
    ws = dev.empty((n.value + 256,), np.uint8)
    out = dev.full((M, D), float("nan"))
    dsd, xd, idd, wd = dev.put(ds), dev.put(x), dev.put(ids), dev.put(w)  # held until the calls are done
    capi.call("gx_moe_experts", dev.ctx.ptr, wgu.ptr, wdn.ptr, capi.vp(dsd), capi.vp(xd), D, M, k, capi.vp(idd),
              capi.vp(wd), capi.vp(out), D, capi.vp(ws), n.value)
    got = dev.get(out)
    for t in range(M):
        if M > 1 and t == 1:
            assert np.all(np.isnan(got[t]))
            continue
        parts = np.stack([orc.expert_unit(gu[e], dn[e], x[t], D, F, quant=orc.F32)
                          for e in ids[t]])
        want = orc.expert_reduce(parts, ids[t], w[t], D, down_scale=ds)
        np.testing.assert_array_equal(got[t].view(np.uint32), want.view(np.uint32))
    mixed = dev.weight(synth.q4_0_weights(g, E * D, F), capi.Q4_0, D, F, count=E)
    with pytest.raises(capi.GxError):
        capi.call("gx_moe_experts", dev.ctx.ptr, wgu.ptr, mixed.ptr, None, capi.vp(xd), D, M, k, capi.vp(idd),
                  capi.vp(wd), capi.vp(out), D, capi.vp(ws), n.value)
