"""The CPU baseline (oracle/cpu_avx2.c: golem's AVX2 kernels and worker pool)
against the generic restatement, on the bars golem's own tests set:

- Q6_K: the AVX2 kernel is bit-identical to dotQ6_KGo (nn/dot_q6_k_test.go:51-75).
- Q4_0: x1, x4 and x8 agree with dotQ4_0Go within 1e-3 relative + 1e-6
  (nn/dot_q4_0_avx2_test.go:14-79); a row cut into two stretches gives exactly
  the row done in one call (:81-130).  x1, x4 and x8 also agree with each other
  bit for bit: the same per-column instructions, which golem relies on when a
  batch finishes on the narrower kernels (nn/dot_q4_0.go:156-160).
- The pool: any thread count gives the same bits (rows are independent; the
  split never cuts a row).
"""
import numpy as np
import pytest

import oracle
from golem_amd import synth

pytestmark = pytest.mark.skipif(not oracle.host_has_avx2(), reason="no AVX2/FMA/F16C on this host")

BEGIN, FINISH = 1, 2


def portable(orc, w, b, column, n):
    state = np.zeros(9, dtype=np.float32)
    lib = orc.load()
    lib.orc_dot_q4_0_go(orc._p(w), orc._p(b.Q), orc._p(b.Scales), orc._p(b.Corr), b.stride, 0, column, n,
                        orc._p(state))
    return np.float32(lib.orc_fold(orc._p(state), np.float32(state[8])))


def golem_like_rows(g, n):
    """A row as golem's AVX2 test draws it: random bytes, scale bytes kept to
    sane fp16 magnitudes (high byte 0x30..0x33)."""
    blocks = n // 32
    w = g.integers(0, 256, size=blocks * 18, dtype=np.uint8)
    w[0::18] = g.integers(0, 256, size=blocks, dtype=np.uint8)
    w[1::18] = 0x30 + g.integers(0, 4, size=blocks, dtype=np.uint8)
    return w


@pytest.mark.parametrize("n", [32, 64, 256, 1536, 4096])
@pytest.mark.parametrize("size", [1, 3, 4, 7, 8, 11, 16])
def test_q4_0_kernels_against_portable(n, size):
    g = synth.rng(7 + n + size)
    w = golem_like_rows(g, n)
    F = (g.random((size, n), dtype=np.float32) * 2 - 1).astype(np.float32)
    b = oracle.Batch(F).quantize()
    want = np.array([portable(oracle, w, b, c, n) for c in range(size)], dtype=np.float32)

    def bar(got, c):
        assert abs(float(got) - float(want[c])) <= 1e-3 * abs(float(want[c])) + 1e-6, (n, size, c, got, want[c])

    one = np.zeros(size, dtype=np.float32)
    for c in range(size):
        st = np.zeros(72, dtype=np.float32)
        oracle.cpu_dot_q4_0(w, b, 0, c, n, st, BEGIN | FINISH, 1)
        one[c] = st[0]
        bar(st[0], c)
    for cols in (4, 8):
        for c in range(0, size - cols + 1, cols):
            st = np.zeros(72, dtype=np.float32)
            oracle.cpu_dot_q4_0(w, b, 0, c, n, st, BEGIN | FINISH, cols)
            for j in range(cols):
                bar(st[j], c + j)
            np.testing.assert_array_equal(st[:cols].view(np.uint32), one[c:c + cols].view(np.uint32))
            if n >= 64 and (n // 2) % 32 == 0:
                half = n // 2
                split = np.zeros(72, dtype=np.float32)
                oracle.cpu_dot_q4_0(w, b, 0, c, half, split, BEGIN, cols)
                oracle.cpu_dot_q4_0(w[half // 32 * 18:], b, half // 32, c, n - half, split, FINISH, cols)
                np.testing.assert_array_equal(split[:cols].view(np.uint32), st[:cols].view(np.uint32))


@pytest.mark.parametrize("rows,cols,size", [(64, 2560, 1), (37, 3840, 3), (21, 512, 13)])
def test_q4_0_mat_vec_tiled(rows, cols, size):
    """matVecQ4_0Rows' stretches of 2048 and row tiles (K=2560 and 3840 take
    the tiled branch, 3840 with a partial last stretch), against the generic
    product, and independent of the thread count."""
    g = synth.rng(rows + cols)
    w = synth.q4_0_weights(g, rows, cols)
    b = oracle.Batch(synth.activations(g, size, cols)).quantize()
    want = oracle.mat_vec_q4_0_rows(w, b, rows)
    got1 = oracle.cpu_mat_vec_q4_0(w, b, rows, 1)
    gotn = oracle.cpu_mat_vec_q4_0(w, b, rows, oracle.host_threads())
    np.testing.assert_array_equal(got1.view(np.uint32), gotn.view(np.uint32))
    for c in range(size):
        rel, at = oracle.compare_floats(got1[c], want[c])
        assert rel <= 1e-3, (c, rel, at)


@pytest.mark.parametrize("rows,cols,size", [(300, 2560, 1), (40, 512, 3)])
def test_q6_k_bit_exact_against_portable(rows, cols, size):
    g = synth.rng(cols + size)
    w = synth.q6_k_weights(g, rows, cols)
    x = synth.activations(g, size, cols)
    x[0, :256] = 0.0                        # a zero superblock
    b = oracle.Batch(x).quantize_k()
    want = oracle.mat_vec_q6_k_rows(w, b, rows)
    for threads in (1, oracle.host_threads()):
        got = oracle.cpu_mat_vec_q6_k(w, b, rows, threads)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q6_k_extreme_scales():
    """Sub-scales at -64 and 63 and magnitudes at 0 and 63: the int16 pair sums
    of VPMADDUBSW stay in range and the result stays bit-exact."""
    g = synth.rng(99)
    rows, cols = 8, 512
    w = synth.q6_k_weights(g, rows, cols).reshape(rows * 2, 210)
    w[0::2, 192:208] = np.uint8(0xC0)       # -64
    w[1::2, 192:208] = np.uint8(63)
    w[:4, :192] = 0xFF                       # magnitude 63 everywhere
    w[4:8, :192] = 0x00                      # magnitude 0
    w = w.reshape(-1)
    x = np.full((1, cols), -1.0, dtype=np.float32)
    x[0, ::3] = 1.0
    b = oracle.Batch(x).quantize_k()
    np.testing.assert_array_equal(oracle.cpu_mat_vec_q6_k(w, b, rows, 1).view(np.uint32),
                                  oracle.mat_vec_q6_k_rows(w, b, rows).view(np.uint32))


@pytest.mark.parametrize("rows,cols,size", [(64, 2560, 7), (40, 4096, 4), (16, 9728, 5)])
def test_packed_q4_0_against_portable(rows, cols, size):
    """The packed x4/x1 kernels (dotPackedQ4_0x4AVX2 and dotPackedQ4_0AVX2
    restated) against dotPackedQ4_0Go through matVecPackedQ4_0Rows (the
    oracle): golem states they agree to rounding, not to the bit
    (nn/pack_q4_0.go:128-133), so within 1e-5 of RMS per column; a batch's
    column is bit-identical to the same column alone (the x1 kernel is the x4
    kernel for one column) and to any thread count.  Sizes cover columns past
    the last group of four and rows past one 2048-input tile (K_TILE)."""
    g = synth.rng(rows + cols + size)
    w = np.concatenate([golem_like_rows(g, cols) for _ in range(rows)])
    packed = oracle.pack_q4_0(w, rows, cols)
    b = oracle.Batch(synth.activations(g, size, cols)).quantize()
    threads = oracle.host_threads()
    oracle.cpu_lib(threads)
    got = oracle.cpu_mat_vec_packed_q4_0(packed, b, rows, threads)
    want = oracle.mat_vec_packed_q4_0_rows(packed, b, rows)
    for c in range(size):
        rel, at = oracle.compare_floats(got[c], want[c])
        assert rel <= 1e-5, f"column {c}: {rel:.3g} of RMS at {at}"
    one = oracle.cpu_mat_vec_packed_q4_0(packed, b, rows, 1)
    np.testing.assert_array_equal(got.view(np.uint32), one.view(np.uint32))
    for c in (0, size - 1):
        bc = oracle.Batch(b.F[c:c + 1]).quantize()
        alone = oracle.cpu_mat_vec_packed_q4_0(packed, bc, rows, threads)
        np.testing.assert_array_equal(alone[0].view(np.uint32), got[c].view(np.uint32))


def test_moe_ffn_against_portable():
    """Route + ExpertFFN through golem's x86 kernels (the CPU baseline of
    config 4) against the oracle's generic restatement: the same experts
    and routing weights bit for bit (both route through DotF32's x86 order,
    dotF32AVX2), and the output within 1e-3 of RMS (golem's own
    AVX2-against-Go bar, dot_q4_0_avx2_test.go:68)."""
    D, F, E, k, batch = 256, 64, 16, 4, 3
    g = synth.rng(440)
    router = (g.standard_normal((E, D)) * 0.02).astype(np.float32)
    gate_up = synth.q4_0_weights(g, E * 2 * F, D)
    down = synth.q4_0_weights(g, E * D, F)
    resid = synth.activations(g, batch, D)
    moe = oracle.CpuMoE(router, gate_up, down, D, F, E, k, batch)
    out, ids, wts = moe.run(resid, 2)
    gu_b, dn_b = 2 * F * (D // 32) * 18, D * (F // 32) * 18
    for t in range(batch):
        _, want_ids, want_w = oracle.route_one(resid[t], router, k)
        assert list(ids[t]) == list(want_ids), (t, ids[t], want_ids)
        np.testing.assert_array_equal(np.asarray(wts[t]).view(np.uint32), np.asarray(want_w).view(np.uint32))
        parts = [oracle.expert_unit(gate_up[i * gu_b:(i + 1) * gu_b], down[i * dn_b:(i + 1) * dn_b], resid[t], D, F)
                 for i in want_ids]
        want = oracle.expert_reduce(np.stack(parts), want_ids, want_w, D)
        rel, at = oracle.compare_floats(out[t], want)
        assert rel <= 1e-3, f"position {t}: {rel:.3g} of RMS at {at}"
    # every thread count gives the same bits (the sections' splits change nothing)
    one, _, _ = moe.run(resid, 1)
    one = one.copy()
    many, _, _ = moe.run(resid, 8)
    np.testing.assert_array_equal(one.view(np.uint32), many.view(np.uint32))


def test_qwen_token_against_portable():
    """golem's Qwen3 decode token through its x86 kernels (the CPU baseline of
    config 3) against the oracle's generic restatement of the engine, fed the
    same caches: the hidden state after the final norm within 1e-3 of RMS
    (golem's AVX2-against-Go bar; DotF32's and Axpy's orders differ) and the
    logits' greedy id equal; two thread counts give the same bits."""
    import math
    from oracle.qwen import QwenOracle
    cfg = synth.QwenConfig(256, 512, 2, 4, 2, 64, 1024, 16)
    w = synth.qwen_weights(cfg, 450, symmetric=True)
    om = QwenOracle(cfg, w)
    prompt = [int(t) for t in synth.rng(451).integers(0, cfg.vocab, 6)]
    om.reset()
    om.forward(prompt, 0)
    cpu = oracle.CpuQwen(cfg, w)
    for L, (kc, vc) in enumerate(cpu.caches):
        kc[:] = om.K[L]
        vc[:] = om.V[L]
    tok, pos = 17, len(prompt)
    lib = oracle.load()
    cos, sin = np.zeros(cfg.head_dim // 2, np.float32), np.zeros(cfg.head_dim // 2, np.float32)
    lib.orc_rope_prepare(cfg.head_dim, pos, cfg.rope_base, oracle._p(cos), oracle._p(sin))
    x = om.embed(tok).astype(np.float32).copy()
    logits = cpu.token(x, pos, cos, sin, 2).copy()
    want = om.forward([tok], pos)[0]
    rel, at = oracle.compare_floats(x, want)
    assert rel <= 1e-3, f"hidden state {rel:.3g} of RMS at {at}"
    want_logits = om.logits(want)
    assert int(np.argmax(logits)) == int(np.argmax(want_logits))
    # the caches hold the position's key and value as golem stores them
    for L, (kc, vc) in enumerate(cpu.caches):
        assert oracle.compare_floats(kc[pos], om.K[L][pos])[0] <= 1e-3
    x2 = om.embed(tok).astype(np.float32).copy()
    cpu.token(x2, pos, cos, sin, 8)
    np.testing.assert_array_equal(x.view(np.uint32), x2.view(np.uint32))
    assert math.isfinite(float(logits.max()))


@pytest.mark.parametrize("n", [1, 7, 8, 9, 31, 32, 33, 40, 64, 100, 703, 704, 2816, 4099])
def test_dot_f32_avx2_order_against_the_instructions(n):
    """orc_dot_f32_avx2 (the router's DotF32, restated as scalar C in
    dotF32AVX2's order) against the AVX2 instructions themselves
    (cpu_avx2.c: VMULPS / VADDPS in the kernel's register order): bit for
    bit, every length class -- whole groups of 32, eights, a tail."""
    g = synth.rng(460 + n)
    a = (g.standard_normal(n) * 3).astype(np.float32)
    b = (g.standard_normal(n) * 0.02).astype(np.float32)
    want = np.float32(oracle.cpu_lib().cpu_dot_f32(oracle._p(a), oracle._p(b), n))
    got = np.float32(oracle.dot_f32_avx2(a, b))
    assert got.view(np.uint32) == want.view(np.uint32), (n, got, want)
