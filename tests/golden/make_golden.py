"""Writes hot_path_slices.npz: small slices of the benchmark configurations
with the oracle's outputs, frozen as data so that a change to the oracle or
to the device path shows up against fixed vectors.

golem's own quant fixtures (testdata/gemma/quants) are absent from the
reference, so these vectors come from this project's oracle (the C
restatement of golem's engine, oracle/oracle.c), whose functions are
pinned by golem's known answers and by closed forms in
tests/test_oracle_*.py.  Inputs are drawn exactly as bench.py draws configs
0, 1 and 4 (golem_amd/synth.py), then cut:

  c0  the first 64 rows of config 0's Q4_0 matrix (9728 x 2560, seed 0) and
      its activation: Q8_0 form, golem's per-block accumulators, y
  c1  the first 64 rows of config 1's Q6_K head (151936 x 2560, seed 1) and
      its activation: Q8_K form, per-superblock integers, y
  c4  a router of 128 experts over 256 inputs (seed 4): logits in golem's
      x86 DotF32 order (dotF32AVX2), the top 8
      and their weights (Route / chooseExperts)

Run from the repository root: python tests/golden/make_golden.py"""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "..", ".."))
import oracle  # noqa: E402
from golem_amd import synth  # noqa: E402

OUT = os.path.join(os.path.dirname(__file__), "hot_path_slices.npz")
ROWS = 64


def main():
    out = {}
    g0 = synth.rng(0)
    w0 = synth.q4_0_weights(g0, 9728, 2560)
    x0 = synth.activations(g0, 1, 2560)
    w0s = w0[:ROWS * 80 * 18].copy()
    b0 = oracle.Batch(x0).quantize()
    out.update(c0_w=w0s, c0_x=x0, c0_q=b0.q_rows(), c0_scales=b0.scales_rows(), c0_corr=b0.corr_rows(),
               c0_acc=oracle.q4_0_block_acc(w0s, b0, ROWS), c0_y=oracle.mat_vec_q4_0_rows(w0s, b0, ROWS))
    del w0
    g1 = synth.rng(1)
    w1 = synth.q6_k_weights(g1, 151936, 2560)
    x1 = synth.activations(g1, 1, 2560)
    w1s = w1[:ROWS * 10 * 210].copy()
    del w1
    b1 = oracle.Batch(x1).quantize_k()
    out.update(c1_w=w1s, c1_x=x1, c1_qk=b1.QK.copy(), c1_kscales=b1.KScales.copy(), c1_bsums=b1.BSums.copy(),
               c1_isum=oracle.q6_k_block_isum(w1s, b1, ROWS), c1_y=oracle.mat_vec_q6_k_rows(w1s, b1, ROWS))
    g4 = synth.rng(4)
    router = (g4.standard_normal((128, 256)) * 0.02).astype(np.float32)
    tok = g4.standard_normal(256).astype(np.float32)
    logits, ids, weights = oracle.route_one(tok, router, 8)
    out.update(c4_router=router, c4_x=tok, c4_logits=logits, c4_ids=ids, c4_weights=weights)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: " + ", ".join(f"{k} {v.shape} {v.dtype}" for k, v in out.items()))


if __name__ == "__main__":
    main()
