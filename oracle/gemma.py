"""The oracle's restatement of Gemma's mixture feed-forward half: moeHalf
(gemma/block.go:146-206) over the oracle's primitives, position by position.
Test infrastructure only: the device path never calls it.

  shared  = Down . Q8_0(GELUTable(Gate . normed) * (Up . normed))      block.go:163-176
  exp_in  = RMSNormPlain(resid, pre_ffw_norm_2)                         block.go:178-186
  experts = ExpertFFN(exp_in): Route(resid), units, Axpy sum            moe.go:112-180
  shared  = RMSNormPlain(shared, post_ffw_norm_1)                       block.go:195-205
  experts = RMSNormPlain(experts, post_ffw_norm_2)
  out     = resid + RMSNormPlain(shared + experts, post_ffw_norm)

The products are golem's Matrix.rows over Q8_0 batches (matrix_rows), the
router in DotF32's x86 (dotF32AVX2) order (route_one), the expert units and their
sum orc_expert_unit / orc_expert_reduce.
"""
import numpy as np

from . import (Batch, Q4_0, expert_reduce, expert_unit, gelu_table, matrix_rows, rms_norm_plain, route_one)


def moe_half(cfg, w, resid, normed=None):
    """resid [M][dim] float32; normed: a quantised Batch of RMSNormPlain(resid,
    ffn_norm) (computed here when None).  Returns (out, shared, experts, ids,
    weights) with shared / experts post-normed, as golem's buffers hold them."""
    D, F, E, FE, k = cfg.dim, cfg.ffn, cfg.experts, cfg.expert_ffn, cfg.used
    resid = np.asarray(resid, np.float32)
    M = resid.shape[0]
    if normed is None:
        normed = Batch(np.stack([rms_norm_plain(r, w["ffn_norm"], cfg.eps) for r in resid])).quantize()
    gate = matrix_rows(Q4_0, w["gate"], F, D, normed)
    up = matrix_rows(Q4_0, w["up"], F, D, normed)
    mid = np.stack([gelu_table(gate[t]) * up[t] for t in range(M)]).astype(np.float32)
    shared = matrix_rows(Q4_0, w["down"], D, F, Batch(mid).quantize())
    gu_row = 2 * FE * (D // 32) * 18
    dn_row = D * (FE // 32) * 18
    experts = np.zeros((M, D), np.float32)
    all_ids = np.zeros((M, k), np.int32)
    all_w = np.zeros((M, k), np.float32)
    for t in range(M):
        exp_in = rms_norm_plain(resid[t], w["pre_ffw_norm_2"], cfg.eps)
        _, ids, wts = route_one(resid[t], w["router"], k, cfg.eps, w["router_scale"])
        parts = np.stack([expert_unit(w["gate_up_exps"][e * gu_row:(e + 1) * gu_row],
                                      w["down_exps"][e * dn_row:(e + 1) * dn_row], exp_in, D, FE) for e in ids])
        experts[t] = expert_reduce(parts, ids, wts, D, w["down_scale"])
        all_ids[t], all_w[t] = ids, wts
    out = np.zeros((M, D), np.float32)
    for t in range(M):
        shared[t] = rms_norm_plain(shared[t], w["post_ffw_norm_1"], cfg.eps)
        experts[t] = rms_norm_plain(experts[t], w["post_ffw_norm_2"], cfg.eps)
        combined = rms_norm_plain(shared[t] + experts[t], w["post_ffw_norm"], cfg.eps)
        out[t] = resid[t] + combined
    return out, shared, experts, all_ids, all_w
