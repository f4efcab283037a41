"""The feed-forward half of a Gemma mixture block on the device: golem's
moeHalf (gemma/block.go:146-206) around the expert products.

Two branches leave the same residual.  The dense one (the shared expert) is
the ordinary GELU-gated feed forward under ffn_norm: Gate and Up in one Q4_0
product (their rows stacked, gates first), GELUTable(gate) * up to Q8_0, then
Down.  The expert one normalises the residual under pre_ffw_norm_2, routes
the residual (Route, gemma/moe.go:34-97) and runs the chosen experts
(ExpertFFN, gemma/moe.go:112-180).  The join post-normalises each branch
(post_ffw_norm_1, post_ffw_norm_2), adds them, normalises the sum under
post_ffw_norm and adds it to the residual.

Per step on the device, M positions:
  gx_matmul_q4_0  (Gate|Up)           normed Q8_0 -> gu [M][2*ffn]
  gx_geglu_quant                        gu -> Q8_0 of GELUTable(gate) * up
  gx_matmul_q4_0  (Down)              -> shared [M][dim]
  gx_norm_quant   (pre_ffw_norm_2)    resid -> the experts' input
  gx_moe_route    (router, scale)     resid -> ids, weights
  gx_moe_experts  (stacks, scales)    -> experts [M][dim]
  gx_moe_join     (three post-norms)  -> out = resid + post_ffw_norm(...)
"""

import numpy as np
import torch

from . import capi


class MoEConfig:
    """A Gemma mixture block's feed-forward geometry (gemma/config.go:
    Dim, Blocks[i].FFN, Experts, ExpertsUsed, ExpertFFN, Eps)."""

    def __init__(self, dim, ffn, experts, used, expert_ffn, eps=1e-6):
        self.dim, self.ffn, self.experts, self.used, self.expert_ffn = dim, ffn, experts, used, expert_ffn
        self.eps = eps


def moe_weights(cfg, g):
    """Random weights of the block's feed-forward half, as config 4 draws
    them: Q4_0 matrices as in config 0, the router fp32 N(0, 0.02), norms
    and scales 1 + N(0, 0.05).  A dict of numpy arrays."""
    from . import synth

    def gains(n):
        return (1.0 + 0.05 * g.standard_normal(n)).astype(np.float32)

    D, F, E, FE = cfg.dim, cfg.ffn, cfg.experts, cfg.expert_ffn
    return {
        "ffn_norm": gains(D),
        "gate": synth.q4_0_weights(g, F, D), "up": synth.q4_0_weights(g, F, D), "down": synth.q4_0_weights(g, D, F),
        "router": (0.02 * g.standard_normal((E, D))).astype(np.float32), "router_scale": gains(D),
        "pre_ffw_norm_2": gains(D), "post_ffw_norm": gains(D), "post_ffw_norm_1": gains(D),
        "post_ffw_norm_2": gains(D),
        "gate_up_exps": synth.q4_0_weights(g, E * 2 * FE, D), "down_exps": synth.q4_0_weights(g, E * D, FE),
        "down_scale": gains(E),
    }


class MoEHalf:
    def __init__(self, ctx, cfg, w, max_batch):
        self.ctx, self.cfg, self.max_batch = ctx, cfg, max_batch
        D, F, E, FE = cfg.dim, cfg.ffn, cfg.experts, cfg.expert_ffn

        def dev(a):
            return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()

        self.gate_up = capi.Weight(ctx, np.concatenate([w["gate"], w["up"]]), capi.Q4_0, 2 * F, D)
        self.down = capi.Weight(ctx, w["down"], capi.Q4_0, D, F)
        self.router = capi.Weight(ctx, w["router"], capi.F32, E, D)
        self.gate_up_exps = capi.Weight(ctx, w["gate_up_exps"], capi.Q4_0, 2 * FE, D, count=E)
        self.down_exps = capi.Weight(ctx, w["down_exps"], capi.Q4_0, D, FE, count=E)
        for k in ("ffn_norm", "router_scale", "pre_ffw_norm_2", "post_ffw_norm", "post_ffw_norm_1",
                  "post_ffw_norm_2", "down_scale"):
            setattr(self, k, dev(w[k]))
        M = max_batch

        def q8(K):
            return (torch.empty((M, K), dtype=torch.int8, device="cuda"),
                    torch.empty((M, K // 32), dtype=torch.float32, device="cuda"),
                    torch.empty((M, K // 32), dtype=torch.int32, device="cuda"))

        self.normed = q8(D)
        self.mid = q8(F)
        self.gu = torch.empty((M, 2 * F), dtype=torch.float32, device="cuda")
        self.shared = torch.empty((M, D), dtype=torch.float32, device="cuda")
        self.exp_in = torch.empty((M, D), dtype=torch.float32, device="cuda")
        self.experts_out = torch.empty((M, D), dtype=torch.float32, device="cuda")
        self.logits = torch.empty((M, E), dtype=torch.float32, device="cuda")
        self.ids = torch.empty((M, cfg.used), dtype=torch.int32, device="cuda")
        self.weights = torch.empty((M, cfg.used), dtype=torch.float32, device="cuda")
        n = capi.size_out("gx_moe_workspace_bytes", M, cfg.used, D, FE, E)
        self.ws = torch.empty(((n + 255) // 256 * 256,), dtype=torch.uint8, device="cuda")

    def forward(self, resid, out, normed=None):
        """moeHalf for the M = resid.shape[0] positions of resid [M][dim]
        (device): out [M][dim] (may be resid) receives resid + the joined
        branches.  normed: the Q8_0 (q, scales, qsum) of RMSNormPlain(resid,
        ffn_norm) when the caller has it (golem's Block computes it); else it
        is computed here.  Afterwards self.shared / self.experts_out hold the
        post-normed branches (golem's MoEShared / MoEExperts)."""
        cfg, vp, call, ctx = self.cfg, capi.vp, capi.call, self.ctx.ptr
        M, D, F = int(resid.shape[0]), cfg.dim, cfg.ffn
        if M > self.max_batch:
            raise ValueError(f"gemma: {M} positions exceed the batch {self.max_batch}")
        eps = np.float32(cfg.eps)
        if normed is None:
            nq, ns, nqs = self.normed
            call("gx_norm_quant", ctx, vp(resid), D, None, D, vp(self.ffn_norm), M, D, eps, None, 0, vp(nq), vp(ns),
                 vp(nqs))
            normed = (nq, ns, nqs)
        nq, ns, nqs = normed
        # the shared expert: the dense feed forward (block.go:163-176)
        call("gx_matmul_q4_0", ctx, self.gate_up.ptr, vp(nq), vp(ns), vp(nqs), None, M, 0, 2 * F, None,
             vp(self.gu), 2 * F)
        mq, ms, mqs = self.mid
        call("gx_geglu_quant", ctx, vp(self.gu), 2 * F, M, F, vp(mq), vp(ms), vp(mqs))
        call("gx_matmul_q4_0", ctx, self.down.ptr, vp(mq), vp(ms), vp(mqs), None, M, 0, D, None, vp(self.shared), D)
        # the experts, from the same residual under their own norm (block.go:178-188)
        call("gx_norm_quant", ctx, vp(resid), D, None, D, vp(self.pre_ffw_norm_2), M, D, eps, vp(self.exp_in), D,
             None, None, None)
        call("gx_moe_route", ctx, self.router.ptr, vp(self.router_scale), vp(resid), D, M, cfg.used, eps,
             vp(self.logits), vp(self.ids), vp(self.weights))
        call("gx_moe_experts", ctx, self.gate_up_exps.ptr, self.down_exps.ptr, vp(self.down_scale), vp(self.exp_in),
             D, M, cfg.used, vp(self.ids), vp(self.weights), vp(self.experts_out), D, vp(self.ws), self.ws.numel())
        # the join (block.go:190-205)
        call("gx_moe_join", ctx, vp(self.shared), D, vp(self.experts_out), D, vp(resid), D, vp(self.post_ffw_norm_1),
             vp(self.post_ffw_norm_2), vp(self.post_ffw_norm), M, D, eps, vp(out), D)
        return out

    def free(self):
        for w in (self.gate_up, self.down, self.router, self.gate_up_exps, self.down_exps):
            w.free()
