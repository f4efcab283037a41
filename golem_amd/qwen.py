"""golem's Qwen3 dense decoder (qwen/) with every step on the device.

qwen.Model.ForwardBatch (qwen/model.go:127-175) for M consecutive positions:
the embedding rows (TokenEmbd.Row, a Q6_K dequantisation), then per block
(qwen/block.go:32-102):

    gx_norm_quant      x += previous FFN output; RMSNormPlain(attn_norm); Q8_0
    gx_qwen_qkv_rope   Q, K and V, stacked by rows into one Q4_0 matrix, then
                       head norms, RoPE, fp16 query, fp16 cache entries (for
                       a batch in the product's epilogue: gx_matmul_q4_0 +
                       gx_qwen_qk_rope bit for bit)
    gx_qwen_attention  scores, softmax, values; Q8_0 of the heads
    gx_matmul_q4_0     O
    gx_norm_quant      x += attention; RMSNormPlain(ffn_norm); Q8_0
    gx_matmul_q4_0     Gate and Up, stacked with rows interleaved by 32
    gx_swiglu_quant    silu(gate) * up; Q8_0
    gx_matmul_q4_0     Down

and the final norm (the last block's residual folded in).  Logits
(qwen/model.go:181-194) is QuantizeK plus the tied Q6_K head; greedy picks the
largest logit, the lower id on ties.  Stacking Q/K/V and Gate/Up changes no
result: every output row is its own product.

One position (a decode step) takes fewer launches: each pre-norm runs inside
the product after it (gx_norm_matmul_q4_0 for Q|K|V), and the FFN's norm,
Gate|Up product, SwiGLU and Q8_0 are one kernel (gx_norm_swiglu_q4_0), and
the head norms, RoPE, cache store and attention are one kernel
(gx_qwen_rope_attention), the same values bit for bit.

Every kernel treats a position on its own, so a prompt read in one batch
gives, bit for bit, what the same tokens give one at a time (golem's
TestBatchAgreesWithOneAtATime, qwen/model_test.go:79).

A decode step (one position) can be captured once into a HIP graph and
replayed: the token and its position are read from the device (the previous
step's argmax and a device counter), and the attention is launched for the
whole cache (max_pos = context - 1; the kernels stop at each position's own
prefix), so every replay runs the same launches.  A replay computes exactly
what the eager step computes.
"""
import ctypes
import math

import numpy as np
import torch

from . import capi

# gx_qwen_rope_attention reads at most this many cached positions (the
# one-kernel decode attention's limit); longer prefixes take the two calls.
FUSED_ATTENTION_MAX = 767


def rope_tables(dims, context, base):
    """RoPETable.Prepare (nn/rope.go:33-59) for positions 0 .. context-1:
    theta = pos * base^(-2i/dims) in float64, cos and sin rounded to float32,
    through the C library's pow, cos and sin."""
    half = dims // 2
    cos = np.empty((context, half), np.float32)
    sin = np.empty((context, half), np.float32)
    freqs = [math.pow(base, -2 * float(i) / float(dims)) for i in range(half)]
    for p in range(context):
        for i in range(half):
            theta = float(p) * freqs[i]
            cos[p, i] = math.cos(theta)
            sin[p, i] = math.sin(theta)
    return cos, sin


def interleave_rows(gate, up, rows, cols):
    """Gate and Up (Q4_0, rows x cols each) stacked into one matrix with
    their rows interleaved by 32: 32 gate rows, the same 32 up rows, and so
    on.  A 64-row tile then holds both halves of 32 SwiGLU outputs."""
    rb = cols // 32 * 18
    g = np.asarray(gate, np.uint8).reshape(rows // 32, 32 * rb)
    u = np.asarray(up, np.uint8).reshape(rows // 32, 32 * rb)
    return np.ascontiguousarray(np.concatenate([g, u], axis=1)).reshape(-1)


class _Q8:
    """A Q8_0 batch on the device: q [M][K], scales and qsum [M][K/32]."""

    def __init__(self, M, K):
        self.q = torch.empty((M, K), dtype=torch.int8, device="cuda")
        self.s = torch.empty((M, K // 32), dtype=torch.float32, device="cuda")
        self.qs = torch.empty((M, K // 32), dtype=torch.int32, device="cuda")


class QwenModel:
    """attention: "parallel" runs decode steps' attention with its softmax
    total and value sums in a parallel order (gx_qwen_rope_attention_parallel
    / gx_qwen_attention_parallel) and prompts (more than four positions) on
    the matrix cores: golem's values within float rounding, so a prompt read
    in one batch and the same tokens read one at a time agree only to that
    rounding.  "golem" keeps golem's serial order bit for bit, and with it
    golem's batch == one at a time."""

    def __init__(self, ctx, cfg, weights, max_batch, attention="parallel"):
        if attention not in ("parallel", "golem"):
            raise ValueError(f"qwen: attention order {attention!r}")
        self.ctx, self.cfg, self.max_batch = ctx, cfg, max_batch
        self.graph = None
        self.slot_graphs = {}  # captured lock-step slot steps, by conversation count
        self.set_attention(attention)
        vp, call = capi.vp, capi.call
        qd, kvd = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        self.qd, self.kvd = qd, kvd

        def dev(a, dtype=torch.float32):
            return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).cuda()

        self.blocks = []
        for b in weights["blocks"]:
            self.blocks.append({
                "qkv": capi.Weight(ctx, np.concatenate([b["q"], b["k"], b["v"]]), capi.Q4_0, qd + 2 * kvd, cfg.dim),
                "o": capi.Weight(ctx, b["o"], capi.Q4_0, cfg.dim, qd),
                "gu": capi.Weight(ctx, interleave_rows(b["gate"], b["up"], cfg.ffn, cfg.dim), capi.Q4_0,
                                  2 * cfg.ffn, cfg.dim),
                "down": capi.Weight(ctx, b["down"], capi.Q4_0, cfg.dim, cfg.ffn),
                "attn_norm": dev(b["attn_norm"]), "ffn_norm": dev(b["ffn_norm"]),
                "q_norm": dev(b["q_norm"]), "k_norm": dev(b["k_norm"]),
            })
        # the tied embedding / head: Q6_K (config 3) or Q4_0 (a pure Q4_0 checkpoint)
        self.head_quant = weights.get("token_embd_quant", capi.Q6_K)
        if self.head_quant not in (capi.Q6_K, capi.Q4_0):
            raise ValueError("qwen: the tied head must be Q6_K or Q4_0")
        self.embd = capi.Weight(ctx, weights["token_embd"], self.head_quant, cfg.vocab, cfg.dim)
        self.output_norm = dev(weights["output_norm"])
        # a row for every position of the cache (a multiple of 8), as the
        # kernels' contract has it
        cos, sin = rope_tables(cfg.head_dim, (cfg.max_context + 7) // 8 * 8, cfg.rope_base)
        self.rope_cos, self.rope_sin = dev(cos), dev(sin)
        # one conversation until set_slots says otherwise
        self._make_caches(1)

        M = max_batch
        self.xs = torch.empty((M, cfg.dim), dtype=torch.float32, device="cuda")
        self.xs2 = torch.empty((1, cfg.dim), dtype=torch.float32, device="cuda")  # the fused steps' other residual
        self.x8 = _Q8(M, cfg.dim)
        self.qkv = torch.empty((M, qd + 2 * kvd), dtype=torch.float32, device="cuda")
        self.qh = torch.empty((M, qd), dtype=torch.int16, device="cuda")
        self.set8 = _Q8(M, qd)
        self.attn = torch.empty((M, cfg.dim), dtype=torch.float32, device="cuda")
        self.gu = torch.empty((M, 2 * cfg.ffn), dtype=torch.float32, device="cuda")
        self.mid8 = _Q8(M, cfg.ffn)
        self.ffn = torch.empty((M, cfg.dim), dtype=torch.float32, device="cuda")
        self.hidden = torch.empty((M, cfg.dim), dtype=torch.float32, device="cuda")
        self.positions = torch.empty((M,), dtype=torch.int32, device="cuda")
        self.slot_ids = torch.zeros((M,), dtype=torch.int32, device="cuda")  # each token's conversation
        self.tokens = torch.empty((M,), dtype=torch.int32, device="cuda")
        self.k8 = torch.empty((M, cfg.dim), dtype=torch.int8, device="cuda")
        self.ks = torch.empty((M, cfg.dim // 256), dtype=torch.float32, device="cuda")
        self.bs = torch.empty((M, cfg.dim // 16), dtype=torch.int16, device="cuda")
        self.logit = torch.empty((M, cfg.vocab), dtype=torch.float32, device="cuda")
        self.next_id = torch.empty((M,), dtype=torch.int32, device="cuda")
        self.pos_dev = torch.zeros((1,), dtype=torch.int32, device="cuda")  # the graph's position counter
        self.history = torch.zeros((cfg.max_context + 1,), dtype=torch.int32, device="cuda")
        self.graph = None
        self.slot_graphs = {}
        n = capi.size_out("gx_qwen_attention_workspace_bytes", M, cfg.heads, cfg.max_context - 1)
        self.attn_ws = torch.empty((n + 255) // 256 * 256, dtype=torch.uint8, device="cuda")
        self._vp, self._call = vp, call

    def _make_caches(self, n):
        """n conversations of max_context // n positions each (SetSlots,
        qwen/slots.go:19-37).  Per layer, keys in 16-byte pieces
        [slot][kv_head][head_dim/8][context][8] and values transposed
        [slot][kv_head][head_dim][context]."""
        cfg = self.cfg
        self.nslots, self.slot = n, 0
        self.slot_context = cfg.max_context // n
        self.context = (self.slot_context + 7) // 8 * 8
        kshape = (n, cfg.kv_heads, cfg.head_dim // 8, self.context, 8)
        vshape = (n, cfg.kv_heads, cfg.head_dim, self.context)
        self.kc = self.vc = None
        self.kc = [torch.zeros(kshape, dtype=torch.int16, device="cuda") for _ in range(cfg.layers)]
        self.vc = [torch.zeros(vshape, dtype=torch.int16, device="cuda") for _ in range(cfg.layers)]

    def set_attention(self, attention):
        """Switch the decode steps' attention order ("parallel" or "golem");
        a captured step is dropped."""
        if attention not in ("parallel", "golem"):
            raise ValueError(f"qwen: attention order {attention!r}")
        sfx = "_parallel" if attention == "parallel" else ""
        self._rope_attention, self._attention = "gx_qwen_rope_attention" + sfx, "gx_qwen_attention" + sfx
        self.graph = None
        self.slot_graphs = {}

    def set_slots(self, n):
        """SetSlots (qwen/slots.go:19-37): n independent conversations, each
        holding max_context // n positions; replaces whatever was cached."""
        if n < 1:
            raise ValueError(f"qwen: {n} slots")
        if self.cfg.max_context // n < 1:
            raise ValueError(f"qwen: a context of {self.cfg.max_context} cut into {n} slots leaves no position each")
        self.graph = None  # a captured step addressed the caches being replaced
        self.slot_graphs = {}
        self._make_caches(n)

    def use_slot(self, i):
        """UseSlot (qwen/slots.go:62-78): forward() goes to conversation i."""
        if not 0 <= i < self.nslots:
            raise IndexError(f"qwen: slot {i} of {self.nslots}")
        self.slot = i

    def reset(self):
        """Forget the conversations (Model.Reset): the caches are cleared."""
        for k, v in zip(self.kc, self.vc):
            k.zero_()
            v.zero_()

    def _mm(self, w, act, M, y, ldy):
        vp = self._vp
        self._call("gx_matmul_q4_0", self.ctx.ptr, w.ptr, vp(act.q), vp(act.s), vp(act.qs), None, M, 0, w.rows,
                   None, vp(y), ldy)

    def forward(self, tokens, start_pos):
        """ForwardBatch: tokens is a device int32 tensor of M ids (or a host
        sequence, uploaded); returns the device hidden states [M][dim] after
        the final norm (a view of reused storage)."""
        cfg = self.cfg
        if not torch.is_tensor(tokens):
            tokens = torch.tensor(np.asarray(tokens, dtype=np.int32), device="cuda")
        M = int(tokens.shape[0])
        if M > self.max_batch or start_pos + M > self.slot_context:
            raise ValueError(f"qwen: {M} positions from {start_pos} exceed the batch {self.max_batch} "
                             f"or the context {self.slot_context}")
        self.tokens[:M].copy_(tokens)
        torch.arange(start_pos, start_pos + M, dtype=torch.int32, out=self.positions[:M])
        if self.nslots > 1:
            self.slot_ids[:M].fill_(self.slot)
        self._blocks(M, start_pos + M - 1, own_slot=True)
        return self.hidden[:M]

    def forward_slots(self, tokens, slots, positions):
        """ForwardSlots (qwen/place.go:33-41): token i at position
        positions[i] of conversation slots[i], all in one pass over the
        weights; each token's arithmetic is what it would be alone.  Returns
        the device hidden states [M][dim] after the final norm."""
        M = len(tokens)
        if not (len(slots) == len(positions) == M) or M > self.max_batch or M == 0:
            raise ValueError(f"qwen: {M} tokens, {len(slots)} slots, {len(positions)} positions "
                             f"(batch {self.max_batch})")
        for sl, pos in zip(slots, positions):
            if not 0 <= sl < self.nslots:
                raise IndexError(f"qwen: slot {sl} of {self.nslots}")
            if not 0 <= pos < self.slot_context:
                raise ValueError(f"qwen: position {pos} is past a slot's {self.slot_context}")
        self.tokens[:M].copy_(torch.tensor(np.asarray(tokens, dtype=np.int32)))
        self.positions[:M].copy_(torch.tensor(np.asarray(positions, dtype=np.int32)))
        self.slot_ids[:M].copy_(torch.tensor(np.asarray(slots, dtype=np.int32)))
        self._blocks(M, int(max(positions)))
        return self.hidden[:M]

    def residual(self, tokens, start_pos, blocks):
        """The residual stream of M >= 2 consecutive tokens after the first
        `blocks` blocks (0: the embedding rows), as ForwardBatch computes it
        before the final norm: a host [M][dim] float32 copy.  For checking a
        deep model block by block."""
        M = len(tokens)
        if M < 2 or M > self.max_batch or start_pos + M > self.slot_context:
            raise ValueError(f"qwen: {M} positions from {start_pos} for a block-by-block residual")
        self.tokens[:M].copy_(torch.tensor(np.asarray(tokens, dtype=np.int32)))
        torch.arange(start_pos, start_pos + M, dtype=torch.int32, out=self.positions[:M])
        if self.nslots > 1:
            self.slot_ids[:M].fill_(self.slot)
        self._blocks(M, start_pos + M - 1, blocks, own_slot=True)
        self.ctx.sync()
        if blocks == 0:
            return self.xs[:M].cpu().numpy().copy()
        return (self.xs[:M] + self.ffn[:M]).cpu().numpy()  # the last block's residual add

    def _blocks(self, M, max_pos, blocks=None, one_per_slot=False, own_slot=False):
        """The embedding rows, every block and the final norm for the M tokens
        and positions already in self.tokens / self.positions (with `blocks`:
        only the first that many blocks, and no final norm).  one_per_slot:
        the M tokens belong to M different conversations (a lock-step step),
        so the head norms, RoPE, cache stores and attention run as one
        kernel.  own_slot: the M tokens are the current conversation's
        (forward), whose caches the attention then reads as a lone
        conversation's."""
        cfg, vp, call, ctx = self.cfg, self._vp, self._call, self.ctx.ptr
        call("gx_weight_rows", ctx, self.embd.ptr, 0, vp(self.tokens), M, vp(self.xs))
        if M == 1:
            return self._blocks_one(max_pos)
        qd, kvd = self.qd, self.kvd
        sl = vp(self.slot_ids) if self.nslots > 1 else None
        for i, b in enumerate(self.blocks):
            if blocks is not None and i >= blocks:
                return
            add = None if i == 0 else vp(self.ffn)
            call("gx_norm_quant", ctx, vp(self.xs), cfg.dim, add, cfg.dim, vp(b["attn_norm"]), M, cfg.dim,
                 np.float32(cfg.eps), None, 0, vp(self.x8.q), vp(self.x8.s), vp(self.x8.qs))
            if one_per_slot and max_pos < FUSED_ATTENTION_MAX:
                self._mm(b["qkv"], self.x8, M, self.qkv, qd + 2 * kvd)
                call("gx_qwen_rope_attention_slots", ctx, vp(self.qkv), qd + 2 * kvd, M, cfg.heads, cfg.kv_heads,
                     cfg.head_dim, max_pos, vp(self.positions), vp(b["q_norm"]), vp(b["k_norm"]),
                     vp(self.rope_cos), vp(self.rope_sin), np.float32(cfg.eps), vp(self.kc[i]), vp(self.vc[i]),
                     self.context, vp(self.set8.q), vp(self.set8.s), vp(self.set8.qs), sl, self.nslots,
                     1 if self._attention.endswith("_parallel") else 0)
            else:
                # the product and the heads' norms, RoPE and stores (one
                # kernel for a batch: the product's epilogue)
                call("gx_qwen_qkv_rope", ctx, b["qkv"].ptr, vp(self.x8.q), vp(self.x8.s), vp(self.x8.qs), M,
                     cfg.heads, cfg.kv_heads, cfg.head_dim, vp(self.positions), vp(b["q_norm"]), vp(b["k_norm"]),
                     vp(self.rope_cos), vp(self.rope_sin), np.float32(cfg.eps), vp(self.qh), vp(self.kc[i]),
                     vp(self.vc[i]), self.context, sl, self.nslots, vp(self.qkv))
                if sl is None or not own_slot:
                    kca, vca, sla = self.kc[i], self.vc[i], sl
                else:
                    # a prompt of the current conversation reads that slot's
                    # caches as a lone conversation's: the same kernels, and
                    # so the same values, as the model without slots
                    kca, vca, sla = self.kc[i][self.slot], self.vc[i][self.slot], None
                call(self._attention, ctx, vp(self.qh), M, cfg.heads, cfg.kv_heads, cfg.head_dim,
                     max_pos, vp(self.positions), vp(kca), vp(vca), self.context,
                     vp(self.set8.q), vp(self.set8.s), vp(self.set8.qs), vp(self.attn_ws), self.attn_ws.numel(),
                     sla, self.nslots if sla is not None else 0)
            self._mm(b["o"], self.set8, M, self.attn, cfg.dim)
            call("gx_norm_quant", ctx, vp(self.xs), cfg.dim, vp(self.attn), cfg.dim, vp(b["ffn_norm"]), M, cfg.dim,
                 np.float32(cfg.eps), None, 0, vp(self.x8.q), vp(self.x8.s), vp(self.x8.qs))
            # the product and SwiGLU + Q8_0 in one kernel (its epilogue)
            call("gx_matmul_swiglu_q4_0", ctx, b["gu"].ptr, vp(self.x8.q), vp(self.x8.s), vp(self.x8.qs), M,
                 vp(self.mid8.q), vp(self.mid8.s), vp(self.mid8.qs))
            self._mm(b["down"], self.mid8, M, self.ffn, cfg.dim)
        if blocks is not None:
            return
        call("gx_norm_quant", ctx, vp(self.xs), cfg.dim, vp(self.ffn), cfg.dim, vp(self.output_norm), M, cfg.dim,
             np.float32(cfg.eps), vp(self.hidden), cfg.dim, None, None, None)

    def _blocks_one(self, max_pos):
        """The blocks for one position, with each pre-norm fused into the
        product after it, and the SwiGLU with its Q8_0 into the Gate/Up
        product (the same values bit for bit).  The residual moves between two buffers, since a
        fused product's workgroups all read it while one writes x + add."""
        cfg, vp, call, ctx = self.cfg, self._vp, self._call, self.ctx.ptr
        qd, kvd = self.qd, self.kvd
        sl = vp(self.slot_ids) if self.nslots > 1 else None
        eps = np.float32(cfg.eps)
        cur, other = self.xs, self.xs2
        for i, b in enumerate(self.blocks):
            if i == 0:
                call("gx_norm_matmul_q4_0", ctx, b["qkv"].ptr, vp(cur), None, vp(b["attn_norm"]), eps, None, 0,
                     b["qkv"].rows, vp(self.qkv))
            else:
                call("gx_norm_matmul_q4_0", ctx, b["qkv"].ptr, vp(cur), vp(self.ffn), vp(b["attn_norm"]), eps,
                     vp(other), 0, b["qkv"].rows, vp(self.qkv))
                cur, other = other, cur
            if max_pos < FUSED_ATTENTION_MAX:  # head norms + RoPE + cache store + attention, one kernel
                call(self._rope_attention, ctx, vp(self.qkv), qd + 2 * kvd, cfg.heads, cfg.kv_heads,
                     cfg.head_dim, max_pos, vp(self.positions), vp(b["q_norm"]), vp(b["k_norm"]),
                     vp(self.rope_cos), vp(self.rope_sin), eps, vp(self.kc[i]), vp(self.vc[i]), self.context,
                     vp(self.set8.q), vp(self.set8.s), vp(self.set8.qs), sl, self.nslots)
            else:
                call("gx_qwen_qk_rope", ctx, vp(self.qkv), qd + 2 * kvd, 1, cfg.heads, cfg.kv_heads,
                     cfg.head_dim, vp(self.positions), vp(b["q_norm"]), vp(b["k_norm"]), vp(self.rope_cos),
                     vp(self.rope_sin), eps, vp(self.qh), vp(self.kc[i]), vp(self.vc[i]), self.context, sl,
                     self.nslots)
                call(self._attention, ctx, vp(self.qh), 1, cfg.heads, cfg.kv_heads, cfg.head_dim,
                     max_pos, vp(self.positions), vp(self.kc[i]), vp(self.vc[i]), self.context,
                     vp(self.set8.q), vp(self.set8.s), vp(self.set8.qs), vp(self.attn_ws), self.attn_ws.numel(),
                     sl, self.nslots)
            self._mm(b["o"], self.set8, 1, self.attn, cfg.dim)
            call("gx_norm_swiglu_q4_0", ctx, b["gu"].ptr, vp(cur), vp(self.attn), vp(b["ffn_norm"]), eps,
                 vp(other), vp(self.mid8.q), vp(self.mid8.s), vp(self.mid8.qs))
            cur, other = other, cur
            self._mm(b["down"], self.mid8, 1, self.ffn, cfg.dim)
        call("gx_norm_quant", ctx, vp(cur), cfg.dim, vp(self.ffn), cfg.dim, vp(self.output_norm), 1, cfg.dim,
             eps, vp(self.hidden), cfg.dim, None, None, None)

    def _decode_step(self):
        """One greedy step read entirely from the device: token self.tokens[0]
        at position self.pos_dev.  Leaves the next token in self.tokens[0] and
        in self.history[position + 1], and advances the position."""
        self._blocks(1, self.slot_context - 1)
        self.logits(0)
        # the argmax, straight into the next step's token, and the history
        # entry, counter and position of the next step, in one launch pair
        self._call("gx_argmax_step", self.ctx.ptr, self._vp(self.logit), self.cfg.vocab, self._vp(self.tokens),
                   self._vp(self.history), self.history.numel(), self._vp(self.pos_dev), self._vp(self.positions))

    def capture_decode(self):
        """Records _decode_step into a HIP graph (once).  The library's stream
        is the capture stream while recording."""
        if self.graph is not None:
            return
        if self.nslots > 1:
            raise ValueError("qwen: the captured decode step serves one conversation")
        torch.cuda.synchronize()
        stream = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        self._call("gx_set_stream", self.ctx.ptr, ctypes.c_void_p(stream.cuda_stream))
        try:
            with torch.cuda.graph(graph, stream=stream):
                self._decode_step()
        finally:
            self._call("gx_set_stream", self.ctx.ptr, None)
        torch.cuda.synchronize()
        self.graph = graph

    def logits(self, row):
        """Logits of hidden state `row` (of the last forward): the tied head
        (qwen/model.go:181-194), Q6_K over the Q8_K form or Q4_0 over the Q8_0
        form; the device logits [vocab] (reused storage)."""
        cfg, vp, call, ctx = self.cfg, self._vp, self._call, self.ctx.ptr
        h = self.hidden[row:row + 1]
        if self.head_quant == capi.Q4_0:
            a = self.x8  # free once the blocks are done
            call("gx_quantize_q8_0", ctx, vp(h), cfg.dim, 1, cfg.dim, vp(a.q), vp(a.s), vp(a.qs), None, None)
            call("gx_matmul_q4_0", ctx, self.embd.ptr, vp(a.q), vp(a.s), vp(a.qs), None, 1, 0, cfg.vocab, None,
                 vp(self.logit), cfg.vocab)
            return self.logit[0]
        call("gx_quantize_q8_k", ctx, vp(h), cfg.dim, 1, cfg.dim, vp(self.k8), vp(self.ks), vp(self.bs))
        call("gx_matmul_q6_k", ctx, self.embd.ptr, vp(self.k8), vp(self.ks), vp(self.bs), 1, 0, cfg.vocab, None,
             vp(self.logit), cfg.vocab)
        return self.logit[0]

    def start_slots(self, tokens, positions):
        """Seeds lock-step decoding of conversations 0 .. n-1: token i (a
        host id, or a device int32 tensor of n ids) at position positions[i]
        of slot i."""
        n = len(positions)
        if not 0 < n <= min(self.nslots, self.max_batch):
            raise ValueError(f"qwen: {n} conversations for {self.nslots} slots")
        if max(positions) >= self.slot_context:
            raise ValueError(f"qwen: position {max(positions)} is past a slot's {self.slot_context}")
        t = tokens if torch.is_tensor(tokens) else torch.tensor(np.asarray(tokens, dtype=np.int32))
        self.tokens[:n].copy_(t)
        self.positions[:n].copy_(torch.tensor(np.asarray(positions, dtype=np.int32)))
        if self.nslots > 1:
            self.slot_ids[:n].copy_(torch.arange(n, dtype=torch.int32))
        self._slot_pos = list(positions)

    def slots_step(self, n, graph=False):
        """One lock-step decode step of conversations 0 .. n-1 from the
        tokens and positions on the device (the server's batch of slots,
        cmd/golem-server/runner.go:233-297): one pass over the weights and one
        head read for all n; the next ids replace the tokens (and stay in
        next_id[:n]) and every position advances.  graph: the step as a
        replay of its captured form (capture_slots), the same values bit for
        bit."""
        top = max(self._slot_pos)
        if top >= self.slot_context:
            raise ValueError(f"qwen: position {top} is past a slot's {self.slot_context}")
        if graph:
            self.capture_slots(n)
            self.slot_graphs[n].replay()
        else:
            self._slots_device_step(n, top)
        self._slot_pos = [p + 1 for p in self._slot_pos]
        return self.next_id[:n]

    def _slots_device_step(self, n, max_pos):
        self._blocks(n, max_pos, one_per_slot=self.nslots > 1)
        self.logits_batch(range(n))
        # the picks, each row's next token and its position advanced, in one launch
        self._call("gx_argmax_slots_step", self.ctx.ptr, self._vp(self.logit), self.cfg.vocab, n, self.cfg.vocab,
                   self._vp(self.next_id), self._vp(self.tokens), self._vp(self.positions))

    def capture_slots(self, n):
        """Records the device work of slots_step(n) into a HIP graph (once per
        n): the attention is launched for a slot's whole context and each
        token stops at its own prefix, read from the device, so one recording
        serves every step."""
        if self.slot_graphs.get(n) is not None:
            return
        if not 0 < n <= min(self.nslots, self.max_batch):
            raise ValueError(f"qwen: {n} conversations for {self.nslots} slots")
        torch.cuda.synchronize()
        stream = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        self._call("gx_set_stream", self.ctx.ptr, ctypes.c_void_p(stream.cuda_stream))
        try:
            with torch.cuda.graph(graph, stream=stream):
                self._slots_device_step(n, self.slot_context - 1)
        finally:
            self._call("gx_set_stream", self.ctx.ptr, None)
        torch.cuda.synchronize()
        self.slot_graphs[n] = graph

    def logits_batch(self, rows):
        """LogitsBatch (qwen/model.go:200-214): the logits of several hidden
        states of the last forward in one read of the head; device [n][vocab]
        (reused storage), each row what logits() gives it alone."""
        cfg, vp, call, ctx = self.cfg, self._vp, self._call, self.ctx.ptr
        rows = list(rows)
        n = len(rows)
        if not 0 < n <= self.max_batch:
            raise ValueError(f"qwen: {n} states for a batch of {self.max_batch}")
        if rows == list(range(rows[0], rows[0] + n)):
            h = self.hidden[rows[0]:rows[0] + n]
        else:
            h = self.attn[:n]  # free once the blocks are done
            h.copy_(self.hidden[rows])
        if self.head_quant == capi.Q4_0:
            a = self.x8
            call("gx_quantize_q8_0", ctx, vp(h), cfg.dim, n, cfg.dim, vp(a.q), vp(a.s), vp(a.qs), None, None)
            call("gx_matmul_q4_0", ctx, self.embd.ptr, vp(a.q), vp(a.s), vp(a.qs), None, n, 0, cfg.vocab, None,
                 vp(self.logit), cfg.vocab)
        else:
            call("gx_quantize_q8_k", ctx, vp(h), cfg.dim, n, cfg.dim, vp(self.k8), vp(self.ks), vp(self.bs))
            call("gx_matmul_q6_k", ctx, self.embd.ptr, vp(self.k8), vp(self.ks), vp(self.bs), n, 0, cfg.vocab, None,
                 vp(self.logit), cfg.vocab)
        return self.logit[:n]

    def next_tokens(self, rows):
        """The greedy ids after several hidden states (one head read), left
        on the device: next_id[:n]."""
        n = len(list(rows))
        self.logits_batch(rows)
        self._call("gx_argmax", self.ctx.ptr, self._vp(self.logit), self.cfg.vocab, n, self.cfg.vocab,
                   self._vp(self.next_id))
        return self.next_id[:n]

    def next_token(self, row):
        """The greedy id after hidden state `row`, left on the device."""
        self.logits(row)
        self._call("gx_argmax", self.ctx.ptr, self._vp(self.logit), self.cfg.vocab, 1, self.cfg.vocab,
                   self._vp(self.next_id))
        return self.next_id[:1]

    def greedy(self, prompt, steps, graph=False):
        """The prompt in one batch, then `steps` greedy tokens, each fed back
        from the device (graph: the decode steps as replays of the captured
        step).  Returns the ids (host list)."""
        if len(prompt) + steps - 1 > self.cfg.max_context:
            raise ValueError(f"qwen: {steps} tokens after {len(prompt)} exceed the context {self.cfg.max_context}")
        self.reset()
        self.forward(prompt, 0)
        tok = self.next_token(len(prompt) - 1)
        if graph:
            self.capture_decode()
            self.start_decode(tok, len(prompt))
            for _ in range(steps - 1):
                self.graph.replay()
            return self.decoded(len(prompt), steps)
        ids = []
        pos = len(prompt)
        for s in range(steps):
            ids.append(tok.clone())
            if s + 1 < steps:
                self.forward(tok, pos)
                tok = self.next_token(0)
                pos += 1
        return [int(t.item()) for t in ids]

    def start_decode(self, tok, pos):
        """Seeds the captured step: token `tok` (device) at position `pos`,
        also recorded as the history's entry `pos`."""
        if pos >= self.cfg.max_context:
            raise ValueError(f"qwen: position {pos} is past the context {self.cfg.max_context}")
        self.tokens[:1].copy_(tok)
        self.history[pos:pos + 1].copy_(tok)
        self.pos_dev.fill_(pos)
        self.positions[:1].fill_(pos)

    def decoded(self, pos, steps):
        """The ids of `steps` greedy tokens from position `pos`: the seed
        and those the replays left in the history."""
        return [int(t) for t in self.history[pos:pos + steps].cpu().tolist()]

    def free(self):
        for b in self.blocks:
            for k in ("qkv", "o", "gu", "down"):
                b[k].free()
        self.embd.free()
