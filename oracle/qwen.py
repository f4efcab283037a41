"""golem's Qwen3 dense decoder (qwen/), restated over the oracle's C
primitives, for checking the device decoder.

TEST INFRASTRUCTURE ONLY: the tests are its only importers.

Every float operation happens either in oracle.c (norms, RoPE, DotF32,
softmax, Axpy, SwiGLU, the Q4_0 / Q6_K products, the quantisers) or as one
numpy float32 operation that rounds exactly as Go's float32 does (the
residual adds).  The structure follows golem:

  ForwardBatch / ForwardMixed  qwen/model.go:127-175
  Block                        qwen/block.go:32-102
  Attention                    qwen/attention.go:34-127
  LayerCache.Store             qwen/cache.go:52-60 (entries rounded through fp16)
  Embed                        qwen/model.go:107-109 (TokenEmbd.Row: DequantizeQ6_K, or
                               dequantizeQ4_0Row for a Q4_0 table)
  Logits                       qwen/model.go:181-194 (QuantizeK + MatVecQ6_K, or the
                               Q8_0 form + Matrix.rows for a Q4_0 head)

Dense matrices are repacked as golem repacks them at load (Matrix.Repack,
nn/matrix.go:40-46) and multiplied through Matrix.rows' packed path.
"""
import math

import numpy as np

from . import (Batch, Q4_0, Q6_K, _p, dequantize_q4_0_row, dequantize_q6_k, load, mat_vec_q6_k_rows,
               matrix_rows, pack_q4_0, rms_norm_plain)


class QwenOracle:
    """repacked=False multiplies the dense matrices in golem's row layout
    (Matrix.rows without Repack: matVecQ4_0Rows, dotQ4_0Go) instead of the
    8-row packed form golem's loader builds -- golem's other generic form of
    the same product, equal to it up to float rounding."""

    def __init__(self, cfg, weights, repacked=True):
        self.cfg, self.w = cfg, weights
        qd, kvd = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
        self.shapes = {"q": (qd, cfg.dim), "k": (kvd, cfg.dim), "v": (kvd, cfg.dim), "o": (cfg.dim, qd),
                       "gate": (cfg.ffn, cfg.dim), "up": (cfg.ffn, cfg.dim), "down": (cfg.dim, cfg.ffn)}
        self.packed = [{n: pack_q4_0(b[n], *self.shapes[n]) if repacked else None for n in self.shapes}
                       for b in weights["blocks"]]
        self.K = [np.zeros((cfg.max_context, cfg.kv_heads, cfg.head_dim), np.float32) for _ in range(cfg.layers)]
        self.V = [np.zeros_like(k) for k in self.K]
        # the tied embedding / head: Q6_K (config 3) or Q4_0 (a pure Q4_0 file)
        self.head_quant = weights.get("token_embd_quant", Q6_K)
        self.row_bytes = cfg.dim // 256 * 210 if self.head_quant == Q6_K else cfg.dim // 32 * 18

    def reset(self):
        for k, v in zip(self.K, self.V):
            k[:] = 0
            v[:] = 0

    def _mat(self, layer, name, batch):
        rows, cols = self.shapes[name]
        return matrix_rows(Q4_0, self.w["blocks"][layer][name], rows, cols, batch, packed=self.packed[layer][name])

    @staticmethod
    def _round_half(x):
        out = np.array(x, dtype=np.float32).reshape(-1)
        load().orc_round_half_n(_p(out), len(out))
        return out.reshape(np.shape(x))

    def embed(self, token):
        row = self.w["token_embd"][token * self.row_bytes:(token + 1) * self.row_bytes]
        if self.head_quant == Q4_0:
            return dequantize_q4_0_row(row, self.cfg.dim)
        return dequantize_q6_k(row, self.cfg.dim)

    def forward(self, tokens, start_pos):
        """ForwardBatch: hidden states after the final norm, one per token."""
        cfg = self.cfg
        xs = np.stack([self.embed(t) for t in tokens]).astype(np.float32)
        pos = [start_pos + i for i in range(len(tokens))]
        for layer in range(cfg.layers):
            self.block(layer, xs, pos)
        return np.stack([rms_norm_plain(x, self.w["output_norm"], cfg.eps) for x in xs])

    def norm(self, layer, xs, which):
        """A block's pre-norm (qwen/block.go:45-52, 59-68): RMSNormPlain of
        every position with the block's attn_norm or ffn_norm gain, and the
        Q8_0 form of the result."""
        gain = self.w["blocks"][layer][which]
        return Batch(np.stack([rms_norm_plain(x, gain, self.cfg.eps) for x in xs])).quantize()

    def swiglu(self, gate, up):
        """SwiGLURange (nn/swiglu.go:77-82) of every position: silu(gate) * up."""
        lib, mid = load(), np.array(gate, dtype=np.float32)
        for t in range(len(mid)):
            g, u = np.ascontiguousarray(mid[t]), np.ascontiguousarray(up[t], dtype=np.float32)
            lib.orc_swiglu_range(_p(g), _p(u), 0, self.cfg.ffn)
            mid[t] = g
        return mid

    def block(self, layer, xs, pos):
        normed = self.norm(layer, xs, "attn_norm")
        attn = self.attention(layer, normed, pos)
        xs += attn
        normed = self.norm(layer, xs, "ffn_norm")
        mid = self.swiglu(self._mat(layer, "gate", normed), self._mat(layer, "up", normed))
        ffn = self._mat(layer, "down", Batch(mid).quantize())
        xs += ffn

    def attention(self, layer, normed, pos):
        q, k, v = (self._mat(layer, n, normed) for n in ("q", "k", "v"))
        return self._mat(layer, "o", Batch(self.attend(layer, q, k, v, pos)).quantize())

    def attend(self, layer, q, k, v, pos, only=None):
        """Attention's head-by-head part and the attention proper
        (qwen/attention.go:57-124) from the Q, K and V projections of the
        batch: per-head norms, RoPE, fp16 query and cache entries, then every
        head's output (the floats the O projection's Q8_0 is made from).
        only: the batch rows whose outputs are wanted (every row's keys and
        values still go into the cache); the result then has one row each."""
        cfg, bw, lib = self.cfg, self.w["blocks"][layer], load()
        hd, batch = cfg.head_dim, len(q)
        rows = list(range(batch)) if only is None else [int(t) for t in only]
        wanted = set(rows)
        qh = np.zeros_like(q)
        cos = np.zeros(hd // 2, np.float32)
        sin = np.zeros(hd // 2, np.float32)
        for t in range(batch):
            lib.orc_rope_prepare(hd, pos[t], cfg.rope_base, _p(cos), _p(sin))
            for h in range(cfg.heads if t in wanted else 0):
                head = rms_norm_plain(q[t, h * hd:(h + 1) * hd], bw["q_norm"], cfg.eps)
                lib.orc_rope_apply(_p(head), hd, _p(cos), _p(sin))
                qh[t, h * hd:(h + 1) * hd] = self._round_half(head)
            for h in range(cfg.kv_heads):
                kh = rms_norm_plain(k[t, h * hd:(h + 1) * hd], bw["k_norm"], cfg.eps)
                lib.orc_rope_apply(_p(kh), hd, _p(cos), _p(sin))
                self.K[layer][pos[t], h] = self._round_half(kh)
                self.V[layer][pos[t], h] = self._round_half(v[t, h * hd:(h + 1) * hd])
        per_kv = cfg.heads // cfg.kv_heads
        scale = np.float32(1 / math.sqrt(float(hd)))
        out = np.zeros((len(rows), cfg.heads * hd), np.float32)
        scores = np.zeros(cfg.max_context, np.float32)
        Kl, Vl = self.K[layer], self.V[layer]
        for i, t in enumerate(rows):
            for h in range(cfg.heads):
                query = np.ascontiguousarray(qh[t, h * hd:(h + 1) * hd])
                dst = np.zeros(hd, np.float32)
                lib.orc_attend(_p(query), _p(Kl), _p(Vl), cfg.kv_heads, hd, h // per_kv, pos[t] + 1, scale,
                               _p(scores), _p(dst))
                out[i, h * hd:(h + 1) * hd] = dst
        return out

    def logits(self, hidden):
        """Logits for one hidden state: the tied head, Q6_K over the Q8_K form
        or Q4_0 over the Q8_0 form (the embedding is never repacked)."""
        if self.head_quant == Q4_0:
            b = Batch(np.asarray(hidden, np.float32)[None, :]).quantize()
            return matrix_rows(Q4_0, self.w["token_embd"], self.cfg.vocab, self.cfg.dim, b)[0]
        b = Batch(np.asarray(hidden, np.float32)[None, :]).quantize_k()
        return mat_vec_q6_k_rows(self.w["token_embd"], b, self.cfg.vocab)[0]

    def greedy(self, prompt, steps):
        """Prompt read in one batch, then `steps` greedy tokens (argmax, ties to
        the lower id, qwen/model_test.go:118-126).  Returns (ids, margins) with
        margins the top-1 minus top-2 logit of every step."""
        self.reset()
        hidden = self.forward(prompt, 0)[-1]
        ids, margins = [], []
        pos = len(prompt)
        for _ in range(steps):
            lg = self.logits(hidden)
            top = int(np.argmax(lg))
            srt = np.sort(lg)
            ids.append(top)
            margins.append(float(srt[-1] - srt[-2]))
            hidden = self.forward([top], pos)[0]
            pos += 1
        return ids, margins
