"""Seeded synthetic inputs for the configurations of the benchmark.

The same bytes feed the GPU path, the oracle and the CPU baseline, so the
choice of generator does not affect parity; numpy's PCG64 is deterministic
across machines.  Distributions follow the benchmark's configs:

  Q4_0 weights: per block d = fp16(|N(0,1)| * 0.02), 32 nibbles U{0..15}
                stored +8 (byte j: low nibble weight j, high weight j+16;
                golem nn/dot_q4_0.go:3-13).
  Q6_K weights: ql/qh bytes uniform (6-bit values U{0..63}), 16 int8
                sub-scales U{-64..63}, d = fp16(|N(0,1)| * 0.002)
                (layout nn/dequant_q6_k.go:3-15).
  Activations:  float32 N(0,1).
"""
import numpy as np

Q4_0_BLOCK_BYTES = 18
Q6_K_BLOCK_BYTES = 210


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def q4_0_weights(g, rows, cols, scale=0.02, symmetric=False):
    """GGUF Q4_0 bytes for a rows x cols matrix (uint8 array).  symmetric draws
    nibbles from 1..15 (weights -7..7, mean zero) instead of 0..15."""
    assert cols % 32 == 0
    blocks = rows * (cols // 32)
    out = np.empty((blocks, Q4_0_BLOCK_BYTES), dtype=np.uint8)
    d = (np.abs(g.standard_normal(blocks)) * scale).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(blocks, 2)
    if symmetric:
        lo = g.integers(1, 16, size=(blocks, 16), dtype=np.uint8)
        hi = g.integers(1, 16, size=(blocks, 16), dtype=np.uint8)
        out[:, 2:] = lo | (hi << 4)
    else:
        out[:, 2:] = g.integers(0, 256, size=(blocks, 16), dtype=np.uint8)
    return out.reshape(-1)


def q6_k_weights(g, rows, cols, scale=0.002):
    """GGUF Q6_K bytes for a rows x cols matrix (uint8 array)."""
    assert cols % 256 == 0
    sbs = rows * (cols // 256)
    out = np.empty((sbs, Q6_K_BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:192] = g.integers(0, 256, size=(sbs, 192), dtype=np.uint8)
    out[:, 192:208] = g.integers(-64, 64, size=(sbs, 16), dtype=np.int8).view(np.uint8)
    d = (np.abs(g.standard_normal(sbs)) * scale).astype(np.float16)
    out[:, 208:210] = d.view(np.uint8).reshape(sbs, 2)
    return out.reshape(-1)


def activations(g, m, k):
    return g.standard_normal((m, k)).astype(np.float32)


class QwenConfig:
    """A Qwen3 dense decoder's geometry (golem's qwen.Config / BlockConfig,
    qwen/config.go): every block alike, full-width NeoX RoPE."""

    def __init__(self, dim, ffn, layers, heads, kv_heads, head_dim, vocab, max_context, rope_base=1e6, eps=1e-6):
        self.dim, self.ffn, self.layers = dim, ffn, layers
        self.heads, self.kv_heads, self.head_dim = heads, kv_heads, head_dim
        self.vocab, self.max_context = vocab, max_context
        self.rope_base, self.eps = rope_base, eps

    def __repr__(self):
        return (f"QwenConfig(dim={self.dim}, ffn={self.ffn}, layers={self.layers}, heads={self.heads}/"
                f"{self.kv_heads}x{self.head_dim}, vocab={self.vocab}, ctx={self.max_context})")


def qwen3_4b(max_context=640):
    """Config 3: Qwen3-4B's shape (36 blocks, 2560 wide, FFN 9728, 32 query
    and 8 key-value heads of 128, vocab 151936, RoPE base 1e6, eps 1e-6)."""
    return QwenConfig(2560, 9728, 36, 32, 8, 128, 151936, max_context)


def qwen_weights(cfg, seed, symmetric=False):
    """Random weights of that shape, drawn as config 3 specifies: every linear
    matrix Q4_0 as in config 0, the tied embedding / output head Q6_K as in
    config 1, norms 1 + N(0, 0.02).  A dict of numpy arrays: matrices as GGUF
    bytes (row-major), norms as float32.  symmetric: zero-mean Q4_0 nibbles
    (config 3's nibbles have mean -0.5 after centring, which drives every
    position towards the same token; tests use both)."""
    g = rng(seed)

    def norm(n):
        return (1.0 + 0.02 * g.standard_normal(n)).astype(np.float32)

    qd, kvd = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    blocks = []
    for _ in range(cfg.layers):
        blocks.append({
            "attn_norm": norm(cfg.dim),
            "q": q4_0_weights(g, qd, cfg.dim, symmetric=symmetric), "q_norm": norm(cfg.head_dim),
            "k": q4_0_weights(g, kvd, cfg.dim, symmetric=symmetric), "k_norm": norm(cfg.head_dim),
            "v": q4_0_weights(g, kvd, cfg.dim, symmetric=symmetric),
            "o": q4_0_weights(g, cfg.dim, qd, symmetric=symmetric),
            "ffn_norm": norm(cfg.dim),
            "gate": q4_0_weights(g, cfg.ffn, cfg.dim, symmetric=symmetric),
            "up": q4_0_weights(g, cfg.ffn, cfg.dim, symmetric=symmetric),
            "down": q4_0_weights(g, cfg.dim, cfg.ffn, symmetric=symmetric),
        })
    return {"blocks": blocks, "output_norm": norm(cfg.dim),
            "token_embd": q6_k_weights(g, cfg.vocab, cfg.dim)}
