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


def q4_0_weights(g, rows, cols, scale=0.02):
    """GGUF Q4_0 bytes for a rows x cols matrix (uint8 array)."""
    assert cols % 32 == 0
    blocks = rows * (cols // 32)
    out = np.empty((blocks, Q4_0_BLOCK_BYTES), dtype=np.uint8)
    d = (np.abs(g.standard_normal(blocks)) * scale).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(blocks, 2)
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
