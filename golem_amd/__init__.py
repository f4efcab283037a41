"""golem_amd: golem's quantized linear-layer path (Q4_0 / Q6_K products, their
activation quantisers and the MoE expert products) as hand-written HIP for
MI355X (gfx950), behind the C ABI of include/golem_hip.h.

Modules:
  capi   ctypes binding of libgolem_hip.so (no CPU fallback)
  synth  seeded synthetic inputs of the benchmark configurations
  build  the in-tree hipcc build
"""
__all__ = ["capi", "synth", "build"]
