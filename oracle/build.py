"""Builds the oracle's C restatement into oracle/liboracle.so.

gcc -O2 -ffp-contract=off with no -march: SSE scalar float32 arithmetic, one
rounding per operation, no fused multiply-add -- the float semantics of
golem's Go code compiled for amd64 at GOAMD64=v1.

golem itself cannot be built here: its path is Go and Go assembly, and no Go
toolchain exists in this image, so there is no oracle/_ref build.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
CPU_LIB = os.path.join(HERE, "libcpu_avx2.so")


def _gcc(src, out, flags, verbose):
    tmp = out + ".tmp"
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", "-Wall", *flags,
           "-o", tmp, src, "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build of {os.path.basename(src)} failed:\n{r.stderr}")
    if r.stderr.strip() and verbose:
        print(r.stderr)
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")


def build(verbose=True):
    """liboracle.so (generic restatement) and libcpu_avx2.so (golem's AVX2
    kernels and worker pool, the CPU baseline; -mavx2 -mfma -mf16c, loaded
    only on a host that has them)."""
    _gcc(os.path.join(HERE, "oracle.c"), LIB, [], verbose)
    _gcc(os.path.join(HERE, "cpu_avx2.c"), CPU_LIB, ["-mavx2", "-mfma", "-mf16c", "-pthread"], verbose)
    return LIB


if __name__ == "__main__":
    build()
