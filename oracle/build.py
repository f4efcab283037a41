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


def build(verbose=True):
    src = os.path.join(HERE, "oracle.c")
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared",
           "-Wall", "-o", tmp, src, "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stderr}")
    if r.stderr.strip() and verbose:
        print(r.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
