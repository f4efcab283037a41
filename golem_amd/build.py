"""Builds libgolem_hip.so in-tree for gfx950 with hipcc.

Every HIP source under golem_amd/csrc is compiled to an object and the
objects are linked into golem_amd/libgolem_hip.so.  The build always runs
(it is the "does it build" check); objects go to golem_amd/_build/.

Flags that matter for parity and safety:
  -ffp-contract=off   no silent a*b+c fusion: the kernels write fmaf where
                      they mean it, everything else rounds per operation as
                      golem's amd64 code does.
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no packed-fp32 VALU instructions in the device code.
  -mllvm -amdgpu-mfma-vgpr-form
                      MFMA results in ordinary VGPRs: the epilogue's fma reads
                      them directly instead of copying each out of an AGPR.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libgolem_hip.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    obj = os.path.join(OUT_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so;
    # that line is expected and dropped.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    return src, obj, r.returncode, err


def build(verbose=True):
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sources()
    objs = []
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        for src, obj, rc, err in ex.map(_compile, srcs):
            if err.strip() and verbose:
                print(err, file=sys.stderr)
            if rc != 0:
                raise RuntimeError(f"hipcc failed on {src}:\n{err}")
            objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
