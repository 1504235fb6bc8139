"""Build libmxq_hip.so (gfx950) from the .hip sources next to this file.

    python build.py            compile every *.hip to an object (in parallel) and link the shared library
                               into ../mxq/libmxq_hip.so

Device code is built with -ffp-contract=off (the datapath's multiply and add must round separately),
float32 denormals preserved, no fast-math, and packed-fp32 instructions disabled.
"""
import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.normpath(os.path.join(HERE, "..", "mxq"))
INCLUDE = os.path.normpath(os.path.join(HERE, "..", "..", "include"))
OBJDIR = os.path.join(HERE, "_build")
LIB = os.path.join(PKG, "libmxq_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("MXQ_OFFLOAD_ARCH", "gfx950")

FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-mcode-object-version=5",
         "-ffp-contract=off", "-fno-fast-math", "-fno-gpu-flush-denormals-to-zero",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-command-line-argument", "-I", INCLUDE, "-I", HERE]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build(jobs: int = 8, verbose: bool = False) -> str:
    """Compile and link; returns the library path.  Always rebuilds (the build check runs it every round)."""
    os.makedirs(OBJDIR, exist_ok=True)
    # regenerate the log2 threshold table so the committed copy can never drift from its generator
    _run([sys.executable, os.path.join(HERE, "gen_log2_edges.py")])
    srcs = sorted(glob.glob(os.path.join(HERE, "*.hip")))
    objs = [os.path.join(OBJDIR, os.path.basename(s)[:-4] + ".o") for s in srcs]

    def one(pair):
        src, obj = pair
        cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)
        return obj

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(one, zip(srcs, objs)))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
