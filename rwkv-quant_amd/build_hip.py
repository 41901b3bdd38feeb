"""Build librwkvq_hip.so from csrc/*.hip for gfx950 with hipcc.

    python rwkv-quant_amd/build_hip.py

The shared library lands in rwkv_quant/backends/hip/ (in-tree), next to
its ctypes binding.
"""
import glob
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "rwkv_quant", "backends", "hip", "librwkvq_hip.so")
ARCH = os.environ.get("RWKVQ_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # keep the compiler from forming packed fp32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err)


def build(verbose=True, out=OUT, defines=()):
    """Compile every csrc/*.hip to an object (in parallel, one hipcc per
    file), then link them into one shared library next to `out`."""
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    defs = [f"-D{d}" for d in defines]
    tmp = out + ".tmp"
    with tempfile.TemporaryDirectory(prefix="rwkvq_build_") as objdir:
        objs = [os.path.join(objdir, os.path.basename(f) + ".o")
                for f in srcs]
        jobs = max(1, min(len(srcs), os.cpu_count() or 1, 16))
        with ThreadPoolExecutor(jobs) as pool:
            list(pool.map(lambda so: _run(["hipcc", *FLAGS, *defs, "-c",
                                           so[0], "-o", so[1]], verbose),
                          zip(srcs, objs)))
        _run(["hipcc", "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs,
              "-o", tmp], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    import argparse
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=OUT)
    ap.add_argument("-D", dest="defines", action="append", default=[])
    a = ap.parse_args()
    print(build(out=a.out, defines=a.defines))
    sys.exit(0)
