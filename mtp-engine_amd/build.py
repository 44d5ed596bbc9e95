"""Build the gfx950 C-ABI library libmtp_hip.so in-tree with hipcc.

Usage: python mtp-engine_amd/build.py [--verbose] [--jobs N]

Every csrc/*.hip translation unit is compiled to an object in parallel
(objects under mtp-engine_amd/_build/), then linked into
mtp_hip/libmtp_hip.so next to the Python package, so it travels with the
source tree; nothing is installed.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJDIR = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "mtp_hip", "libmtp_hip.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    # Packed FP32 instructions stay off: hipcc may only emit scalar/vector
    # fp32 arithmetic in these kernels.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(cand):
        return cand
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: set ROCM_PATH")
    return found


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd[-3:])}")
    return res


def build(verbose: bool = False, jobs: int = 0) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = [os.path.join(OBJDIR, os.path.basename(s)[:-4] + ".o") for s in srcs]
    t0 = time.time()
    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [hipcc(), *HIPCC_FLAGS, "-c", "-o", o, s], verbose)
                for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = OUT + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} in {time.time() - t0:.1f}s", flush=True)
    return OUT


if __name__ == "__main__":
    j = 0
    if "--jobs" in sys.argv:
        j = int(sys.argv[sys.argv.index("--jobs") + 1])
    build(verbose="--verbose" in sys.argv or "-v" in sys.argv, jobs=j)
