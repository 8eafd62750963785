"""Builds libmingmoe.so (HIP, gfx950) next to this file with hipcc.

    python build_lib.py            # compile csrc/*.hip in parallel and link the shared library

Every HIP translation unit is compiled for gfx950 only, with packed fp32 instructions disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops), and linked into one shared library with a plain
C ABI (include/mingmoe.h); the Python modules load it with ctypes.
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc")
INC = os.path.join(ROOT, "include")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libmingmoe.so")
ARCH = "gfx950"

FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{INC}", f"-I{SRC}"]


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(cc, src, obj):
    cmd = [cc, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that line is noise
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{err}")
    return err


def build(verbose=False, jobs=None):
    """Compiles every csrc/*.hip for gfx950 and links libmingmoe.so; returns the library path."""
    cc = hipcc()
    os.makedirs(OBJ, exist_ok=True)
    srcs = sorted(f for f in os.listdir(SRC) if f.endswith(".hip"))
    objs = [os.path.join(OBJ, f[:-4] + ".o") for f in srcs]
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        futs = {ex.submit(_compile, cc, os.path.join(SRC, s), o): s for s, o in zip(srcs, objs)}
        for f in concurrent.futures.as_completed(futs):
            warn = f.result()
            if verbose and warn.strip():
                print(f"[{futs[f]}]\n{warn}", file=sys.stderr)
    tmp = LIB + ".tmp"
    r = subprocess.run([cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp], capture_output=True,
                       text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of libmingmoe.so failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
